"""Batched decode on the config-3 model: B sequences over one copy of the
weights stepping in lockstep (zh_engine_generate_batch), each with its own KV
cache pre-filled to 4096 positions (seeded N(0,1) fp16), greedy-decoding from
a one-token prompt, so every timed step is a decode step of all B sequences.

    python -m zinc_amd.batch_bench [--seqs 1 2 4] [--steps 64]

Prints one JSON line per B: aggregate tok/s (B x steps / wall time) and the
milliseconds per batched step. The projections and the LM head stream their
weights once per step for all B sequences (batched DMMV); attention reads
each sequence's own KV cache. The step is issued launch by launch (no graph
replay), so B = 1 here runs below the graph-replayed single-sequence bench.
"""
import argparse
import json
import sys
import time

import numpy as np

from . import hip
from .engine import DENSE_8B, InferenceEngine

PREFILL = 4096


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--seqs", type=int, nargs="+", default=[1, 2, 4])
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=4)
    a = ap.parse_args()
    ctx = hip.Context(0)
    cfg = dict(DENSE_8B)
    cfg["max_ctx"] = (PREFILL + 2 * (a.warmup + a.steps) + 16 + 15) // 16 * 16
    base = InferenceEngine(ctx, cfg)
    engines = [base]
    rng = np.random.default_rng(77)
    for B in a.seqs:
        while len(engines) < B:
            engines.append(base.share(ctx))
        es = engines[:B]
        for v, e in enumerate(es):
            e.prefill_kv_random(PREFILL, 7 + v)
        ctx.sync()
        prompts = rng.integers(0, cfg["vocab"], (B, 1))
        warm = InferenceEngine.generate_batch(es, prompts, a.warmup, start_pos=PREFILL)
        nxt = np.array([[w[-1]] for w in warm])
        pos = PREFILL + a.warmup
        ctx.sync()
        t0 = time.perf_counter()
        toks = InferenceEngine.generate_batch(es, nxt, a.steps, start_pos=pos)
        ctx.sync()
        wall = time.perf_counter() - t0
        out = {"workload": "config 3 model, batched greedy decode at KV context 4096+ (one weight stream, B sequences)",
               "seqs": B, "steps": a.steps, "agg_tok_s": round(B * a.steps / wall, 1),
               "ms_per_batched_step": round(wall * 1e3 / a.steps, 3),
               "distinct_tokens": [len(set(t)) for t in toks]}
        print(json.dumps(out), flush=True)
    for e in engines[1:]:
        e.deinit()
    base.deinit()
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
