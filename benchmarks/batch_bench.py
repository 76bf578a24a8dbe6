"""Batched decode on the config-3 model: B sequences over one copy of the
weights stepping in lockstep (zh_engine_generate_batch), each with its own KV
cache pre-filled to 4096 positions (seeded N(0,1) fp16), greedy-decoding from
a one-token prompt, so every timed step is a decode step of all B sequences.

    python -m benchmarks.batch_bench [--seqs 1 2 4] [--steps 64] [--streams S]

Prints one JSON line per B: aggregate tok/s (B x steps / wall time) and the
milliseconds per batched step. The projections and the LM head stream their
weights once per step for all B sequences (batched DMMV); attention reads
each sequence's own KV cache. The step is issued launch by launch (no graph
replay), so B = 1 here runs below the graph-replayed single-sequence bench.
With --streams S > 1, S batches of B sequences each run at once, each on its
own context (HIP stream) and host thread (aggregate over S x B sequences).
"""
import argparse
import json
import sys
import threading
import time

import numpy as np

from zinc_amd import hip
from zinc_amd.engine import DENSE_8B, InferenceEngine

PREFILL = 4096


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--seqs", type=int, nargs="+", default=[1, 2, 4])
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--streams", type=int, default=1)
    a = ap.parse_args()
    S = max(1, a.streams)
    ctxs = [hip.Context(0) for _ in range(S)]
    cfg = dict(DENSE_8B)
    cfg["max_ctx"] = (PREFILL + 2 * (a.warmup + a.steps) + 16 + 15) // 16 * 16
    base = InferenceEngine(ctxs[0], cfg)
    groups = [[base]] + [[] for _ in range(S - 1)]
    rng = np.random.default_rng(77)
    for B in a.seqs:
        for g in range(S):
            while len(groups[g]) < B:
                groups[g].append(base.share(ctxs[g]))
        sets = [grp[:B] for grp in groups]
        for g, es in enumerate(sets):
            for v, e in enumerate(es):
                e.prefill_kv_random(PREFILL, 7 + 16 * g + v)
        for c in ctxs:
            c.sync()
        prompts = [rng.integers(0, cfg["vocab"], (B, 1)) for _ in range(S)]
        nxt = []
        for g, es in enumerate(sets):
            warm = InferenceEngine.generate_batch(es, prompts[g], a.warmup, start_pos=PREFILL)
            nxt.append(np.array([[w[-1]] for w in warm]))
        pos = PREFILL + a.warmup
        for c in ctxs:
            c.sync()
        toks = [None] * S

        def run(g):
            toks[g] = InferenceEngine.generate_batch(sets[g], nxt[g], a.steps, start_pos=pos)
        th = [threading.Thread(target=run, args=(g,)) for g in range(S)]
        t0 = time.perf_counter()
        for t in th:
            t.start()
        for t in th:
            t.join()
        for c in ctxs:
            c.sync()
        wall = time.perf_counter() - t0
        out = {"workload": "config 3 model, batched greedy decode at KV context 4096+ (one weight stream, B sequences)",
               "seqs": B, "streams": S, "steps": a.steps, "agg_tok_s": round(S * B * a.steps / wall, 1),
               "ms_per_batched_step": round(wall * 1e3 / a.steps, 3),
               "distinct_tokens": [len(set(t)) for grp in toks for t in grp]}
        print(json.dumps(out), flush=True)
    for grp in groups:
        for e in grp:
            if e is not base:
                e.deinit()
    base.deinit()
    for c in ctxs:
        c.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
