"""Config 4 measurement: sparse-MoE decoder decode loop (48 layers, hidden 2048,
32 q / 4 kv heads, 128 experts top-8 with expert FFN 768; experts Q4_K,
router/attention Q8_0, lm-head Q6_K), batch 1, KV context pre-filled to 8192
positions with N(0,1) fp16, then greedy decode of 256 tokens from a 16-token
random-id prompt, seeded random-init weights.

    python -m benchmarks.moe_bench [--steps 256] [--warmup 16]

Prints one JSON line: decode tok/s, the engine's bytes-per-token model
(dmmvMetrics + flashAttnMetrics with fp16 KV and the 8 selected experts) and
the fraction of the 8 TB/s roofline, and per-layer launch-group times (HIP
events over replays with the step's arguments) against their algorithmic
bytes.
"""
import argparse
import json
import sys
import time

import numpy as np

from zinc_amd import hip
from zinc_amd.engine import MOE_48L, InferenceEngine

PEAK = 8000.0
PREFILL = 8192
N_PROMPT = 16


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--pages", choices=["ident", "shuffle"], default="ident",
                    help="KV page table: identity, or a seeded permutation (the paged attention kernel)")
    a = ap.parse_args()
    ctx = hip.Context(0)
    cfg = dict(MOE_48L)
    cfg["max_ctx"] = (PREFILL + N_PROMPT + a.warmup + a.steps + 16 + 15) // 16 * 16
    eng = InferenceEngine(ctx, cfg)
    if a.pages == "shuffle":
        eng.set_pages(np.random.default_rng(17).permutation(cfg["max_ctx"] // 16).astype(np.uint32))
    eng.prefill_kv_random(PREFILL, 7)
    ctx.sync()
    rng = np.random.default_rng(4321)
    prompt = [int(t) for t in rng.integers(0, cfg["vocab"], N_PROMPT)]
    warm = eng.generate(prompt, max(a.warmup, 1), start_pos=PREFILL)
    pos = PREFILL + N_PROMPT + len(warm) - 1
    ctx.sync()
    t0 = time.perf_counter()
    ctx.record(0)
    toks = eng.generate([warm[-1]], a.steps, start_pos=pos)
    ctx.record(1)
    ctx.sync()
    wall = time.perf_counter() - t0
    gpu_ms = ctx.elapsed_ms(0, 1)
    tok_s = a.steps / wall
    bpt = eng.bytes_per_token(pos + a.steps // 2)
    # per-layer launch groups, replayed with the step's own arguments
    L = pos + a.steps
    per = {}
    for g in eng.GROUPS:
        us = eng.time_kernel(g, 4 * cfg["n_layers"])
        nb = eng.group_bytes(g, L)
        per[g] = {"us": round(us, 3), "GBs": round(nb / us / 1e3, 1), "frac": round(nb / us / 1e3 / PEAK, 4)}
    eng.deinit()
    ctx.close()
    out = {"workload": "config 4: sparse-MoE decoder (48L, 2048 hidden, 32q/4kv heads, 128 experts top-8, "
                       "expert FFN 768, vocab 151936), batch 1, greedy decode at KV context 8192+",
           "steps": a.steps, "tok_s": round(tok_s, 2), "ms_per_token": round(wall * 1e3 / a.steps, 4),
           "gpu_ms_per_token": round(gpu_ms / a.steps, 4), "context_start": pos, "bytes_per_token": bpt,
           "token_roofline_frac": round(bpt * tok_s / 1e9 / PEAK, 4), "distinct_tokens": len(set(toks)),
           "per_kernel": per}
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
