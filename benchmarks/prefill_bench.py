"""Config 5 measurement: batched prefill of 512 random tokens on the 8B-shape
dense model (MFMA dequant-GEMM, fp16 operands, f32 accumulation), then greedy
decode over a 32768-position fp16 KV cache.

    python -m benchmarks.prefill_bench [--prefill 512] [--long-ctx 32768] [--steps 128]

Prints one JSON line. GEMM FLOPs per prefill = 2 * N * sum(M * K) over the
36 layers' Q, K, V, O, gate, up, down projections (7.11 TFLOP
for N = 512); attention FLOPs are not counted in that figure.
"""
import argparse
import json
import sys
import time

import numpy as np

from zinc_amd import hip
from zinc_amd.engine import DENSE_8B, InferenceEngine

PEAK_FP16_TFLOPS = 2500.0  # MI355X dense fp16 MFMA


def gemm_flops(cfg, n):
    H, qd, kvd, F = cfg["hidden"], cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"], cfg["ffn"]
    per_layer = qd * H + 2 * kvd * H + H * qd + 2 * F * H + H * F
    return 2.0 * n * per_layer * cfg["n_layers"]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--prefill", type=int, default=512)
    ap.add_argument("--long-ctx", type=int, default=32768)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--reps", type=int, default=5)
    a = ap.parse_args()
    ctx = hip.Context(0)
    cfg = dict(DENSE_8B)
    cfg["max_ctx"] = (max(a.long_ctx + a.steps + 32, a.prefill) + 15) // 16 * 16
    eng = InferenceEngine(ctx, cfg)
    rng = np.random.default_rng(5)
    toks = [int(t) for t in rng.integers(0, cfg["vocab"], a.prefill)]
    eng.prefill(toks, start_pos=0)  # warm-up (allocates the prefill buffers)
    ctx.sync()
    best = 1e9
    for _ in range(a.reps):
        ctx.record(0)
        eng.prefill(toks, start_pos=0)
        ctx.record(1)
        ctx.sync()
        best = min(best, ctx.elapsed_ms(0, 1))
    fl = gemm_flops(cfg, a.prefill)
    out = {"workload": f"config 5: batched prefill of {a.prefill} tokens, 8B-shape dense Q4_K_M",
           "prefill_ms": round(best, 3), "prefill_tok_s": round(a.prefill / (best * 1e-3), 1),
           "gemm_tflop": round(fl / 1e12, 3), "gemm_tflops_achieved": round(fl / (best * 1e-3) / 1e12, 1),
           "mfma_peak_frac": round(fl / (best * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 4)}
    # long-context decode: KV pre-filled to long_ctx with N(0,1) fp16
    t0 = time.time()
    eng.prefill_kv_random(a.long_ctx, 7)
    ctx.sync()
    prompt = [int(t) for t in rng.integers(0, cfg["vocab"], 2)]
    eng.generate(prompt, 8, start_pos=a.long_ctx)  # warm-up
    ctx.sync()
    ctx.record(2)
    gen = eng.generate([prompt[-1]], a.steps, start_pos=a.long_ctx + 9)
    ctx.record(3)
    ctx.sync()
    ms = ctx.elapsed_ms(2, 3)
    L = a.long_ctx + 9 + a.steps // 2
    bpt = eng.bytes_per_token(L)
    out.update({"long_ctx": a.long_ctx, "decode_tok_s": round(a.steps / (ms * 1e-3), 1),
                "decode_bytes_per_token": bpt, "decode_hbm_frac": round(bpt * a.steps / (ms * 1e-3) / 8e12, 4),
                "distinct_tokens": len(set(gen)), "kv_prefill_s": round(time.time() - t0, 1)})
    eng.deinit()
    ctx.close()
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
