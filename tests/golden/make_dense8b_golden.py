"""Writes tests/golden/dense8b_greedy256.json: the CPU oracle's greedy decode
of the BASELINE config-3 model (8B-shaped dense Qwen3, Q4_K_M mix, seeded
random-init weights, KV pre-filled to 4096 positions with N(0,1) fp16), a
16-token random prompt at positions 4096..4111, then 256 greedy tokens.

The oracle restates the reference's CPU path (dequantRow + serial f32 dot,
forward.zig / forward_metal.zig); the GPU test compares the engine's tokens to
this fixture. Also records the top-1/top-2 logit margin of every step.

Run: python tests/golden/make_dense8b_golden.py   (~10 min on 8 cores)
"""
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import oracle as orc  # noqa: E402
from zinc_amd.engine import DENSE_8B  # noqa: E402

PREFILL, N_PROMPT, N_GEN, KV_SEED, PROMPT_SEED = 4096, 16, 256, 7, 1234


def main():
    cfg = dict(DENSE_8B)
    cfg["max_ctx"] = PREFILL + N_PROMPT + N_GEN
    t0 = time.time()
    om = orc.Model(cfg, nthreads=os.cpu_count())
    om.prefill_kv_random(PREFILL, KV_SEED)
    print(f"model built in {time.time() - t0:.0f}s", flush=True)
    prompt = [int(t) for t in np.random.default_rng(PROMPT_SEED).integers(0, cfg["vocab"], N_PROMPT)]
    pos = PREFILL
    for t in prompt[:-1]:
        om.decode_step(t, pos)
        pos += 1
    tok, toks, margins = prompt[-1], [], []
    for i in range(N_GEN):
        tok, lg = om.decode_step(tok, pos, want_logits=True)
        s = np.sort(lg)
        margins.append(float(s[-1] - s[-2]) / float(np.abs(lg).max()))
        toks.append(int(tok))
        pos += 1
        if i % 16 == 0:
            print(f"step {i} tok {tok} rel-margin {margins[-1]:.3g} ({time.time() - t0:.0f}s)", flush=True)
    out = {"config": {k: (v if not isinstance(v, float) else float(v)) for k, v in cfg.items()},
           "prefill": PREFILL, "kv_seed": KV_SEED, "prompt": prompt, "tokens": toks,
           "rel_margins": margins, "generator": "oracle/zinc_oracle.c zo_model_decode_step"}
    with open(os.path.join(HERE, "dense8b_greedy256.json"), "w") as f:
        json.dump(out, f)
    print("min relative margin", min(margins))


if __name__ == "__main__":
    main()
