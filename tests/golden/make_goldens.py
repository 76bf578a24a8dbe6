"""Writes the full-size parity fixtures for BASELINE configs 4 and 5 with the
CPU oracle (oracle/zinc_oracle.c, which restates the reference's
dequantRow + serial f32 dot decode path, forward.zig / forward_metal.zig):

  moe48        config 4: 48-layer MoE (hidden 2048, 32 q / 4 kv heads, 128
               experts top-8, expert FFN 768; experts Q4_K, router and
               attention Q8_0, LM head Q6_K over vocab 151936), KV prefilled to
               8192 positions, a 16-token prompt, then 256 greedy tokens
               -> moe48_greedy256.json, and every decode step's per-layer
               expert selection and router gap -> moe48_routing.npz
  dense8b_32k  config 5 decode: the 8B-shaped dense model (config 3's),
               KV prefilled to 32768 positions, a 16-token prompt, then 128
               greedy tokens -> dense8b_32k_greedy128.json
  prefill512   config 5 prefill: the 8B layer shapes (4 layers, vocab 8192),
               a 512-token random prompt decoded token by token, then 16 greedy
               tokens; the logits after the prompt and the last layer's K/V
               rows at a few positions -> prefill512_8b4l.npz

Run: python tests/golden/make_goldens.py NAME [NAME ...]   (minutes each on 8 cores)
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
from zinc_amd.engine import DENSE_8B, MOE_48L  # noqa: E402

N_PROMPT, KV_SEED, PROMPT_SEED = 16, 7, 1234


def greedy_fixture(cfg, prefill, n_gen, out_name):
    t0 = time.time()
    cfg = dict(cfg)
    cfg["max_ctx"] = (prefill + N_PROMPT + n_gen + 15) // 16 * 16
    om = orc.Model(cfg, nthreads=os.cpu_count())
    om.prefill_kv_random(prefill, KV_SEED)
    print(f"{out_name}: model built in {time.time() - t0:.0f}s", flush=True)
    prompt = [int(t) for t in np.random.default_rng(PROMPT_SEED).integers(0, cfg["vocab"], N_PROMPT)]
    routed = cfg.get("n_experts", 0) > 0
    r_ids, r_gaps = [], []

    def record_routing():
        if routed:
            sel = [om.routing(layer) for layer in range(cfg["n_layers"])]
            r_ids.append([s[0].tolist() for s in sel])
            r_gaps.append([s[2] for s in sel])

    pos = prefill
    for t in prompt[:-1]:
        om.decode_step(t, pos)
        record_routing()
        pos += 1
    tok, toks, margins, gaps = prompt[-1], [], [], []
    for i in range(n_gen):
        tok, lg = om.decode_step(tok, pos, want_logits=True)
        s = np.sort(lg)
        margins.append(float(s[-1] - s[-2]) / float(np.abs(lg).max()))
        gaps.append(min(om.route_gap(), 1.0))
        record_routing()
        toks.append(int(tok))
        pos += 1
        if i % 16 == 0:
            print(f"  step {i} tok {tok} rel-margin {margins[-1]:.3g} ({time.time() - t0:.0f}s)", flush=True)
    om.close()
    out = {"config": {k: (v if not isinstance(v, float) else float(v)) for k, v in cfg.items()},
           "prefill": prefill, "kv_seed": KV_SEED, "prompt": prompt, "tokens": toks,
           "rel_margins": margins, "route_gaps": gaps, "generator": "oracle/zinc_oracle.c zo_model_decode_step"}
    with open(os.path.join(HERE, out_name), "w") as f:
        json.dump(out, f)
    if routed:
        # decode step s (the prompt's first N_PROMPT - 1 tokens, then the
        # generated steps), layer l: the oracle's selected experts and that
        # layer's router gap (zo_model_routing)
        np.savez_compressed(os.path.join(HERE, out_name.split("_")[0] + "_routing.npz"),
                            ids=np.array(r_ids, dtype=np.uint8), gaps=np.array(r_gaps, dtype=np.float32))
    print(f"{out_name}: min relative margin {min(margins):.3g}, {time.time() - t0:.0f}s", flush=True)


PREFILL512_CFG = dict(DENSE_8B, n_layers=4, vocab=8192, max_ctx=512 + 32, seed=1241)
PREFILL512_N, PREFILL512_GEN, PREFILL512_ROWS = 512, 16, (0, 1, 255, 510, 511)


def prefill512():
    t0 = time.time()
    cfg = dict(PREFILL512_CFG)
    om = orc.Model(cfg, nthreads=os.cpu_count())
    prompt = np.random.default_rng(PROMPT_SEED + 1).integers(0, cfg["vocab"], PREFILL512_N).astype(np.uint32)
    for p, t in enumerate(prompt[:-1]):
        om.decode_step(int(t), p)
    tok, logits = om.decode_step(int(prompt[-1]), PREFILL512_N - 1, want_logits=True)
    kv = np.stack([np.stack([om.kv(cfg["n_layers"] - 1, w, r) for r in PREFILL512_ROWS]) for w in (0, 1)])
    toks, pos = [int(tok)], PREFILL512_N
    for _ in range(PREFILL512_GEN - 1):
        tok = om.decode_step(int(tok), pos)
        toks.append(int(tok))
        pos += 1
    om.close()
    np.savez_compressed(os.path.join(HERE, "prefill512_8b4l.npz"), prompt=prompt, logits=logits,
                        kv_rows=np.array(PREFILL512_ROWS, np.uint32), kv=kv, tokens=np.array(toks, np.uint32),
                        config=json.dumps({k: (v if not isinstance(v, float) else float(v)) for k, v in cfg.items()}))
    print(f"prefill512: {time.time() - t0:.0f}s, tokens {toks}", flush=True)


def main():
    for name in sys.argv[1:] or ["moe48", "dense8b_32k", "prefill512"]:
        if name == "moe48":
            greedy_fixture(MOE_48L, 8192, 256, "moe48_greedy256.json")
        elif name == "dense8b_32k":
            greedy_fixture(DENSE_8B, 32768, 128, "dense8b_32k_greedy128.json")
        elif name == "prefill512":
            prefill512()
        else:
            raise SystemExit(f"unknown fixture {name}")


if __name__ == "__main__":
    main()
