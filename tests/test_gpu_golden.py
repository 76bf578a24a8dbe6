"""Full-size parity: the GPU engine decoding the config-3 model (8B-shaped
dense Qwen3, Q4_K_M mix, seeded random-init weights, 4096-token KV prefill)
must reproduce the CPU oracle's 256 greedy tokens exactly. The fixture
tests/golden/dense8b_greedy256.json was written by make_dense8b_golden.py
beside it (the oracle restates forward.zig's decodeStep + sampleGreedy)."""
import json
import os

import pytest

pytestmark = pytest.mark.gpu

FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "dense8b_greedy256.json")


def test_dense8b_greedy_256_token_exact():
    import zinc_amd
    g = json.load(open(FIXTURE))
    cfg = dict(g["config"])
    assert cfg["hidden"] == 4096 and cfg["n_layers"] == 36 and cfg["vocab"] == 151936
    ctx = zinc_amd.Context(0)
    try:
        eng = zinc_amd.InferenceEngine(ctx, cfg)
        eng.prefill_kv_random(g["prefill"], g["kv_seed"])
        got = eng.generate(g["prompt"], len(g["tokens"]), start_pos=g["prefill"])
        eng.deinit()
    finally:
        ctx.close()
    ref = g["tokens"]
    bad = [i for i in range(len(ref)) if got[i] != ref[i]]
    assert not bad, (f"first mismatch at step {bad[0]} (oracle margin there "
                     f"{g['rel_margins'][bad[0]]:.2e} of max |logit|)")
