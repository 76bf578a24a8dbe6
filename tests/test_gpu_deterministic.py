"""Deterministic decode: the per-XCD launches add their partial rows into the
residual as 64-bit fixed point (integer atomics commute), so the same
decode on the same device gives bit-identical logits, hidden state and
tokens, whatever order the atomics land in. (The reference adds each
contribution in a fixed order: dispatchDmmvAcc, forward.zig:8219-8229;
moe_weighted_acc.comp.)"""
import numpy as np
import pytest

from test_gpu_engine import MOE_C4
from test_gpu_qkv_attn import FUSED

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    import zinc_amd
    c = zinc_amd.Context(0)
    yield c
    c.close()


def _run(ctx, cfg, prefill, prompt, n):
    import zinc_amd
    eng = zinc_amd.InferenceEngine(ctx, cfg)
    eng.prefill_kv_random(prefill, 3)
    toks = eng.generate(prompt, n, start_pos=prefill)
    out = (toks, eng.logits().copy(), eng.hidden().copy())
    # the same engine again, after per-group replays (which leave sums in the
    # residual's accumulator; the engine clears it)
    eng.time_kernel("ffn", 4)
    toks2 = eng.generate(prompt, n, start_pos=prefill)
    again = (toks2, eng.logits().copy(), eng.hidden().copy())
    kernels = eng.group_kernels("ffn")
    eng.deinit()
    return out, again, kernels


@pytest.mark.parametrize("name,cfg,launch", [("dense", FUSED, "k_ffn_xcd"), ("moe", MOE_C4, "k_moe_xcd")])
def test_decode_is_bit_identical(ctx, name, cfg, launch):
    prompt = [int(t) for t in np.random.default_rng(8).integers(0, cfg["vocab"], 5)]
    a, a2, kernels = _run(ctx, cfg, 300, prompt, 24)
    assert launch in kernels
    b, _, _ = _run(ctx, cfg, 300, prompt, 24)
    for x, y in ((a, a2), (a, b)):
        assert x[0] == y[0]
        assert np.array_equal(x[1].view(np.uint32), y[1].view(np.uint32)), name
        assert np.array_equal(x[2].view(np.uint32), y[2].view(np.uint32)), name
    ctx.sync()
