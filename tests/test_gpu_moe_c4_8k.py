"""Config 4's decode step at its real context: the config-4 layer shapes
(hidden 2048, 32 q / 4 kv heads, Q8_0 attention and router, 128 experts top-8,
expert FFN 768) in two layers over an 8K fp16 KV cache, against the CPU
oracle (forward.zig:5958-6500 for the MoE FFN, topKSoftmax :496-537,
attention.zig:199-316 for the attention).

At 8K context the fused attention launch (one kv head per XCD pair) streams
five 64-token sub-chunks per workgroup (the fourth into the weight region once
the rows are computed, the fifth into the first sub-chunk's slot) and reads the
Q8_0 rows as 68-byte block pairs; the MoE launch selects its experts on every
XCD. Checked per step: the logits and the hidden state within the decode
tolerance, the new token's K/V rows within one f16 ulp plus 1e-5 of the
head's largest element (layer 0; 1e-4 past it), and each layer's selected experts equal to
the oracle's wherever the oracle's router gap (k-th selected minus best
unselected logit, over max |router logit|) exceeds ROUTE_EXACT."""
import numpy as np
import pytest

from test_gpu_engine import MOE_C4

pytestmark = pytest.mark.gpu

C4_8K = dict(MOE_C4, max_ctx=8192 + 64)
# The GPU's hidden state differs from the oracle's by ~1e-5 of its scale (the
# same sums in another order), which can flip a selection whose gap is of
# that order; above this the selection must be the oracle's.
ROUTE_EXACT = 1e-4


@pytest.fixture(scope="module")
def ctx():
    import zinc_amd
    c = zinc_amd.Context(0)
    yield c
    c.close()


def _check_step(eng, om, tok, pos):
    hd = C4_8K["head_dim"]
    eng_st = __import__("zinc_amd").DecodeState()
    eng_st.position = pos
    eng.decode_step(eng_st, tok, True)
    g_tok, g_log, g_h = eng.sample_greedy(), eng.logits(), eng.hidden()
    o_tok, o_log = om.decode_step(tok, pos, want_logits=True)
    o_h = om.hidden()
    scale = np.abs(o_log).max()
    d_log = np.abs(g_log - o_log).max()
    d_h = np.abs(g_h - o_h).max()
    print(f"pos {pos}: |logit - oracle| {d_log / scale:.2e} of scale, |hidden - oracle| "
          f"{d_h / np.abs(o_h).max():.2e} of scale", flush=True)
    assert d_log <= 1e-4 + 1e-3 * scale, (d_log, scale)
    assert d_h <= 1e-4 + 1e-3 * np.abs(o_h).max(), d_h
    for layer in range(C4_8K["n_layers"]):
        for which in (0, 1):
            g = eng.read_kv(layer, which, pos, 1).view(np.float16).astype(np.float32)
            o16 = om.kv(layer, which, pos).view(np.float16)
            o = o16.astype(np.float32)
            rowmax = np.repeat(np.abs(o).reshape(-1, hd).max(axis=1), hd)
            # one f16 ulp (of the larger value: a rounding may cross a binade)
            # plus 1e-5 of the head's largest element; past layer 0 the
            # layer's input carries the hidden state's ~1e-5 drift, which the
            # Q8_0 projection (weights ~1.5, K = 2048) turns into up to ~1e-4
            # of the row maximum before the f16 rounding
            ulp = np.spacing(np.maximum(np.abs(o16), np.abs(g).astype(np.float16))).astype(np.float32)
            bound = ulp + (1e-5 if layer == 0 else 1e-4) * rowmax
            assert (np.abs(g - o) <= bound).all(), (pos, layer, which, float(np.abs(g - o).max()))
        g_ids, g_w = eng.routing(layer)
        o_ids, o_w, gap = om.routing(layer)
        print(f"  layer {layer}: gpu experts {sorted(g_ids.tolist())}, oracle {sorted(o_ids.tolist())}, "
              f"gap {gap:.2e}", flush=True)
        assert len(set(g_ids.tolist())) == len(g_ids) and abs(float(g_w.sum()) - 1.0) < 1e-5
        # experts with a positive weight: the same, with the same weights (a
        # selection that softmax underflow fills with zero-weight experts has
        # no tie among the ones that contribute, and which zero-weight
        # experts fill it does not change the output)
        g_pos = {int(e): float(x) for e, x in zip(g_ids, g_w) if x > 0}
        o_pos = {int(e): float(x) for e, x in zip(o_ids, o_w) if x > 0}
        if gap > ROUTE_EXACT:
            assert sorted(g_pos) == sorted(o_pos), (pos, layer, gap)
            assert all(abs(g_pos[e] - o_pos[e]) <= 1e-4 for e in o_pos), (pos, layer)
            if gap != float("inf"):
                assert sorted(g_ids.tolist()) == sorted(o_ids.tolist()), (pos, layer, gap)
    return g_tok, o_tok


@pytest.mark.parametrize("prefill", [8000, 8192])
def test_moe_c4_8k_steps_match_oracle(ctx, orc, prefill):
    import zinc_amd
    eng = zinc_amd.InferenceEngine(ctx, C4_8K)
    # the fused launches are the ones under test
    assert "k_qkv_attn" in eng.group_kernels("qkv_attn_o") and ";" not in eng.group_kernels("qkv_attn_o")
    assert "k_moe_xcd" in eng.group_kernels("ffn")
    om = orc.Model(C4_8K)
    eng.prefill_kv_random(prefill, 5)
    om.prefill_kv_random(prefill, 5)
    tok = 23
    for pos in (prefill, prefill + 1, prefill + 2):
        g_tok, o_tok = _check_step(eng, om, tok, pos)
        assert g_tok == o_tok
        tok = o_tok
    ctx.sync()  # no wait gave up, no expert id clamped
    eng.deinit()
    om.close()


def test_moe_c4_8k_many_positions(ctx, orc):
    """Every position of a 72-step stretch past 8192 (chunk and sub-chunk
    boundaries move with the context length), fed the oracle's tokens: the
    logits within the decode tolerance at each step."""
    import zinc_amd
    eng = zinc_amd.InferenceEngine(ctx, dict(C4_8K, max_ctx=8192 + 128))
    om = orc.Model(dict(C4_8K, max_ctx=8192 + 128))
    prefill = 8190
    eng.prefill_kv_random(prefill, 3)
    om.prefill_kv_random(prefill, 3)
    st = zinc_amd.DecodeState()
    tok, bad = 41, []
    for pos in range(prefill, prefill + 72):
        st.position = pos
        eng.decode_step(st, tok, True)
        g_log = eng.logits()
        o_tok, o_log = om.decode_step(tok, pos, want_logits=True)
        scale = np.abs(o_log).max()
        d = np.abs(g_log - o_log).max()
        if d > 1e-4 + 1e-3 * scale:
            bad.append((pos, float(d / scale)))
        tok = o_tok
    print(f"positions past {prefill}: {len(bad)} outside the tolerance {bad[:10]}", flush=True)
    ctx.sync()
    eng.deinit()
    om.close()
    assert not bad, bad[:10]
