"""The sparse-MoE FFN in one launch with one selected expert per XCD
(k_moe_xcd: ffn_norm, router, top-8, the experts' gate/up + SwiGLU and down,
the weighted sum) on config 4's layer shapes: against the CPU oracle
(forward.zig's MoE path: router DMMV, topKSoftmax, expert DMMVs, weighted
accumulation) and against the engine's per-group launches."""
import numpy as np
import pytest

from test_gpu_engine import MOE_C4

pytestmark = pytest.mark.gpu
# below this router gap (k-th selected minus best unselected logit, over max
# |logit|) the GPU's selection may differ from the oracle's
ROUTE_EXACT = 1e-4


@pytest.fixture(scope="module")
def ctx():
    import zinc_amd
    c = zinc_amd.Context(0)
    yield c
    c.close()


def _engine(ctx, cfg, ffn=True):
    import zinc_amd
    eng = zinc_amd.InferenceEngine(ctx, cfg)
    eng.set_fused_ffn(ffn)
    return eng


def test_moe_launch_is_used(ctx):
    eng = _engine(ctx, MOE_C4)
    assert eng.group_kernels("ffn") == "k_moe_xcd(MoeP)" or (
        "k_moe_xcd" in eng.group_kernels("ffn") and ";" not in eng.group_kernels("ffn"))
    eng.set_fused_ffn(False)
    assert "k_moe_xcd" not in eng.group_kernels("ffn")
    eng.deinit()


@pytest.mark.parametrize("prefill", [0, 300])
def test_moe_step_matches_oracle(ctx, orc, prefill):
    import zinc_amd
    eng = _engine(ctx, MOE_C4)
    om = orc.Model(MOE_C4)
    if prefill:
        eng.prefill_kv_random(prefill, 7)
        om.prefill_kv_random(prefill, 7)
    st = zinc_amd.DecodeState()
    st.position = prefill
    eng.decode_step(st, 29, True)
    g_tok, g_log = eng.sample_greedy(), eng.logits()
    o_tok, o_log = om.decode_step(29, prefill, want_logits=True)
    scale = np.abs(o_log).max()
    assert np.abs(g_log - o_log).max() <= 1e-4 + 1e-3 * scale, (np.abs(g_log - o_log).max(), scale)
    assert g_tok == o_tok
    o_h = om.hidden()
    assert np.abs(eng.hidden() - o_h).max() <= 1e-4 + 1e-3 * np.abs(o_h).max()
    ctx.sync()  # no wait gave up, no expert id clamped
    eng.deinit()
    om.close()


def test_moe_equals_per_group_launches(ctx):
    """Same state through either FFN path: equal greedy tokens, logits within
    the tolerance (the experts' sums are added in another order)."""
    prefill = 200
    prompt = [int(t) for t in np.random.default_rng(11).integers(0, MOE_C4["vocab"], 5)]
    out = {}
    for ffn in (True, False):
        eng = _engine(ctx, MOE_C4, ffn)
        eng.prefill_kv_random(prefill, 4)
        out[ffn] = (eng.generate(prompt, 16, start_pos=prefill), eng.logits())
        eng.deinit()
    assert out[True][0] == out[False][0]
    scale = np.abs(out[False][1]).max()
    assert np.abs(out[True][1] - out[False][1]).max() <= 1e-4 + 1e-3 * scale


def test_moe_repeatable_after_replays(ctx):
    """A second generation from the same state repeats the first bit for
    bit, with group replays (which leave sums in the residual)
    and a weight re-pack between."""
    eng = _engine(ctx, MOE_C4)
    prefill = 150
    eng.prefill_kv_random(prefill, 6)
    prompt = [int(t) for t in np.random.default_rng(2).integers(0, MOE_C4["vocab"], 4)]
    got = eng.generate(prompt, 12, start_pos=prefill)
    lg = eng.logits()
    eng.time_kernel("ffn", 4)
    eng.tensor_bytes(2)  # (output_norm) hands out the arena: the packed copy is rebuilt before the next step
    again = eng.generate(prompt, 12, start_pos=prefill)
    # the residual's sums are fixed point, independent of the order of the
    # 8 XCDs' atomics: the second run is bit-identical
    assert np.array_equal(eng.logits().view(np.uint32), lg.view(np.uint32))
    assert again == got
    ctx.sync()
    eng.deinit()


def test_moe_wait_give_up_reports_and_recovers(orc):
    """With the wait limit at 0 every bounded wait gives up at once (every
    workgroup still finishes): the output is NaN, zh_sync reports
    WaitTimeout; the next steps with the default limit equal those of an
    engine that never gave up, and match the oracle (logits within the decode
    tolerance wherever every layer's router gap exceeds ROUTE_EXACT: below it
    the hidden state's ~1e-5 difference from the oracle may flip an expert)."""
    import zinc_amd
    c = zinc_amd.Context(0)
    try:
        eng = _engine(c, MOE_C4)
        clean = _engine(c, MOE_C4)
        assert "k_moe_xcd" in eng.group_kernels("ffn")
        om = orc.Model(MOE_C4)
        st = zinc_amd.DecodeState()
        c.set_attn_wait_limit(0)
        st.position = 0
        eng.decode_step(st, 5, True)
        assert np.isnan(eng.hidden()).any()
        with pytest.raises(zinc_amd.ZincError) as e:
            c.sync()
        assert e.value.name == "WaitTimeout"
        c.sync()
        c.set_attn_wait_limit(50000)
        # the failed position again: until this step writes them, its cache
        # rows hold what the failed step wrote (NaN where a wait gave up),
        # which the attention's masked tail rows copy
        _, o_log = om.decode_step(5, 0, want_logits=True)
        st.position = 0
        eng.decode_step(st, 5, True)
        scale = np.abs(o_log).max()
        assert np.abs(eng.logits() - o_log).max() <= 1e-4 + 1e-3 * scale
        st.position = 0
        clean.decode_step(st, 5, False)
        for step in range(1, 3):
            st.position = step
            eng.decode_step(st, 9 + step, True)
            g_log = eng.logits()
            st.position = step  # (decode_step advanced it)
            clean.decode_step(st, 9 + step, True)
            c_log = clean.logits()
            o_tok, o_log = om.decode_step(9 + step, step, want_logits=True)
            scale = np.abs(o_log).max()
            gaps = [om.routing(layer)[2] for layer in range(MOE_C4["n_layers"])]
            print(f"step {step}: |recovered - clean| {np.abs(g_log - c_log).max() / scale:.2e}, "
                  f"|recovered - oracle| {np.abs(g_log - o_log).max() / scale:.2e} of scale, "
                  f"router gaps {gaps}", flush=True)
            assert np.abs(g_log - c_log).max() <= 1e-4 * scale, step
            if min(gaps) > ROUTE_EXACT:
                assert np.abs(g_log - o_log).max() <= 1e-4 + 1e-3 * scale, step
        c.sync()
        eng.deinit()
        clean.deinit()
        om.close()
    finally:
        c.close()
