"""The dense FFN in one launch split by XCD (k_ffn_xcd: ffn_norm, gate/up +
SwiGLU, down + residual; the SwiGLU slice exchanged through each XCD's L2)
together with the split residual it shares with the fused attention launch,
on the 8B model's layer shapes: against the CPU oracle (forward.zig's
ffn_norm / gate-up / SwiGLU / down DMMVs) and against the engine's
per-group launches."""
import numpy as np
import pytest

from test_gpu_qkv_attn import FUSED

pytestmark = pytest.mark.gpu


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


def test_ffn_launch_is_used(ctx):
    eng = _engine(ctx, FUSED)
    assert eng.group_kernels("ffn") == "k_ffn_xcd" or "k_ffn_xcd" in eng.group_kernels("ffn")
    assert ";" not in eng.group_kernels("ffn")
    eng.set_fused_ffn(False)
    assert "k_ffn_xcd" not in eng.group_kernels("ffn")
    eng.deinit()
    # without the fused attention (whose O phase starts the split residual)
    # the FFN runs as separate launches
    eng = _engine(ctx, FUSED)
    eng.set_fused_attn(False)
    assert "k_ffn_xcd" not in eng.group_kernels("ffn")
    eng.deinit()


@pytest.mark.parametrize("prefill", [0, 100, 4000])
def test_ffn_step_matches_oracle(ctx, orc, prefill):
    import zinc_amd
    eng = _engine(ctx, FUSED)
    om = orc.Model(FUSED)
    if prefill:
        eng.prefill_kv_random(prefill, 7)
        om.prefill_kv_random(prefill, 7)
    st = zinc_amd.DecodeState()
    st.position = prefill
    eng.decode_step(st, 23, True)
    g_tok, g_log = eng.sample_greedy(), eng.logits()
    o_tok, o_log = om.decode_step(23, prefill, want_logits=True)
    scale = np.abs(o_log).max()
    assert np.abs(g_log - o_log).max() <= 1e-4 + 1e-3 * scale, (np.abs(g_log - o_log).max(), scale)
    assert g_tok == o_tok
    # the residual stream after the last layer (folded into hidden)
    o_h = om.hidden()
    assert np.abs(eng.hidden() - o_h).max() <= 1e-4 + 1e-3 * np.abs(o_h).max()
    ctx.sync()  # no wait gave up
    eng.deinit()
    om.close()


def test_ffn_equals_per_group_launches(ctx):
    """Same engine state through either FFN path: equal greedy tokens, logits
    within the tolerance (the residual is summed in another order)."""
    prefill = 2500
    prompt = [int(t) for t in np.random.default_rng(8).integers(0, FUSED["vocab"], 5)]
    out = {}
    for ffn in (True, False):
        eng = _engine(ctx, FUSED, ffn)
        eng.prefill_kv_random(prefill, 4)
        out[ffn] = (eng.generate(prompt, 24, start_pos=prefill), eng.logits())
        eng.deinit()
    assert out[True][0] == out[False][0]
    scale = np.abs(out[False][1]).max()
    assert np.abs(out[True][1] - out[False][1]).max() <= 1e-4 + 1e-3 * scale


def test_ffn_generate_token_exact_and_repeatable(ctx, orc):
    """Greedy generation equals the oracle's; a second run from the same state
    repeats it (flag epochs advance per launch; the split residual's atomic
    sums are cleared by the launches themselves and by the step's fold)."""
    eng = _engine(ctx, FUSED)
    om = orc.Model(FUSED)
    prefill, n_gen = 1200, 20
    eng.prefill_kv_random(prefill, 6)
    om.prefill_kv_random(prefill, 6)
    prompt = [int(t) for t in np.random.default_rng(2).integers(0, FUSED["vocab"], 6)]
    got = eng.generate(prompt, n_gen, start_pos=prefill)
    eng.time_kernel("ffn", 8)       # replays between the runs leave sums behind, reset after timing
    eng.time_kernel("qkv_attn_o", 8)
    again = eng.generate(prompt, n_gen, start_pos=prefill)
    pos = prefill
    for t in prompt[:-1]:
        om.decode_step(t, pos)
        pos += 1
    ref, tok = [], prompt[-1]
    for _ in range(n_gen):
        tok = om.decode_step(tok, pos)
        pos += 1
        ref.append(int(tok))
    assert got == ref, f"first mismatch at {next(i for i in range(n_gen) if got[i] != ref[i])}"
    assert again == got
    ctx.sync()
    eng.deinit()
    om.close()


def test_ffn_wait_give_up_reports_and_recovers(orc):
    """With the wait limit at 0 (every bounded wait gives up at once; every
    workgroup still finishes) the step's output is NaN and zh_sync reports
    WaitTimeout; the next steps with the default limit match the oracle."""
    import zinc_amd
    c = zinc_amd.Context(0)
    try:
        eng = _engine(c, FUSED)
        assert "k_ffn_xcd" in eng.group_kernels("ffn")
        om = orc.Model(FUSED)
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
        for step in range(1, 3):
            st.position = step
            eng.decode_step(st, 9 + step, True)
            g_log = eng.logits()
            o_tok, o_log = om.decode_step(9 + step, step, want_logits=True)
            scale = np.abs(o_log).max()
            assert np.abs(g_log - o_log).max() <= 1e-4 + 1e-3 * scale, step
        c.sync()
        eng.deinit()
        om.close()
    finally:
        c.close()
