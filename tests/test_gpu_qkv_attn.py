"""The decode step's Q/K/V projection and attention in one launch
(k_qkv_attn: one kv head per XCD, the exchanges through the XCD's L2) on the
8B model's layer shapes, against the CPU oracle (forward.zig's Q/K/V DMMVs +
qk norm / RoPE / KV write + flash decode) and against the two-launch path of
the same engine."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# config 3's layer shapes (hidden 4096, 32 q / 8 kv heads, Q4_K attention,
# ffn 12288) in two layers and a small vocabulary
FUSED = dict(n_layers=2, hidden=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=12288, vocab=4000,
             n_experts=0, n_experts_used=0, expert_ffn=0, max_ctx=4224,
             type_attn=12, type_ffn_gate_up=12, type_ffn_down=14, type_lm_head=14, type_embd=12,
             type_router=8, rope_base=1e6, eps=1e-6, seed=91)


@pytest.fixture(scope="module")
def ctx():
    import zinc_amd
    c = zinc_amd.Context(0)
    yield c
    c.close()


def _engine(ctx, cfg, fused=True):
    import zinc_amd
    eng = zinc_amd.InferenceEngine(ctx, cfg)
    eng.set_fused_attn(fused)
    return eng


def test_fused_launch_is_used(ctx):
    eng = _engine(ctx, FUSED)
    assert "k_qkv_attn" in eng.group_kernels("qkv_attn")
    # with the O projection: one launch for the three groups
    assert "k_qkv_attn" in eng.group_kernels("qkv_attn_o") and ";" not in eng.group_kernels("qkv_attn_o")
    eng.set_fused_attn(False)
    names = eng.group_kernels("qkv_attn")
    assert "k_qkv_attn" not in names and "attn" in names
    eng.deinit()
    # shapes it does not take run the two launches
    small = dict(FUSED, n_kv_heads=4)
    eng = _engine(ctx, small)
    assert "k_qkv_attn" not in eng.group_kernels("qkv_attn")
    eng.deinit()


# 100: one sub-chunk per chunk, most chunks empty; 4000: three 64-token
# sub-chunks per chunk (the last in the region the projection staged x in);
# 4100: the position in chunk 31 with 3 sub-chunks
@pytest.mark.parametrize("prefill", [100, 4000, 4100])
def test_fused_step_matches_oracle(ctx, orc, prefill):
    import zinc_amd
    eng = _engine(ctx, FUSED)
    om = orc.Model(FUSED)
    eng.prefill_kv_random(prefill, 7)
    om.prefill_kv_random(prefill, 7)
    st = zinc_amd.DecodeState()
    st.position = prefill
    eng.decode_step(st, 17, True)
    g_tok, g_log = eng.sample_greedy(), eng.logits()
    o_tok, o_log = om.decode_step(17, prefill, want_logits=True)
    scale = np.abs(o_log).max()
    assert np.abs(g_log - o_log).max() <= 1e-4 + 1e-3 * scale, (np.abs(g_log - o_log).max(), scale)
    assert g_tok == o_tok
    # the new token's K/V rows (layer 0 takes the oracle's own inputs: f16
    # rows equal up to one ulp plus 1e-5 of the head's largest element)
    hd = FUSED["head_dim"]
    for which in (0, 1):
        g = eng.read_kv(0, which, prefill, 1).view(np.float16).astype(np.float32)
        o16 = om.kv(0, which, prefill).view(np.float16)
        o = o16.astype(np.float32)
        rowmax = np.repeat(np.abs(o).reshape(-1, hd).max(axis=1), hd)
        bound = np.spacing(np.abs(o16)).astype(np.float32) + 1e-5 * rowmax
        assert (np.abs(g - o) <= bound).all(), which
    ctx.sync()  # no wait gave up
    eng.deinit()
    om.close()


# longer contexts stream their sub-chunks through the four-slot ring: 8300
# (five per chunk: one slot reused), 11900 (the new token in sub-chunk 5 of its
# chunk, written into its slot after the copy), 12000 (six per chunk)
FUSED_LONG = dict(FUSED, max_ctx=12288)


@pytest.mark.parametrize("prefill", [8300, 11900, 12000])
def test_fused_long_context_matches_oracle(ctx, orc, prefill):
    import zinc_amd
    eng = _engine(ctx, FUSED_LONG)
    assert "k_qkv_attn" in eng.group_kernels("qkv_attn")
    om = orc.Model(FUSED_LONG)
    eng.prefill_kv_random(prefill, 3)
    om.prefill_kv_random(prefill, 3)
    st = zinc_amd.DecodeState()
    for step in range(2):
        st.position = prefill + step
        eng.decode_step(st, 31 + step, True)
        g_log = eng.logits()
        o_tok, o_log = om.decode_step(31 + step, prefill + step, want_logits=True)
        scale = np.abs(o_log).max()
        assert np.abs(g_log - o_log).max() <= 1e-4 + 1e-3 * scale, (step, np.abs(g_log - o_log).max(), scale)
        assert eng.sample_greedy() == o_tok
    ctx.sync()
    eng.deinit()
    om.close()


def test_fused_equals_two_launch_path(ctx):
    """Same engine state through either path: the projection's rows are the
    same arithmetic (bit-identical); the attention differs only in summation
    order, so the greedy tokens agree and the logits within the tolerance."""
    prefill = 3000
    prompt = [int(t) for t in np.random.default_rng(5).integers(0, FUSED["vocab"], 5)]
    out = {}
    for fused in (True, False):
        eng = _engine(ctx, FUSED, fused)
        eng.prefill_kv_random(prefill, 9)
        out[fused] = (eng.generate(prompt, 24, start_pos=prefill), eng.logits())
        eng.deinit()
    assert out[True][0] == out[False][0]
    scale = np.abs(out[False][1]).max()
    assert np.abs(out[True][1] - out[False][1]).max() <= 1e-4 + 1e-3 * scale


def test_fused_generate_token_exact_and_repeatable(ctx, orc):
    """Greedy generation equals the oracle's, and a second generation from the
    same state repeats it: the flags' epochs advance per launch, so flags left
    by the first run never satisfy a wait of the second."""
    eng = _engine(ctx, FUSED)
    om = orc.Model(FUSED)
    prefill, n_gen = 2000, 20
    eng.prefill_kv_random(prefill, 5)
    om.prefill_kv_random(prefill, 5)
    prompt = [int(t) for t in np.random.default_rng(3).integers(0, FUSED["vocab"], 6)]
    got = eng.generate(prompt, n_gen, start_pos=prefill)
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


def test_fused_wait_give_up_reports_and_recovers(orc):
    """With the wait limit at 0 (the host makes every bounded wait give up at
    once; every workgroup still finishes) the attention output is NaN and
    zh_sync reports WaitTimeout; the next step with the default limit matches
    the oracle again."""
    import zinc_amd
    c = zinc_amd.Context(0)
    try:
        eng = _engine(c, FUSED)
        assert "k_qkv_attn" in eng.group_kernels("qkv_attn")
        om = orc.Model(FUSED)
        prefill = 1500
        eng.prefill_kv_random(prefill, 13)
        om.prefill_kv_random(prefill, 13)
        st = zinc_amd.DecodeState()
        c.set_attn_wait_limit(0)
        st.position = prefill
        eng.decode_step(st, 7, True)
        assert np.isnan(eng.hidden()).any()
        with pytest.raises(zinc_amd.ZincError) as e:
            c.sync()
        assert e.value.name == "WaitTimeout"
        c.sync()
        # zh_sync checked the workgroup placement again (it holds: the fused
        # launch stays) and the engine re-records its step
        assert "k_qkv_attn" in eng.group_kernels("qkv_attn")
        c.set_attn_wait_limit(50000)
        # the failed position again: until this step writes them, its cache
        # rows hold what the failed step wrote (NaN where a wait gave up),
        # which the attention's masked tail rows copy
        _, o_log = om.decode_step(7, prefill, want_logits=True)
        st.position = prefill
        eng.decode_step(st, 7, True)
        scale = np.abs(o_log).max()
        assert np.abs(eng.logits() - o_log).max() <= 1e-4 + 1e-3 * scale
        for step in range(1, 3):
            st.position = prefill + step
            eng.decode_step(st, 9 + step, True)
            g_log = eng.logits()
            o_tok, o_log = om.decode_step(9 + step, prefill + step, want_logits=True)
            scale = np.abs(o_log).max()
            assert np.abs(g_log - o_log).max() <= 1e-4 + 1e-3 * scale, step
        c.sync()
        eng.deinit()
        om.close()
    finally:
        c.close()
