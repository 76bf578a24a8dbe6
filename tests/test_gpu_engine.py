"""Whole decode loop on the GPU engine vs the CPU oracle model (same seeded
weights, same KV prefill): logits within tolerance and greedy tokens equal."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SMALL_DENSE = dict(n_layers=3, hidden=512, n_heads=4, n_kv_heads=2, head_dim=128, ffn=1536, vocab=3000,
                   n_experts=0, n_experts_used=0, expert_ffn=0, max_ctx=512,
                   type_attn=12, type_ffn_gate_up=12, type_ffn_down=14, type_lm_head=14, type_embd=12,
                   type_router=8, rope_base=1e6, eps=1e-6, seed=99)
SMALL_MOE = dict(n_layers=2, hidden=512, n_heads=8, n_kv_heads=1, head_dim=128, ffn=0, vocab=2000,
                 n_experts=16, n_experts_used=4, expert_ffn=256, max_ctx=256,
                 type_attn=8, type_ffn_gate_up=12, type_ffn_down=12, type_lm_head=14, type_embd=12,
                 type_router=8, rope_base=1e6, eps=1e-6, seed=98)

# config 4's layer shapes (hidden 2048, 32 q / 4 kv heads, 128 experts top-8,
# expert FFN 768, Q8_0 attention/router) in two layers and a small vocabulary
MOE_C4 = dict(n_layers=2, hidden=2048, n_heads=32, n_kv_heads=4, head_dim=128, ffn=0, vocab=4000,
              n_experts=128, n_experts_used=8, expert_ffn=768, max_ctx=512,
              type_attn=8, type_ffn_gate_up=12, type_ffn_down=12, type_lm_head=14, type_embd=12,
              type_router=8, rope_base=1e6, eps=1e-6, seed=97)


# the streaming kernels' shapes: Q4_K projections at K = 2048, the Q6_K down
# projection at K = 12288 (2048 rows over 256 workgroups: 8 rows each, two
# passes of 5 and 3 rows)
DENSE_RING = dict(n_layers=2, hidden=2048, n_heads=16, n_kv_heads=4, head_dim=128, ffn=12288, vocab=3000,
                  n_experts=0, n_experts_used=0, expert_ffn=0, max_ctx=512,
                  type_attn=12, type_ffn_gate_up=12, type_ffn_down=14, type_lm_head=14, type_embd=12,
                  type_router=8, rope_base=1e6, eps=1e-6, seed=94)


@pytest.fixture(scope="module")
def ctx():
    import zinc_amd
    c = zinc_amd.Context(0)
    yield c
    c.close()


def margin(logits):
    s = np.sort(logits)
    return float(s[-1] - s[-2])


@pytest.mark.parametrize("cfg", [SMALL_DENSE, SMALL_MOE], ids=["dense", "moe"])
def test_engine_weights_match_oracle(ctx, orc, cfg):
    import zinc_amd
    eng = zinc_amd.InferenceEngine(ctx, cfg)
    om = orc.Model(cfg)
    streams = [1, 2, 3] + [orc.S_LAYER(l, k) for l in range(cfg["n_layers"]) for k in range(1, 16)]
    for s in streams:
        ref = om.tensor(s)
        if ref is None:
            continue
        assert np.array_equal(eng.tensor_bytes(s), ref), hex(s)
    eng.deinit()
    om.close()


@pytest.mark.parametrize("cfg", [SMALL_DENSE, SMALL_MOE, MOE_C4, DENSE_RING], ids=["dense", "moe", "moe_c4", "ring"])
def test_engine_decode_matches_oracle(ctx, orc, cfg):
    import zinc_amd
    eng = zinc_amd.InferenceEngine(ctx, cfg)
    om = orc.Model(cfg)
    prefill = 100
    eng.prefill_kv_random(prefill, 7)
    om.prefill_kv_random(prefill, 7)
    # one explicit decodeStep and its logits
    state = zinc_amd.DecodeState()
    state.position = prefill
    tok0 = 17
    eng.decode_step(state, tok0, True)
    g_tok = eng.sample_greedy()
    g_log = eng.logits()
    o_tok, o_log = om.decode_step(tok0, prefill, want_logits=True)
    assert np.allclose(g_log, o_log, rtol=1e-3, atol=1e-4 + 1e-3 * np.abs(o_log).max()), \
        f"max |d| {np.abs(g_log - o_log).max()} vs scale {np.abs(o_log).max()}"
    assert g_tok == o_tok
    # the K/V rows written for the new token: finite, and equal to the
    # oracle's fp16 rows except where the f32 inputs themselves differ by
    # rounding: then by at most one f16 ulp of the element plus 1e-5 of its
    # head's largest element (the f32 rounding of the projection and norm
    # scales with the row, so an element far below the row maximum can move
    # by several of its own ulps). Layer 0's inputs equal the oracle's, so
    # few elements differ at all; later layers take a hidden state that has
    # been through f32 sums in another order, and more elements round to the
    # neighbouring f16 value. With MoE layers that order difference reaches
    # 1e-5 .. 1e-4 of the hidden state's scale (measured, with the same size
    # for either attention kernel: the experts' SwiGLU amplifies it), so past
    # layer 0 the bound is the decode tolerance, 1e-3 of the head's largest
    # element. The share of elements that differ at all is a sanity check
    # (at most 5% at layer 0, half past it: 30% measured on the K = 12288
    # down projection's model, every one within 0.4 of its bound).
    hd = cfg["head_dim"]
    for l in range(cfg["n_layers"]):
        for which in (0, 1):
            g = eng.read_kv(l, which, prefill, 1).view(np.float16)
            o = om.kv(l, which, prefill).view(np.float16)
            assert np.isfinite(g).all()
            g32, o32 = g.astype(np.float32), o.astype(np.float32)
            rowmax = np.repeat(np.abs(o32).reshape(-1, hd).max(axis=1), hd)
            bound = np.spacing(np.abs(o)).astype(np.float32) + (1e-5 if l == 0 else 1e-3) * rowmax
            d = np.abs(g32 - o32)
            frac = 0.05 if l == 0 else 0.5
            assert (d <= bound).all() and (d > 0).mean() < frac, (l, which, (d / bound).max(), (d > 0).mean())
    eng.deinit()
    om.close()


@pytest.mark.parametrize("cfg", [SMALL_DENSE, SMALL_MOE, MOE_C4, DENSE_RING], ids=["dense", "moe", "moe_c4", "ring"])
def test_engine_generate_token_exact(ctx, orc, cfg):
    import zinc_amd
    eng = zinc_amd.InferenceEngine(ctx, cfg)
    om = orc.Model(cfg)
    prefill, n_gen = 64, 24
    eng.prefill_kv_random(prefill, 5)
    om.prefill_kv_random(prefill, 5)
    prompt = [int(t) for t in np.random.default_rng(3).integers(0, cfg["vocab"], 6)]
    got = eng.generate(prompt, n_gen, start_pos=prefill)
    # oracle: per-token decodeStep over the prompt, then greedy
    pos = prefill
    margins = []
    for t in prompt[:-1]:
        om.decode_step(t, pos)
        pos += 1
    ref = []
    tok = prompt[-1]
    for _ in range(n_gen):
        tok, lg = om.decode_step(tok, pos, want_logits=True)
        margins.append(margin(lg))
        pos += 1
        ref.append(int(tok))
    assert got == ref, f"first mismatch at {next(i for i in range(n_gen) if got[i] != ref[i])}; margins {margins}"
    eng.deinit()
    om.close()


def test_engine_context_overflow_is_an_error(ctx):
    import zinc_amd
    eng = zinc_amd.InferenceEngine(ctx, SMALL_DENSE)
    with pytest.raises(zinc_amd.ZincError) as e:
        eng.generate([1, 2], 10, start_pos=SMALL_DENSE["max_ctx"] - 5)
    assert e.value.name == "ContextLengthExceeded"
    st = zinc_amd.DecodeState()
    st.position = SMALL_DENSE["max_ctx"]
    with pytest.raises(zinc_amd.ZincError):
        eng.decode_step(st, 1)
    eng.deinit()


# 16 kv heads put 256 / 16 = 16 chunks per kv head on the device, so a
# context above 2 x 16 x 160 = 5120 tokens makes every attention chunk hold
# several 160-token sub-chunks reduced with an online softmax (here 3 at
# 12000 tokens); the new token's K/V write and substitution then happen in a
# later sub-chunk than the first.
LONG_SUBCHUNK = dict(n_layers=1, hidden=1024, n_heads=16, n_kv_heads=16, head_dim=128, ffn=1024, vocab=1000,
                     n_experts=0, n_experts_used=0, expert_ffn=0, max_ctx=12048,
                     type_attn=12, type_ffn_gate_up=12, type_ffn_down=14, type_lm_head=14, type_embd=12,
                     type_router=8, rope_base=1e6, eps=1e-6, seed=96)


@pytest.mark.parametrize("prefill", [12000, 10001], ids=["12000", "10001"])
def test_engine_long_context_subchunks(ctx, orc, prefill):
    import zinc_amd
    cfg = LONG_SUBCHUNK
    eng = zinc_amd.InferenceEngine(ctx, cfg)
    om = orc.Model(cfg)
    eng.prefill_kv_random(prefill, 11)
    om.prefill_kv_random(prefill, 11)
    state = zinc_amd.DecodeState()
    tok = 5
    for step in range(3):
        state.position = prefill + step
        eng.decode_step(state, tok, True)
        g_tok, g_log = eng.sample_greedy(), eng.logits()
        o_tok, o_log = om.decode_step(tok, prefill + step, want_logits=True)
        scale = np.abs(o_log).max()
        assert np.abs(g_log - o_log).max() <= 1e-4 + 1e-3 * scale, (step, np.abs(g_log - o_log).max(), scale)
        if margin(o_log) > 1e-3 * scale:
            assert g_tok == o_tok
        for which in (0, 1):
            g = eng.read_kv(0, which, prefill + step, 1).view(np.float16).astype(np.float32)
            o = om.kv(0, which, prefill + step).view(np.float16).astype(np.float32)
            assert np.abs(g - o).max() <= 2e-3 * np.abs(o).max(), (step, which)
        tok = int(o_tok)
    eng.deinit()
    om.close()


# Paged KV cache: the engine's page table comes from a page pool
# (KvPagePool, kv_cache.zig:43-125: a fresh pool hands out pages in
# descending order) or is an arbitrary permutation; the decode kernel then
# looks every 16-token page up (logicalTokenToPhysicalToken,
# forward.zig:677-698). Greedy tokens must equal the oracle's (which has no
# paging), and the rows read back through the table must equal the oracle's.
def _pages(cfg, order):
    import zinc_amd
    n = cfg["max_ctx"] // 16
    if order == "pool":
        pool = zinc_amd.KvPagePool(n, 16)
        pages = pool.alloc_pages(7, n)
        assert pages.tolist() == list(range(n - 1, -1, -1)) and pool.free_count() == 0
        return pages
    return np.random.default_rng(17).permutation(n).astype(np.uint32)


@pytest.mark.parametrize("cfg,order", [(SMALL_DENSE, "pool"), (SMALL_DENSE, "shuffle"), (SMALL_MOE, "shuffle"),
                                       (MOE_C4, "pool")], ids=["dense-pool", "dense-shuffle", "moe-shuffle", "moe_c4-pool"])
def test_engine_paged_generate_token_exact(ctx, orc, cfg, order):
    import zinc_amd
    print(f"paged engine {order} heads {cfg['n_heads']}/{cfg['n_kv_heads']}", flush=True)
    eng = zinc_amd.InferenceEngine(ctx, cfg)
    eng.set_pages(_pages(cfg, order))
    om = orc.Model(cfg)
    prefill, n_gen = 64, 24
    eng.prefill_kv_random(prefill, 5)
    om.prefill_kv_random(prefill, 5)
    for which in (0, 1):  # the prefilled rows through the table
        assert np.array_equal(eng.read_kv(0, which, 0, prefill), np.concatenate([om.kv(0, which, t) for t in range(prefill)]))
    prompt = [int(t) for t in np.random.default_rng(3).integers(0, cfg["vocab"], 6)]
    got = eng.generate(prompt, n_gen, start_pos=prefill)
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
    # the rows the decode wrote, read back through the table
    for t in (prefill, prefill + 10, pos - 1):
        for which in (0, 1):
            g = eng.read_kv(1, which, t, 1).view(np.float16).astype(np.float32)
            o = om.kv(1, which, t).view(np.float16).astype(np.float32)
            assert np.abs(g - o).max() <= 2e-3 * np.abs(o).max() + 1e-3, (t, which)
    eng.deinit()
    om.close()


def test_engine_paged_long_context(ctx, orc):
    """12000 tokens over a shuffled table: every chunk streams several
    sub-chunks, each looked up page by page."""
    import zinc_amd
    cfg = LONG_SUBCHUNK
    eng = zinc_amd.InferenceEngine(ctx, cfg)
    eng.set_pages(_pages(cfg, "shuffle"))
    om = orc.Model(cfg)
    prefill = 12000
    eng.prefill_kv_random(prefill, 11)
    om.prefill_kv_random(prefill, 11)
    state = zinc_amd.DecodeState()
    tok = 5
    for step in range(2):
        state.position = prefill + step
        eng.decode_step(state, tok, True)
        g_tok, g_log = eng.sample_greedy(), eng.logits()
        o_tok, o_log = om.decode_step(tok, prefill + step, want_logits=True)
        scale = np.abs(o_log).max()
        assert np.abs(g_log - o_log).max() <= 1e-4 + 1e-3 * scale, (step, np.abs(g_log - o_log).max(), scale)
        if margin(o_log) > 1e-3 * scale:
            assert g_tok == o_tok
        tok = int(o_tok)
    eng.deinit()
    om.close()


def test_engine_set_pages_rejects_bad_tables(ctx):
    import zinc_amd
    eng = zinc_amd.InferenceEngine(ctx, SMALL_DENSE)
    n = SMALL_DENSE["max_ctx"] // 16
    for bad in (np.arange(n - 1, dtype=np.uint32), np.full(n, n, dtype=np.uint32)):
        with pytest.raises(zinc_amd.ZincError) as e:
            eng.set_pages(bad)
        assert e.value.name == "InvalidArgument"
    eng.deinit()


# The in-kernel merge of the decode attention: with at least G chunks per kv
# head the last G arrivals merge one q head each, and the first G-1 of them
# wait (bounded) for the rest. A zero limit makes those mergers give up at
# once: their q heads come out NaN, every kernel completes, zh_sync reports
# WaitTimeout, and the next step with the default limit is correct again (the
# merge counters are consistent after a give-up). One layer, so the poisoned
# step's K/V row (a function of the embedding alone) stays the oracle's.
WAIT_CFG = dict(n_layers=1, hidden=1024, n_heads=16, n_kv_heads=4, head_dim=128, ffn=1024, vocab=1000,
                n_experts=0, n_experts_used=0, expert_ffn=0, max_ctx=2048,
                type_attn=12, type_ffn_gate_up=12, type_ffn_down=14, type_lm_head=14, type_embd=12,
                type_router=8, rope_base=1e6, eps=1e-6, seed=95)


def test_attention_merge_wait_give_up(orc):
    import zinc_amd
    c = zinc_amd.Context(0)
    try:
        cfg = WAIT_CFG
        eng = zinc_amd.InferenceEngine(c, cfg)
        om = orc.Model(cfg)
        prefill = 1500
        eng.prefill_kv_random(prefill, 13)
        om.prefill_kv_random(prefill, 13)
        st = zinc_amd.DecodeState()
        c.set_attn_wait_limit(0)
        st.position = prefill
        eng.decode_step(st, 7, True)
        # the poisoned heads reach the residual stream through the O
        # projection (the later activation quantisers map NaN to 0)
        assert np.isnan(eng.hidden()).any()
        with pytest.raises(zinc_amd.ZincError) as e:
            c.sync()
        assert e.value.name == "WaitTimeout"
        c.sync()  # the error word was cleared
        c.set_attn_wait_limit(50000)
        om.decode_step(7, prefill)
        for step in range(1, 3):
            st.position = prefill + step
            eng.decode_step(st, 9 + step, True)
            eng.sample_greedy()
            g_log = eng.logits()
            o_tok, o_log = om.decode_step(9 + step, prefill + step, want_logits=True)
            scale = np.abs(o_log).max()
            assert np.abs(g_log - o_log).max() <= 1e-4 + 1e-3 * scale, step
        c.sync()
        eng.deinit()
        om.close()
    finally:
        c.close()


# The persistent decode-layers kernel (zh_engine_set_persistent): every
# layer's phases in one launch, grid barriers between them. Same bar as the
# per-phase kernels: the step's logits against the oracle's, greedy tokens
# equal over a generation, on the identity and on a shuffled page table, at
# a context long enough for several sub-chunks per attention chunk.
@pytest.mark.parametrize("order,prefill", [("ident", 100), ("shuffle", 100), ("ident", 400)],
                         ids=["ident", "shuffle", "ident-400"])
def test_engine_persistent_matches_oracle(ctx, orc, order, prefill):
    import zinc_amd
    cfg = dict(DENSE_RING, max_ctx=512)
    eng = zinc_amd.InferenceEngine(ctx, cfg)
    eng.set_persistent(True)
    if order == "shuffle":
        eng.set_pages(_pages(cfg, "shuffle"))
    om = orc.Model(cfg)
    eng.prefill_kv_random(prefill, 7)
    om.prefill_kv_random(prefill, 7)
    st = zinc_amd.DecodeState()
    st.position = prefill
    eng.decode_step(st, 17, True)
    g_tok, g_log = eng.sample_greedy(), eng.logits()
    o_tok, o_log = om.decode_step(17, prefill, want_logits=True)
    assert np.allclose(g_log, o_log, rtol=1e-3, atol=1e-4 + 1e-3 * np.abs(o_log).max()), \
        f"max |d| {np.abs(g_log - o_log).max()} vs scale {np.abs(o_log).max()}"
    assert g_tok == o_tok
    prompt = [int(t) for t in np.random.default_rng(3).integers(0, cfg["vocab"], 6)]
    got = eng.generate(prompt, 16, start_pos=prefill + 1)
    pos = prefill + 1
    for t in prompt[:-1]:
        om.decode_step(t, pos)
        pos += 1
    ref, tok = [], prompt[-1]
    for _ in range(16):
        tok = om.decode_step(tok, pos)
        pos += 1
        ref.append(int(tok))
    assert got == ref, f"first mismatch at {next(i for i in range(16) if got[i] != ref[i])}"
    ctx.sync()  # no barrier gave up
    eng.deinit()
    om.close()
