"""Batched prefill kernels on the GPU vs the CPU oracle.

The dequant-GEMM (dispatchProjectionBatched / mul_mm_q4k.comp) runs on fp16
operands with f32 accumulation: the weights are the oracle's dequantRow values
rounded to fp16 (round to nearest even), X is fp16. Its reference is the f64
product of exactly those fp16 operands, so the only admissible difference is
f32 accumulation rounding: |y - ref| <= 1e-5 * sum|x w| + 1e-6."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    import zinc_amd
    c = zinc_amd.Context(0)
    yield c
    c.close()


def dequant_f16(orc, raw, qtype, M, K):
    return np.stack([orc.dequant_row(raw, r, K, qtype) for r in range(M)]).astype(np.float16)


@pytest.mark.parametrize("qtype", [12, 14])
def test_gemm_one_hot_gives_the_fp16_weights_exactly(ctx, orc, qtype):
    """X = identity (N = K tokens): Y[n][m] = W16[m][n], a single exact product."""
    M, K = 128, 512
    raw = orc.synth_tensor(qtype, M, K, 31, 7)
    W = ctx.upload(raw)
    X = ctx.upload(np.eye(K, dtype=np.float16))
    Y = ctx.alloc(4 * M * K)
    ctx.gemm_xw(qtype, W, 0, X, 0, Y, 0, M, K, K)
    y = Y.download(np.float32, (K, M))
    assert np.array_equal(y, dequant_f16(orc, raw, qtype, M, K).astype(np.float32).T)
    for b in (W, X, Y):
        ctx.free(b)


def test_gemm_rounds_the_f32_dequant_value_to_fp16(ctx):
    """The weight operand is dequantRow's f32 value rounded to fp16, not the
    exact value rounded once: on the block of test_oracle.py's
    test_dequant_q4k_f32_tie_block (f32 value 2051/2048, an fp16 tie) every
    weight is 1 + 2^-9; a conversion fused into the multiply-add gives
    1 + 2^-10."""
    M, K = 128, 256
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([293 / 2048], np.float16).view(np.uint8)
    blk[2:4] = np.array([1], np.uint16).view(np.uint8)  # dmin = 2^-24
    blk[4:16] = [1] * 8 + [0x11] * 4                     # every sc and m = 1
    blk[16:] = 0x77                                      # every q = 7
    W = ctx.upload(np.tile(blk, M))
    X = ctx.upload(np.eye(K, dtype=np.float16))
    Y = ctx.alloc(4 * M * K)
    ctx.gemm_xw(12, W, 0, X, 0, Y, 0, M, K, K)
    y = Y.download(np.float32, (K, M))
    assert np.all(y == np.float32(1 + 2 ** -9)), np.unique(y)
    for b in (W, X, Y):
        ctx.free(b)


@pytest.mark.parametrize("qtype,M,K,N", [
    (12, 256, 512, 37), (12, 1024, 4096, 512), (12, 4096, 4096, 128), (12, 6144, 4096, 300),
    (14, 256, 512, 64), (14, 4096, 12288, 130), (14, 384, 1024, 1),
])
def test_gemm_matches_fp16_operand_reference(ctx, orc, qtype, M, K, N):
    raw = orc.synth_tensor(qtype, M, K, 1000 + M, N)
    w16 = dequant_f16(orc, raw, qtype, M, K).astype(np.float64)
    rng = np.random.default_rng(M * 7 + N)
    x16 = rng.standard_normal((N, K)).astype(np.float16)
    ref = x16.astype(np.float64) @ w16.T
    mag = np.abs(x16.astype(np.float64)) @ np.abs(w16).T
    W, X, Y = ctx.upload(raw), ctx.upload(x16), ctx.alloc(4 * M * N)
    ctx.gemm_xw(qtype, W, 0, X, 0, Y, 0, M, K, N)
    y = Y.download(np.float32, (N, M)).astype(np.float64)
    err = np.abs(y - ref) - (1e-5 * mag + 1e-6)
    assert err.max() <= 0, f"worst excess {err.max()} at {np.unravel_index(err.argmax(), err.shape)}"
    for b in (W, X, Y):
        ctx.free(b)


def test_gemm_accumulates_and_rejects_bad_shapes(ctx, orc):
    import zinc_amd
    M, K, N = 256, 256, 40
    raw = orc.synth_tensor(12, M, K, 5, 5)
    w16 = dequant_f16(orc, raw, 12, M, K).astype(np.float64)
    x16 = np.random.default_rng(3).standard_normal((N, K)).astype(np.float16)
    y0 = np.random.default_rng(4).standard_normal((N, M)).astype(np.float32)
    W, X, Y = ctx.upload(raw), ctx.upload(x16), ctx.upload(y0)
    ctx.gemm_xw(12, W, 0, X, 0, Y, 0, M, K, N, 1)
    y = Y.download(np.float32, (N, M)).astype(np.float64)
    ref = y0 + x16.astype(np.float64) @ w16.T
    mag = np.abs(y0) + np.abs(x16.astype(np.float64)) @ np.abs(w16).T
    assert (np.abs(y - ref) <= 1e-5 * mag + 1e-6).all()
    with pytest.raises(zinc_amd.ZincError):
        ctx.gemm_xw(12, W, 0, X, 0, Y, 0, M, 300, N)      # K not a multiple of 256
    with pytest.raises(zinc_amd.ZincError):
        ctx.gemm_xw(8, W, 0, X, 0, Y, 0, M, K, N)         # Q8_0 has no GEMM path
    with pytest.raises(zinc_amd.ZincError):
        ctx.gemm_xw(12, W, 0, X, 0, Y, 0, M, K, N + 1000)  # X range
    for b in (W, X, Y):
        ctx.free(b)


SMALL_DENSE = dict(n_layers=3, hidden=512, n_heads=4, n_kv_heads=2, head_dim=128, ffn=1536, vocab=3000,
                   n_experts=0, n_experts_used=0, expert_ffn=0, max_ctx=1104,
                   type_attn=12, type_ffn_gate_up=12, type_ffn_down=14, type_lm_head=14, type_embd=12,
                   type_router=8, rope_base=1e6, eps=1e-6, seed=99)


@pytest.mark.parametrize("n_prompt,prefill", [(40, 64), (5, 64), (600, 0)], ids=["40at64", "5at64", "600at0-2chunks"])
def test_engine_prefill_matches_sequential_oracle(ctx, orc, n_prompt, prefill):
    """prefillBatched vs the oracle's token-by-token decodeStep: the K/V rows
    of every prompt token and the last token's logits. The GEMM operands are
    fp16 (relative rounding 2^-11), so the bounds are relative to each row's
    magnitude: K/V |d| <= 5e-3 * max|row|, logits |d| <= 3e-3 * max|logit|
    (measured: about 1.4e-3 of each at the 8B layer shapes,
    test_gpu_golden.py); the greedy token must agree wherever the oracle's
    top-2 margin exceeds twice the logit bound (6e-3 of the scale)."""
    import zinc_amd
    eng = zinc_amd.InferenceEngine(ctx, SMALL_DENSE)
    om = orc.Model(SMALL_DENSE)
    if prefill:
        eng.prefill_kv_random(prefill, 5)
        om.prefill_kv_random(prefill, 5)
    prompt = [int(t) for t in np.random.default_rng(n_prompt).integers(0, SMALL_DENSE["vocab"], n_prompt)]
    eng.prefill(prompt, start_pos=prefill)
    g_tok, g_log = eng.sample_greedy(), eng.logits()
    for i, t in enumerate(prompt):
        o_tok, o_log = om.decode_step(t, prefill + i, want_logits=True)
    scale = np.abs(o_log).max()
    assert np.abs(g_log - o_log).max() <= 3e-3 * scale, np.abs(g_log - o_log).max() / scale
    s = np.sort(o_log)
    if (s[-1] - s[-2]) > 6e-3 * scale:
        assert g_tok == o_tok
    for l in range(SMALL_DENSE["n_layers"]):
        for which in (0, 1):
            g = eng.read_kv(l, which, prefill, n_prompt).view(np.float16).astype(np.float32).reshape(n_prompt, -1)
            o = np.stack([om.kv(l, which, prefill + i) for i in range(n_prompt)]).view(np.float16)
            o = o.astype(np.float32)
            rowmax = np.abs(o).max(axis=1, keepdims=True)
            assert (np.abs(g - o) <= 5e-3 * rowmax).all(), (l, which, (np.abs(g - o) / rowmax).max())
    eng.deinit()
    om.close()


def test_engine_prefill_then_decode_continues(ctx, orc):
    """After a batched prefill the decode loop continues from the prefilled
    KV: greedy tokens match the oracle's sequential run where margins are
    clear (1% of the logit scale)."""
    import zinc_amd
    eng = zinc_amd.InferenceEngine(ctx, SMALL_DENSE)
    om = orc.Model(SMALL_DENSE)
    prompt = [int(t) for t in np.random.default_rng(77).integers(0, SMALL_DENSE["vocab"], 24)]
    eng.prefill(prompt, start_pos=0)
    tok = eng.sample_greedy()
    for i, t in enumerate(prompt):
        o_tok, o_log = om.decode_step(t, i, want_logits=True)
    got, ref = [tok], [o_tok]
    pos = len(prompt)
    st = zinc_amd.DecodeState()
    for _ in range(8):
        st.position = pos
        eng.decode_step(st, got[-1], True)
        got.append(eng.sample_greedy())
        o_tok, o_log = om.decode_step(ref[-1], pos, want_logits=True)
        ref.append(o_tok)
        s = np.sort(o_log)
        if (s[-1] - s[-2]) <= 1e-2 * np.abs(o_log).max() or got[-1] != ref[-1]:
            break
        pos += 1
    assert got == ref, (got, ref)
    eng.deinit()
    om.close()


def _causal_ref(q, k16, v16, pages, nh, nkv, seq_start, scale):
    """f64 causal attention over the paged fp16 cache (cpuAttention per query,
    forward_metal.zig:6600-6646, at positions seq_start + i)."""
    n = q.shape[0]
    hd = 128
    out = np.zeros((n, nh * hd))
    for i in range(n):
        L = seq_start + i + 1
        phys = np.array([pages[t // 16] * 16 + t % 16 for t in range(L)])
        for h in range(nh):
            kvh = h // (nh // nkv)
            K = k16[kvh, phys].astype(np.float64)
            V = v16[kvh, phys].astype(np.float64)
            s = K @ q[i, h * hd:(h + 1) * hd].astype(np.float64) * scale
            p = np.exp(s - s.max())
            out[i, h * hd:(h + 1) * hd] = p @ V / p.sum()
    return out


@pytest.mark.parametrize("nh,nkv,seq_start,n", [(32, 8, 0, 200), (8, 8, 700, 70), (4, 1, 40, 130)],
                         ids=["gqa4-200at0", "mha-70at700", "gqa4-130at40"])
def test_flash_attn_batched_matches_reference(ctx, nh, nkv, seq_start, n):
    """Causal batched attention vs an f64 reference on a permuted page table.
    Operands are fp16 (q and P rounded, relative 2^-11), the output fp16:
    |d| <= 4e-3 * max|row of the reference| + 1e-3."""
    rng = np.random.default_rng(nh * 1000 + seq_start + n)
    cache_tokens = 1024
    n_pages = cache_tokens // 16
    pages = rng.permutation(n_pages).astype(np.uint32)
    k16 = rng.standard_normal((nkv, cache_tokens, 128)).astype(np.float16)
    v16 = rng.standard_normal((nkv, cache_tokens, 128)).astype(np.float16)
    q = rng.standard_normal((n, nh * 128)).astype(np.float32)
    out = ctx.alloc(2 * n * nh * 128)
    ctx.flash_attn_batched(ctx.upload(q), ctx.upload(k16), ctx.upload(v16), ctx.upload(pages), n_pages, cache_tokens,
                           out, nh, nkv, 128, seq_start, n)
    ctx.sync()
    got = out.download(np.float16, n * nh * 128).astype(np.float64).reshape(n, -1)
    ref = _causal_ref(q, k16, v16, pages, nh, nkv, seq_start, 1 / np.sqrt(128))
    bound = 4e-3 * np.abs(ref).reshape(n, nh, 128).max(axis=2).repeat(128, axis=1) + 1e-3
    err = np.abs(got - ref)
    assert (err <= bound).all(), (err.max(), np.unravel_index(err.argmax(), err.shape))
