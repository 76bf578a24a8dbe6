"""GPU parity of each HIP kernel family against the CPU oracle, through the C ABI.

Tolerances (north star): dequantised values bit-exact; DMMV and attention
outputs within 1e-3 relative / 1e-4 absolute of the oracle's f32 result
(|gpu - ref| <= 1e-4 + 1e-3 * |ref|).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 1e-4


@pytest.fixture(scope="module")
def ctx():
    import zinc_amd
    c = zinc_amd.Context(0)
    yield c
    c.close()


def close_enough(got, ref, rtol=RTOL, atol=ATOL):
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    bound = atol + rtol * np.abs(ref.astype(np.float64))
    bad = np.nonzero(err > bound)[0]
    return bad, err


def assert_close(got, ref, what, rtol=RTOL, atol=ATOL):
    bad, err = close_enough(got, ref, rtol, atol)
    assert len(bad) == 0, (f"{what}: {len(bad)}/{len(ref)} outside tol; worst idx {bad[:5]} "
                           f"got {got[bad[:5]]} ref {ref[bad[:5]]}; max err {err.max():.3g}")


# Floor for ill-conditioned (cancelling) dot products: f32 rounding in any
# summation order scales with sum_i |w_i x_i|. The kernels' own error against
# the exact (f64) value is held to 2^-21 of that magnitude (about 4 unit
# roundoffs of the largest partial sum); against the oracle's serial f32
# result the oracle's own measured error |ref32 - ref64| is added, since
# that is the reference rounding, not the kernel's.
NOISE = 2.0 ** -21


def assert_dot_close(got, ref32, ref64, mag, what):
    """Parity bar for DMMV-like outputs: every row within the north-star
    tolerance, |gpu - ref| <= 1e-4 + 1e-3*|ref|, of both the f64 value and
    the oracle's f32 serial dot (the reference's CPU path), widened only by
    the f32 rounding floor above. The floor matters only for cancelling rows
    (|y| << sum|w x|), where any two f32 summation orders -- including the
    reference's own serial loop versus the exact value -- already differ by
    more than 1e-4 + 1e-3*|y|."""
    got = got.astype(np.float64)
    own = np.abs(ref32 - ref64)
    ok64 = np.abs(got - ref64) <= ATOL + RTOL * np.abs(ref64) + NOISE * mag
    ok32 = np.abs(got - ref32) <= ATOL + RTOL * np.abs(ref32) + NOISE * mag + own
    bad = np.nonzero(~(ok32 & ok64))[0]
    worst = float(np.max(np.abs(got - ref64) / np.maximum(mag, 1e-30)))
    assert len(bad) == 0, (f"{what}: {len(bad)}/{len(got)} rows outside tol; idx {bad[:5]} got {got[bad[:5]]} "
                           f"ref32 {ref32[bad[:5]]} ref64 {ref64[bad[:5]]} mag {mag[bad[:5]]}; "
                           f"max |got-ref64|/mag {worst:.3g}")
    return int((~ok32).sum())


QTYPES = [12, 13, 14, 8, 39]


@pytest.mark.parametrize("qtype", QTYPES + [12 | 0x100, 13 | 0x100])
def test_synth_generator_bit_identical(ctx, orc, qtype):
    rows, cols = 7, (2880 if qtype == 39 else 1024)
    n = orc.tensor_bytes(qtype & 0xFF, rows, cols)
    buf = ctx.alloc(n)
    ctx.synth_tensor(buf, 0, qtype, rows, cols, 77, 5)
    got = buf.download(np.uint8, n)
    assert np.array_equal(got, orc.synth_tensor(qtype, rows, cols, 77, 5))
    ctx.free(buf)


def test_synth_vectors_bit_identical(ctx, orc):
    n = 5000
    b = ctx.alloc(n * 4)
    ctx.synth_vector(b, 0, 0, n, 1.0, 3, 9)
    assert np.array_equal(b.download(np.float32, n), orc.synth_normal_f32(n, 3, 9))
    ctx.synth_vector(b, 0, 1, n, 1.0, 3, 9)
    assert np.array_equal(b.download(np.uint16, n), orc.synth_normal_f16(n, 3, 9))
    ctx.synth_vector(b, 0, 2, n, 1.0, 3, 9)
    assert np.array_equal(b.download(np.float32, n), orc.synth_norm_weight(n, 3, 9))
    ctx.free(b)


@pytest.mark.parametrize("qtype", QTYPES + [1, 0])
def test_dequant_bit_exact(ctx, orc, qtype):
    rows, cols = 5, (2880 if qtype == 39 else 1024)
    W = orc.synth_tensor(qtype, rows, cols, 11, 3)
    Wb = ctx.upload(W)
    out = ctx.alloc(rows * cols * 4)
    ctx.dequant_rows(qtype, Wb, 0, 0, rows, cols, out)
    got = out.download(np.float32, rows * cols).reshape(rows, cols)
    ref = orc.dequant(W, rows, cols, qtype)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    ctx.free(Wb)
    ctx.free(out)


def run_dmmv(ctx, orc, qtype, M, K, seed, acc=False, a_off=0):
    W = orc.synth_tensor(qtype, M, K, seed, 1)
    x = orc.synth_normal_f32(K, seed, 2)
    Wb = ctx.alloc(a_off + len(W))
    Wb.upload(W, a_off)
    xb = ctx.upload(x)
    y0 = orc.synth_normal_f32(M, seed, 3) if acc else np.zeros(M, np.float32)
    yb = ctx.upload(y0)
    ctx.dmmv(qtype, Wb, a_off, xb, 0, yb, 0, M, K, int(acc))
    got = yb.download(np.float32, M)
    ref = orc.dmmv(W, qtype, x, M, K, y=y0.copy(), acc_mode=int(acc))
    ref64 = orc.dmmv_f64(W, qtype, x, M, K) + (y0.astype(np.float64) if acc else 0.0)
    mag = orc.dmmv_absdot(W, qtype, x, M, K) + (np.abs(y0.astype(np.float64)) if acc else 0.0)
    for b in (Wb, xb, yb):
        ctx.free(b)
    return got, ref, ref64, mag


@pytest.mark.parametrize("qtype,M,K", [
    (12, 4096, 4096),     # config 1
    (12, 256, 512), (12, 1000, 768), (12, 12288, 4096), (14, 2000, 4096), (14, 4096, 12288),
    (12, 257, 512), (12, 33, 768), (12, 100, 2048), (12, 64, 12288),
    (14, 257, 512), (14, 512, 4096), (14, 64, 12288), (14, 40, 768),
    (8, 257, 4096), (8, 128, 2048), (8, 16, 768),
    (8, 257, 96), (8, 100, 2080), (8, 33, 32),  # Q8_0 rows of an odd block count (K = 32 * odd)
    (13, 4096, 4096), (13, 257, 512), (13, 1000, 768), (13, 64, 12288), (13, 1536, 2048),
    (39, 257, 2880), (39, 4, 32), (39, 100, 1024),
])
def test_dmmv_matches_oracle(ctx, orc, qtype, M, K):
    got, ref, ref64, mag = run_dmmv(ctx, orc, qtype, M, K, 1000 + M + K)
    assert_dot_close(got, ref, ref64, mag, f"dmmv q{qtype} {M}x{K}")


@pytest.mark.parametrize("qtype,M,K", [
    (12, 4096, 4096), (12, 12288, 4096), (12, 257, 512), (12, 64, 12288),
    (14, 4096, 12288), (14, 64, 12288), (14, 2000, 4096), (14, 4096, 6144), (14, 40, 768),
    (8, 257, 4096), (8, 101, 1056), (13, 4096, 4096), (13, 64, 12288),
])
def test_dmmv_xq_matches_oracle(ctx, orc, qtype, M, K):
    """The activation pre-quantised once (zh_quantize_activation: three int8
    limbs under a power-of-two block scale, 24 significant bits) and read by
    zh_dmmv_xq meets the same bar as the f32 entry point. K = 12288 stages
    384 block scales and 768 block sums, more than one per lane of a workgroup."""
    W = orc.synth_tensor(qtype, M, K, 77 + M, 1)
    x = orc.synth_normal_f32(K, 77 + K, 2)
    Wb, xb, yb = ctx.upload(W), ctx.upload(x), ctx.alloc(4 * M)
    xq = ctx.alloc(ctx.xq_bytes(K))
    ctx.quantize_activation(xb, 0, K, xq, 0)
    ctx.dmmv_xq(qtype, Wb, 0, xq, 0, yb, 0, M, K)
    got = yb.download(np.float32, M)
    assert_dot_close(got, orc.dmmv(W, qtype, x, M, K), orc.dmmv_f64(W, qtype, x, M, K),
                     orc.dmmv_absdot(W, qtype, x, M, K), f"dmmv_xq q{qtype} {M}x{K}")
    for b in (Wb, xb, yb, xq):
        ctx.free(b)


@pytest.mark.parametrize("qtype", [12, 13, 14, 8])
def test_dmmv_acc_mode_and_offset(ctx, orc, qtype):
    got, ref, ref64, mag = run_dmmv(ctx, orc, qtype, 300, 1024, 5, acc=True, a_off=4096)
    assert_dot_close(got, ref, ref64, mag, "acc")


def test_dmmv_mxfp4_reference_kat(ctx):
    # forward_metal.zig:14238-14303: e=127, every code byte 0x42, x=1 -> 48
    W = np.zeros(4 * 17, np.uint8)
    for r in range(4):
        W[r * 17] = 127
        W[r * 17 + 1:r * 17 + 17] = 0x42
    Wb, xb, yb = ctx.upload(W), ctx.upload(np.ones(32, np.float32)), ctx.alloc(16)
    ctx.dmmv(39, Wb, 0, xb, 0, yb, 0, 4, 32)
    assert np.all(np.abs(yb.download(np.float32, 4) - 48.0) < 0.01)


def test_dmmv_rejects_bad_shapes(ctx):
    import zinc_amd
    W, x, y = ctx.alloc(1 << 16), ctx.alloc(4096), ctx.alloc(4096)
    with pytest.raises(zinc_amd.ZincError) as e:
        ctx.dmmv(12, W, 0, x, 0, y, 0, 4, 300)  # K % 256
    assert e.value.name == "InvalidArgument"
    with pytest.raises(zinc_amd.ZincError) as e:
        ctx.dmmv(2, W, 0, x, 0, y, 0, 4, 256)  # Q4_0: no kernel
    assert e.value.name == "UnsupportedQuantType"
    with pytest.raises(zinc_amd.ZincError) as e:
        ctx.dmmv(12, W, 0, x, 0, y, 0, 1000, 256)  # W too small
    assert e.value.name == "InvalidArgument"


@pytest.mark.parametrize("qtype,M,K", [(12, 1024, 4096), (12, 768, 2048), (14, 200, 1024), (13, 768, 2048)])
def test_fused_gate_up_swiglu(ctx, orc, qtype, M, K):
    Wg = orc.synth_tensor(qtype, M, K, 21, 1)
    Wu = orc.synth_tensor(qtype, M, K, 21, 2)
    x = orc.synth_normal_f32(K, 21, 3)
    g = orc.dmmv(Wg, qtype, x, M, K)
    u = orc.dmmv(Wu, qtype, x, M, K)
    ref = orc.swiglu(g, u)
    g64, u64 = orc.dmmv_f64(Wg, qtype, x, M, K), orc.dmmv_f64(Wu, qtype, x, M, K)
    sig = 1 / (1 + np.exp(-g64))
    ref64 = g64 * sig * u64
    # first-order propagation of the two dot products' magnitudes through silu(g)*u
    dsilu = np.abs(sig * (1 + g64 * (1 - sig)))
    mag = dsilu * orc.dmmv_absdot(Wg, qtype, x, M, K) * np.abs(u64) + np.abs(g64 * sig) * orc.dmmv_absdot(Wu, qtype, x, M, K)
    bg, bu, bx, by = ctx.upload(Wg), ctx.upload(Wu), ctx.upload(x), ctx.alloc(M * 4)
    ctx.dmmv_fused_gate_up_swiglu(qtype, bg, 0, bu, 0, bx, 0, by, 0, M, K)
    got = by.download(np.float32, M)
    assert_dot_close(got, ref, ref64, mag, "gate_up")


@pytest.mark.parametrize("qt", [12, 13])
def test_dmmv_moe_expert_gather(ctx, orc, qt):
    E, M, K, k = 16, 768, 2048, 4
    W = orc.synth_tensor(qt, E * M, K, 31, 1)
    stride = orc.tensor_bytes(qt, M, K)
    ids = np.array([3, 15, 0, 7], np.uint32)
    xs = orc.synth_normal_f32(k * K, 31, 2)
    routing = np.concatenate([ids, np.full(k, 0.25, np.float32).view(np.uint32)])
    bW, br, bx, by = ctx.upload(W), ctx.upload(routing), ctx.upload(xs), ctx.alloc(k * M * 4)
    ctx.dmmv_moe(qt, bW, stride, br, bx, K, 0, by, 0, M, K, k)
    got = by.download(np.float32, k * M).reshape(k, M)
    for s in range(k):
        We, xe = W[ids[s] * stride:(ids[s] + 1) * stride], xs[s * K:(s + 1) * K]
        assert_dot_close(got[s], orc.dmmv(We, qt, xe, M, K), orc.dmmv_f64(We, qt, xe, M, K),
                         orc.dmmv_absdot(We, qt, xe, M, K), f"moe slot {s}")


def test_dmmv_moe_clamps_bad_expert_id_and_sync_reports_it(ctx, orc):
    """zh_dmmv_moe reads the routing ids on the device only: an id past the
    experts the weights hold is clamped to the last expert (the launch
    completes), and the next zh_sync returns InvalidArgument once."""
    import zinc_amd
    qt, E, M, K, k = 12, 4, 256, 512, 2
    W = orc.synth_tensor(qt, E * M, K, 33, 1)
    stride = orc.tensor_bytes(qt, M, K)
    routing = np.concatenate([np.array([1, 99], np.uint32), np.full(k, 0.5, np.float32).view(np.uint32)])
    xs = orc.synth_normal_f32(k * K, 33, 2)
    bW, br, bx, by = ctx.upload(W), ctx.upload(routing), ctx.upload(xs), ctx.alloc(k * M * 4)
    ctx.dmmv_moe(qt, bW, stride, br, bx, K, 0, by, 0, M, K, k)
    with pytest.raises(zinc_amd.ZincError) as e:
        ctx.sync()
    assert e.value.name == "InvalidArgument"
    ctx.sync()  # reported once
    got = by.download(np.float32, k * M).reshape(k, M)
    We = W[(E - 1) * stride:E * stride]
    xe = xs[K:2 * K]
    assert_dot_close(got[1], orc.dmmv(We, qt, xe, M, K), orc.dmmv_f64(We, qt, xe, M, K),
                     orc.dmmv_absdot(We, qt, xe, M, K), "clamped slot")


def test_rms_norm(ctx, orc):
    n = 4096
    x = orc.synth_normal_f32(n * 3, 4, 1, scale=7.0)
    w = orc.synth_norm_weight(n, 4, 2)
    bx, bw, bo = ctx.upload(x), ctx.upload(w), ctx.alloc(n * 3 * 4)
    ctx.rms_norm(bx, 0, bw, n, bo, 0, n, 3, 1e-6)
    assert_close(bo.download(np.float32, 3 * n), orc.rms_norm_mul(x, w, n, 3, 1e-6), "rms", 1e-5, 1e-6)


def test_swiglu(ctx, orc):
    n = 12288
    g = orc.synth_normal_f32(n, 5, 1, scale=4.0)
    u = orc.synth_normal_f32(n, 5, 2)
    bg, bu, bo = ctx.upload(g), ctx.upload(u), ctx.alloc(n * 4)
    ctx.swiglu(bg, bu, bo, n)
    assert_close(bo.download(np.float32, n), orc.swiglu(g, u), "swiglu", 1e-5, 1e-6)


def kv_setup(ctx, orc, nkv, hd, cache_tokens, L, seed, shuffle_pages=True):
    """Random fp16 K/V for logical tokens [0, L), stored head-major through a
    (shuffled) 16-token page table."""
    n_pages = cache_tokens // 16
    rng = np.random.default_rng(seed)
    pages = rng.permutation(n_pages).astype(np.uint32) if shuffle_pages else np.arange(n_pages, dtype=np.uint32)
    k = orc.synth_normal_f16(L * nkv * hd, seed, 1).reshape(L, nkv, hd)
    v = orc.synth_normal_f16(L * nkv * hd, seed, 2).reshape(L, nkv, hd)
    kc = np.zeros((nkv, cache_tokens, hd), np.uint16)
    vc = np.zeros((nkv, cache_tokens, hd), np.uint16)
    t = np.arange(L)
    phys = pages[t // 16] * 16 + t % 16
    kc[:, phys, :] = k.transpose(1, 0, 2)
    vc[:, phys, :] = v.transpose(1, 0, 2)
    return pages, k, v, kc, vc


@pytest.mark.parametrize("L", [1, 15, 16, 17, 300, 1000, 4096, 4113, 32768])
def test_flash_decode_paged(ctx, orc, L):
    nh, nkv, hd = 32, 8, 128
    cache_tokens = ((L + 15) // 16 + 3) * 16
    pages, k, v, kc, vc = kv_setup(ctx, orc, nkv, hd, cache_tokens, L, 40 + L)
    q = orc.synth_normal_f32(nh * hd, 40 + L, 3)
    ref = orc.attention_f16(q, k.ravel(), v.ravel(), hd, nh, nkv, L)
    bq, bk, bv, bp, bo = ctx.upload(q), ctx.upload(kc), ctx.upload(vc), ctx.upload(pages), ctx.alloc(nh * hd * 4)
    ctx.flash_decode(bq, bk, bv, bp, len(pages), cache_tokens, bo, nh, nkv, hd, L)
    got = bo.download(np.float32, nh * hd)
    assert_close(got, ref, f"flash L={L}")
    if L == 1:  # seq_len 1 returns V (forward.zig:5224-5226)
        vf = v.view(np.float16).astype(np.float32).reshape(nkv, hd)
        assert np.array_equal(got.reshape(nh, hd), np.repeat(vf, nh // nkv, 0))
    for b in (bq, bk, bv, bp, bo):
        ctx.free(b)


def test_flash_decode_moe_gqa8(ctx, orc):
    nh, nkv, hd, L = 32, 4, 128, 2000
    cache_tokens = 2048
    pages, k, v, kc, vc = kv_setup(ctx, orc, nkv, hd, cache_tokens, L, 7)
    q = orc.synth_normal_f32(nh * hd, 7, 3)
    ref = orc.attention_f16(q, k.ravel(), v.ravel(), hd, nh, nkv, L)
    bq, bk, bv, bp, bo = ctx.upload(q), ctx.upload(kc), ctx.upload(vc), ctx.upload(pages), ctx.alloc(nh * hd * 4)
    ctx.flash_decode(bq, bk, bv, bp, len(pages), cache_tokens, bo, nh, nkv, hd, L)
    assert_close(bo.download(np.float32, nh * hd), ref, "flash gqa8")


def test_qk_norm_rope_kv_write(ctx, orc):
    nq, nkv, hd, pos = 32, 8, 128, 4100
    cache_tokens = 4352
    n_pages = cache_tokens // 16
    pages = np.random.default_rng(1).permutation(n_pages).astype(np.uint32)
    q = orc.synth_normal_f32(nq * hd, 8, 1, scale=50.0)
    k = orc.synth_normal_f32(nkv * hd, 8, 2, scale=50.0)
    v = orc.synth_normal_f32(nkv * hd, 8, 3, scale=3.0)
    qw, kw = orc.synth_norm_weight(hd, 8, 4), orc.synth_norm_weight(hd, 8, 5)
    inv = orc.rope_inv_freq(hd, 1e6)
    bq, bqw, bk, bkw, bv, binv = (ctx.upload(a) for a in (q, qw, k, kw, v, inv))
    bkc = ctx.upload(np.zeros(nkv * cache_tokens * hd, np.uint16))
    bvc = ctx.upload(np.zeros(nkv * cache_tokens * hd, np.uint16))
    bp = ctx.upload(pages)
    ctx.qk_norm_rope_kv_write(bq, bqw, bk, bkw, bv, binv, bkc, bvc, bp, n_pages, cache_tokens, nq, nkv, hd, pos, 1e-6)
    rq = orc.rope(orc.per_head_rms_norm(q, qw, hd, nq, 1e-6), hd, hd, nq, pos, inv)
    rk = orc.rope(orc.per_head_rms_norm(k, kw, hd, nkv, 1e-6), hd, hd, nkv, pos, inv)
    assert_close(bq.download(np.float32, nq * hd), rq, "q", 1e-4, 1e-5)
    phys = pages[pos // 16] * 16 + pos % 16
    kc = bkc.download(np.uint16, nkv * cache_tokens * hd).reshape(nkv, cache_tokens, hd)
    vc = bvc.download(np.uint16, nkv * cache_tokens * hd).reshape(nkv, cache_tokens, hd)
    gk = kc[:, phys, :].view(np.float16).astype(np.float32).ravel()
    assert_close(gk, rk, "k cache", 2e-3, 1e-4)  # fp16 storage: half-ulp 4.9e-4 relative
    assert np.array_equal(vc[:, phys, :].ravel(), v.astype(np.float16).view(np.uint16))
    # nothing else written
    mask = np.ones(cache_tokens, bool)
    mask[phys] = False
    assert not kc[:, mask, :].any() and not vc[:, mask, :].any()
    with pytest.raises(Exception):
        ctx.qk_norm_rope_kv_write(bq, bqw, bk, bkw, bv, binv, bkc, bvc, bp, n_pages, cache_tokens, nq, nkv, hd,
                                  cache_tokens, 1e-6)


def test_softmax_topk_and_weighted_acc(ctx, orc):
    for trial, (n, k) in enumerate([(128, 8), (8, 3), (256, 16), (3, 1)]):
        lg = orc.synth_normal_f32(n, 50 + trial, 1)
        if trial == 0:
            lg[[5, 77]] = lg.max() + 1.0  # exact tie: lowest index first
        bl, br = ctx.upload(lg), ctx.alloc(8 * k)
        ctx.softmax_topk(bl, n, k, br)
        r = br.download(np.uint32, 2 * k)
        ids, w = orc.topk_softmax(lg, k)
        assert np.array_equal(r[:k], ids)
        assert np.allclose(r[k:].view(np.float32), w, rtol=1e-5, atol=1e-7)
    H, k = 2048, 8
    a = orc.synth_normal_f32(H, 60, 1)
    b = orc.synth_normal_f32(k * H, 60, 2)
    routing = np.concatenate([np.arange(k, dtype=np.uint32), orc.synth_norm_weight(k, 60, 3).view(np.uint32)])
    ba, bb, br = ctx.upload(a), ctx.upload(b), ctx.upload(routing)
    ctx.moe_weighted_acc(ba, bb, br, H, k, H)
    w = routing[k:].view(np.float32)
    ref = a.copy()
    for i in range(H):
        s = np.float32(0)
        for j in range(k):
            s = np.float32(s + np.float32(w[j] * b[j * H + i]))
        ref[i] = np.float32(ref[i] + s)
    assert_close(ba.download(np.float32, H), ref, "moe acc", 1e-6, 1e-6)


def test_argmax_first_max(ctx, orc):
    for n, seed in [(151936, 1), (100, 2), (1, 3), (70000, 4)]:
        lg = orc.synth_normal_f32(n, seed, 1)
        if n > 10:
            lg[[n - 1, n // 2, 7]] = lg.max() + 0.5  # ties -> lowest index
        bl, br = ctx.upload(lg), ctx.alloc(4)
        ctx.argmax(bl, n, br)
        assert br.download(np.uint32, 1)[0] == orc.argmax(lg)
