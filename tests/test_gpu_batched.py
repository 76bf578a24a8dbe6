"""Batched DMMV (zh_dmmv_batched, zh_dmmv_fused_gate_up_swiglu_batched: the
skinny GEMM of recordBatchDispatchPush, dmmv.zig:880-925) through the C ABI.

Every column of a batched launch must equal the one-vector DMMV of that
column bit for bit where the one-vector path runs the tile kernels (the
weight tile is shared, the per-column arithmetic is the one-vector
kernel's); Q4_K with K = 2048 / 4096 runs the streaming kernel one vector at
a time, whose half-super-block partial sums round in another order, so there
the columns agree to the f32 summation floor (2^-20 of sum |w x|). Every
column meets the oracle bar of the one-vector kernels: |gpu - ref| <= 1e-4 +
1e-3 |ref| (+ the f32 dot-product noise floor of
test_gpu_kernels.assert_dot_close). Column counts cover the 4-, 2- and
1-vector launches and their mixtures (3, 5 and 8 columns)."""
import numpy as np
import pytest

from test_gpu_kernels import assert_dot_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    import zinc_amd
    c = zinc_amd.Context(0)
    yield c
    c.close()


def _ring(qt, K):
    """The one-vector path is the streaming kernel (zh_dmmv_ring.hip)."""
    return qt == 12 and K in (2048, 4096)


def _same(got, ref, mag, ring):
    if not ring:
        return np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    return bool(np.all(np.abs(got.astype(np.float64) - ref) <= 2.0 ** -20 * mag + 1e-30))


def _single(ctx, qt, Wb, x, M, K, y0=None):
    xb = ctx.upload(x)
    yb = ctx.upload(y0 if y0 is not None else np.zeros(M, np.float32))
    ctx.dmmv(qt, Wb, 0, xb, 0, yb, 0, M, K, 1 if y0 is not None else 0)
    out = yb.download(np.float32, M)
    ctx.free(xb)
    ctx.free(yb)
    return out


@pytest.mark.parametrize("qt,M,K", [(12, 4096, 4096), (12, 6144, 4096), (12, 1000, 768), (12, 512, 12288),
                                    (14, 4096, 12288), (14, 1024, 4096), (14, 300, 2048)])
@pytest.mark.parametrize("ncol", [1, 2, 3, 4, 5, 8])
def test_batched_equals_single_columns(ctx, orc, qt, M, K, ncol):
    print(f"batched q{qt} {M}x{K} cols {ncol}", flush=True)
    W = orc.synth_tensor(qt | 0x100 if qt == 12 else qt, M, K, 61 + ncol, 1)
    X = np.stack([orc.synth_normal_f32(K, 61, 10 + v) for v in range(ncol)])
    Wb, Xb, Yb = ctx.upload(W), ctx.upload(X), ctx.alloc(4 * M * ncol)
    ctx.dmmv_batched(qt, Wb, 0, Xb, 0, Yb, 0, M, K, ncol)
    Y = Yb.download(np.float32, M * ncol).reshape(ncol, M)
    ring = _ring(qt, K)
    mags = [orc.dmmv_absdot(W, qt, X[v], M, K) for v in range(ncol)] if ring else [None] * ncol
    for v in range(ncol):
        ref = _single(ctx, qt, Wb, X[v], M, K)
        assert _same(Y[v], ref, mags[v], ring), (v, np.abs(Y[v] - ref).max())
    # and the oracle bar on the first and last columns
    for v in {0, ncol - 1}:
        assert_dot_close(Y[v], orc.dmmv(W, qt, X[v], M, K), orc.dmmv_f64(W, qt, X[v], M, K),
                         orc.dmmv_absdot(W, qt, X[v], M, K), f"batched col {v}")
    # acc_mode 1: Y[v] += W X[v]
    Y0 = np.stack([orc.synth_normal_f32(M, 62, v) for v in range(ncol)])
    Yb.upload(Y0)
    ctx.dmmv_batched(qt, Wb, 0, Xb, 0, Yb, 0, M, K, ncol, 1)
    Y1 = Yb.download(np.float32, M * ncol).reshape(ncol, M)
    for v in range(ncol):
        ref = _single(ctx, qt, Wb, X[v], M, K, Y0[v])
        assert _same(Y1[v], ref, mags[v] + np.abs(Y0[v]) if ring else None, ring), v
    for b in (Wb, Xb, Yb):
        ctx.free(b)


def test_batched_lm_head_shape(ctx, orc):
    """The LM-head shape (M >= 65536: the one-vector path is the lane-per-block
    kernel, so the columns are held to the oracle bar only)."""
    qt, M, K, ncol = 14, 70000, 4096, 4
    W = orc.synth_tensor(qt, M, K, 71, 1)
    X = np.stack([orc.synth_normal_f32(K, 71, 10 + v) for v in range(ncol)])
    Wb, Xb, Yb = ctx.upload(W), ctx.upload(X), ctx.alloc(4 * M * ncol)
    ctx.dmmv_batched(qt, Wb, 0, Xb, 0, Yb, 0, M, K, ncol)
    Y = Yb.download(np.float32, M * ncol).reshape(ncol, M)
    for v in (0, 3):
        assert_dot_close(Y[v], orc.dmmv(W, qt, X[v], M, K, nthreads=8), orc.dmmv_f64(W, qt, X[v], M, K),
                         orc.dmmv_absdot(W, qt, X[v], M, K), f"lm-head col {v}")
    for b in (Wb, Xb, Yb):
        ctx.free(b)


@pytest.mark.parametrize("ncol", [1, 2, 3, 4, 6])
def test_batched_gate_up_equals_single(ctx, orc, ncol):
    qt, M, K = 12, 2048, 4096
    Wg = orc.synth_tensor(qt | 0x100, M, K, 81, 1)
    Wu = orc.synth_tensor(qt | 0x100, M, K, 81, 2)
    X = np.stack([orc.synth_normal_f32(K, 81, 10 + v) for v in range(ncol)])
    bg, bu, Xb, Yb = ctx.upload(Wg), ctx.upload(Wu), ctx.upload(X), ctx.alloc(4 * M * ncol)
    ctx.dmmv_fused_gate_up_swiglu_batched(qt, bg, 0, bu, 0, Xb, 0, Yb, 0, M, K, ncol)
    Y = Yb.download(np.float32, M * ncol).reshape(ncol, M)
    for v in range(ncol):
        xb, yb = ctx.upload(X[v]), ctx.alloc(4 * M)
        ctx.dmmv_fused_gate_up_swiglu(qt, bg, 0, bu, 0, xb, 0, yb, 0, M, K)
        ref = yb.download(np.float32, M)
        # the one-vector path at K = 4096 is the streaming kernel: f32 summation order differs
        assert np.allclose(Y[v], ref, rtol=2e-5, atol=2e-6 * np.abs(ref).max()), (v, np.abs(Y[v] - ref).max())
        ctx.free(xb)
        ctx.free(yb)
    g = orc.dmmv(Wg, qt, X[0], M, K)
    u = orc.dmmv(Wu, qt, X[0], M, K)
    assert np.allclose(Y[0], orc.swiglu(g, u), rtol=1e-3, atol=1e-3 * np.abs(orc.swiglu(g, u)).max())
    for b in (bg, bu, Xb, Yb):
        ctx.free(b)


def test_batched_rejects_bad_arguments(ctx):
    import zinc_amd
    W, X, Y = ctx.alloc(1 << 22), ctx.alloc(1 << 20), ctx.alloc(1 << 20)
    for args, name in [((12, 256, 4096, 0), "InvalidArgument"), ((12, 256, 4096, 17), "InvalidArgument"),
                       ((8, 256, 4096, 2), "UnsupportedQuantType"), ((13, 256, 4096, 2), "UnsupportedQuantType"),
                       ((12, 256, 300, 2), "InvalidArgument"),
                       ((12, 4096, 4096, 2), "InvalidArgument")]:  # W too small
        qt, M, K, n = args
        with pytest.raises(zinc_amd.ZincError) as e:
            ctx.dmmv_batched(qt, W, 0, X, 0, Y, 0, M, K, n)
        assert e.value.name == name, args
    with pytest.raises(zinc_amd.ZincError) as e:
        ctx.dmmv_batched(12, W, 4, X, 0, Y, 0, 256, 4096, 2)  # a_off not 16-byte aligned
    assert e.value.name == "InvalidArgument"
    for b in (W, X, Y):
        ctx.free(b)
