"""zh_flash_decode_noalloc (no allocation: partials and merge counters in a
per-GPU device array) through the C ABI: its output equals zh_flash_decode's
bit for bit on the same inputs, on two calls in a row (the second smaller:
fewer heads, a shorter context, so stale partials of the first call must not
leak into it), and meets the oracle bar. Shapes past the array are rejected."""
import numpy as np
import pytest

from test_gpu_kernels import assert_close, kv_setup

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    import zinc_amd
    c = zinc_amd.Context(0)
    yield c
    c.close()


def _case(ctx, orc, nh, nkv, L, seed):
    hd = 128
    cache_tokens = ((L + 15) // 16 + 3) * 16
    pages, k, v, kc, vc = kv_setup(ctx, orc, nkv, hd, cache_tokens, L, seed)
    q = orc.synth_normal_f32(nh * hd, seed, 3)
    ref = orc.attention_f16(q, k.ravel(), v.ravel(), hd, nh, nkv, L)
    bufs = [ctx.upload(q), ctx.upload(kc), ctx.upload(vc), ctx.upload(pages), ctx.alloc(nh * hd * 4),
            ctx.alloc(nh * hd * 4)]
    return hd, cache_tokens, len(pages), ref, bufs


def test_flash_decode_noalloc_matches_flash_decode(ctx, orc):
    for nh, nkv, L, seed in [(32, 8, 4113, 51), (8, 2, 300, 52)]:  # second call smaller
        print(f"noalloc flash decode {nh}/{nkv} L={L}", flush=True)
        hd, cache_tokens, n_pages, ref, (bq, bk, bv, bp, bo, bo2) = _case(ctx, orc, nh, nkv, L, seed)
        ctx.flash_decode_noalloc(bq, bk, bv, bp, n_pages, cache_tokens, bo, nh, nkv, hd, L)
        ctx.flash_decode(bq, bk, bv, bp, n_pages, cache_tokens, bo2, nh, nkv, hd, L)
        got, want = bo.download(np.float32, nh * hd), bo2.download(np.float32, nh * hd)
        ctx.sync()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), np.abs(got - want).max()
        assert_close(got, ref, f"noalloc L={L}")
        for b in (bq, bk, bv, bp, bo, bo2):
            ctx.free(b)


def test_flash_decode_noalloc_rejects_bad_shapes(ctx):
    import zinc_amd
    b = ctx.alloc(1 << 20)
    with pytest.raises(zinc_amd.ZincError) as e:
        ctx.flash_decode_noalloc(b, b, b, b, 64, 1024, b, 32, 8, 64, 100)  # head_dim 64
    assert e.value.name == "InvalidArgument"
    ctx.free(b)
