"""The host page pool (zh_kv_pool_*, KvPagePool src/scheduler/kv_cache.zig:
43-125) through the C ABI. The cases restate the reference's own tests
(kv_cache.zig:131-230); no GPU is needed (the pool is host code)."""
import pytest


@pytest.fixture
def pool_cls():
    import zinc_amd
    return zinc_amd.KvPagePool


def test_alloc_and_free(pool_cls):  # kv_cache.zig:131-145
    pool = pool_cls(4, 256)
    assert pool.free_count() == 4
    pages = pool.alloc_pages(1, 2)
    assert pool.free_count() == 2 and len(pages) == 2
    pool.free_pages(1)
    assert pool.free_count() == 4


def test_exhaustion(pool_cls):  # kv_cache.zig:147-160
    import zinc_amd
    pool = pool_cls(2, 256)
    pool.alloc_pages(1, 2)
    with pytest.raises(zinc_amd.ZincError) as e:
        pool.alloc_pages(2, 1)
    assert e.value.name == "KvCacheExhausted"
    pool.free_pages(1)
    pool.alloc_pages(2, 1)
    assert pool.free_count() == 1


def test_requests_isolated(pool_cls):  # kv_cache.zig:162-180
    pool = pool_cls(8, 256)
    p1 = pool.alloc_pages(100, 3)
    p2 = pool.alloc_pages(200, 2)
    assert pool.free_count() == 3
    assert not set(p1.tolist()) & set(p2.tolist())
    pool.free_pages(100)
    assert pool.free_count() == 6
    pool.free_pages(200)
    assert pool.free_count() == 8


def test_stack_order_and_reuse(pool_cls):
    """allocPages pops the free stack from its end: a fresh pool hands out
    the highest ids first; freed pages come back on top."""
    pool = pool_cls(8, 16)
    assert pool.alloc_pages(1, 3).tolist() == [7, 6, 5]
    assert pool.alloc_pages(2, 2).tolist() == [4, 3]
    pool.free_pages(1)  # pages 5, 6, 7 pushed in id order
    assert pool.alloc_pages(3, 2).tolist() == [7, 6]


def test_free_nonexistent_is_noop_and_max_context(pool_cls):  # kv_cache.zig:218-230
    pool = pool_cls(4, 16)
    pool.free_pages(999)
    assert pool.free_count() == 4
    assert pool.max_context(3) == 48
