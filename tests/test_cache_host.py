"""Host-side cache bookkeeping: configuration checks, the block allocator's
reference counts and the pinned host store.

Scenarios and expected values follow the reference's tests
(tests/test_config.py:7-17, tests/test_allocator.py:7-60,
tests/test_storage.py:9-84); everything here is CPU-only host logic.
"""

import pytest
import torch

from nano_hisparse.allocator import DeviceAllocator
from nano_hisparse.config import CacheConfig, CapacityError
from nano_hisparse.storage import HostStore, Location, PageLease


@pytest.mark.parametrize("field", ["gpu_pages", "host_pages", "page_size", "kv_heads", "head_dim"])
def test_config_rejects_nonpositive_dimension(field):
    with pytest.raises(ValueError, match=field):
        CacheConfig(**{field: 0})


def test_config_rejects_int8_kv_and_zero_index_budget():
    with pytest.raises(ValueError, match="dtype"):
        CacheConfig(dtype=torch.int8)
    with pytest.raises(ValueError, match="index budget"):
        CacheConfig(index_budget_bytes=0)


def test_config_row_bytes():
    assert CacheConfig(kv_heads=8, head_dim=128, dtype=torch.bfloat16).row_bytes == 4096


# ---- allocator -------------------------------------------------------------------------


def test_unpinned_block_keeps_owner_until_reclaimed():
    alloc = DeviceAllocator(CacheConfig(gpu_pages=2, device="cpu"))
    first = ("a", 0, 0)
    alloc.bind(0, first)
    assert alloc.slots[0].ref_cnt == 1
    reused = []

    def on_reuse(slot):
        reused.append(slot)
        alloc.release(slot, fence="reader-fence")

    alloc.unpin(0, on_reuse)
    alloc.unpin(0, on_reuse)  # a second unpin is a no-op
    assert alloc.slots[0].owner == first and 0 not in alloc.free and alloc.slots[0].ref_cnt == 0
    alloc.reclaim(0)
    assert reused == [0] and alloc.slots[0].fence == "reader-fence" and alloc.slots[0].ref_cnt == 0
    alloc.bind(0, ("b", 0, 0))
    assert alloc.slots[0].ref_cnt == 1
    assert alloc.occupancy["a"] == 0 and alloc.occupancy["b"] == 1


def test_block_reuse_waits_for_every_reader():
    alloc = DeviceAllocator(CacheConfig(gpu_pages=1, device="cpu"))
    owner = ("a", 0, 0)
    alloc.bind(0, owner)
    alloc.incref(0)
    alloc.incref(0)
    assert alloc.slots[0].ref_cnt == 3
    with pytest.raises(RuntimeError, match="active references"):
        alloc.release(0, None)
    alloc.unpin(0, lambda slot: alloc.release(slot, "fence"))
    for remaining in (2, 1):
        assert alloc.slots[0].ref_cnt == remaining
        for call in (lambda: alloc.reclaim(0), lambda: alloc.release(0, None)):
            with pytest.raises(RuntimeError, match="active references"):
                call()
        assert alloc.slots[0].owner == owner
        alloc.decref(0)
    with pytest.raises(RuntimeError, match="no reader"):
        alloc.decref(0)
    alloc.reclaim(0)
    assert alloc.free == {0} and alloc.slots[0].fence == "fence"
    with pytest.raises(RuntimeError, match="unbound"):
        alloc.incref(0)
    alloc.bind(0, owner)  # the same owner again: no generation counter needed
    with pytest.raises(RuntimeError, match="no reader"):
        alloc.decref(0)
    alloc.release(0, None)
    assert alloc.slots[0].ref_cnt == 0


# ---- host store ---------------------------------------------------------------------------


def _store():
    cfg = CacheConfig(gpu_pages=3, host_pages=6, page_size=4, kv_heads=1, head_dim=4, device="cpu")
    return HostStore(cfg, DeviceAllocator(cfg))


def test_append_mirrors_new_rows_only_and_retire_frees_host_pages():
    store = _store()
    store.reserve("a", 12, 1)

    def prepare(page):
        if page.slot is None:
            store.bind(page, min(store.allocator.free), Location.RESIDENT)
            return None
        return PageLease(store, [page])

    k, v = torch.randn(9, 1, 4), torch.randn(9, 1, 4)
    store.append("a", 0, k[:3], v[:3], prepare)
    store.append("a", 0, k[3:], v[3:], prepare)
    host_k, host_v = store.host_kv("a", 0)
    torch.testing.assert_close(host_k, k)
    torch.testing.assert_close(host_v, v)
    assert store.stats["d2h_bytes"] == 9 * 2 * 4 * 4  # each row mirrored once
    first = store.pages["a", 0, 0]
    assert first.content_version == 2 and first.sealed
    old_request = store.requests["a"]
    for page in list(store.pages.values()):
        store.detach(page)
    store.retire("a")
    store.collect()
    store.assert_invariants()
    assert len(store.free_host) == 6
    store.reserve("a", 12, 1)
    assert store.requests["a"] is not old_request
    fresh = store.materialize("a", 0, 0)
    store.bind(fresh, min(store.allocator.free), Location.RESIDENT)
    with pytest.raises(RuntimeError, match="retired page"):
        PageLease(store, [first])
    assert store.allocator.slots[fresh.slot].ref_cnt == 1


def test_reservation_counts_unmaterialized_host_pages():
    store = _store()
    store.reserve("a", 24, 1)
    assert not store.pages and len(store.free_host) == 6
    with pytest.raises(CapacityError, match="host credits"):
        store.reserve("b", 1, 1)
    assert set(store.requests) == {"a"}
    store.assert_invariants()


def test_overlapping_leases_balance_pins_and_released_handles_fail():
    store = _store()
    store.reserve("a", 4, 1)
    page = store.materialize("a", 0, 0)
    store.bind(page, 0, Location.RESIDENT)
    store.allocator.unpin(0, lambda slot: store.detach(page))
    one, two = PageLease(store, [page]), PageLease(store, [page])
    assert store.allocator.slots[0].ref_cnt == page.pins == 2
    one.release()
    assert store.allocator.slots[0].ref_cnt == page.pins == 1
    with pytest.raises(RuntimeError, match="active references"):
        store.allocator.reclaim(0)
    two.release()
    assert store.allocator.slots[0].ref_cnt == page.pins == 0
    store.allocator.reclaim(0)
    store.bind(page, 0, Location.RESIDENT)
    for lease in (one, two):
        for call in (lease.wait, lease.release):
            with pytest.raises(RuntimeError, match="released"):
                call()
    assert store.allocator.slots[0].ref_cnt == 1
    store.assert_invariants()


def test_pool_block_stride_of_contiguous_and_gapped_pools():
    """The launchers pass a pool's block stride to the C ABI: a contiguous
    pool (the CPU cache's) has one block per stride; a pool whose blocks are
    followed by a gap (the GPU cache's padded pool, a strided view) has a
    larger stride; a pool whose blocks are not contiguous is rejected."""
    from nano_hisparse import row_kernels as rk

    pool = rk.padded_pool(6, 4, 2, 8, torch.bfloat16, "cpu")  # contiguous off the GPU
    assert pool.is_contiguous() and pool.shape == (6, 2, 4, 2, 8)
    block = 2 * 4 * 2 * 8
    assert rk.pool_block_stride(pool) == block * 2
    flat = torch.zeros(6 * (block + 3 * 8), dtype=torch.bfloat16)
    gapped = flat.as_strided(pool.shape, (block + 3 * 8, 4 * 2 * 8, 2 * 8, 8, 1))
    assert rk.pool_block_stride(gapped) == (block + 3 * 8) * 2
    with pytest.raises(ValueError, match="contiguous"):
        rk.pool_block_stride(pool.transpose(1, 2))
    with pytest.raises(ValueError, match="blocks"):
        rk.pool_block_stride(pool[0])
