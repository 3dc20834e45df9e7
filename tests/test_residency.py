"""Residency policy: readable unpinned blocks, mirror publication, window and
watermark hot triggers, the two active tails and pressure handling.

Scenarios and expected states follow the reference's
tests/test_residency.py:13-310.
"""

import pytest
import torch

from nano_hisparse.attention import row_attention
from nano_hisparse.config import CacheConfig, CapacityError
from nano_hisparse.hybrid import ACTIVE_TAIL_PAGES, HotConfig, HybridKVCache
from nano_hisparse.row_index import LogicalTopK
from nano_hisparse.selection import dense_attention


def make(device, pages=7, watermark=0, window=64):
    cfg = CacheConfig(gpu_pages=pages, host_pages=128, page_size=4, kv_heads=1, head_dim=8, device=device)
    return HybridKVCache(cfg, HotConfig(4, 4, resident_window_pages=window, transition_watermark=watermark))


def append(cache, name, count):
    k = torch.randn(count, 1, 8, device=cache.device)
    v = torch.randn(count, 1, 8, device=cache.device)
    cache.write(name, 0, k, v)
    return k, v


def positions(cache, values):
    return LogicalTopK(torch.tensor(values, dtype=torch.int32, device=cache.device))


class FakeCompletion:
    """A host-side stand-in for a mirror's completion event."""

    def __init__(self, wait_completes=False):
        self.done, self.waits, self.wait_completes = False, 0, wait_completes

    def query(self):
        return self.done

    def synchronize(self):
        if not self.wait_completes:
            pytest.fail("a policy tick must not wait for a pending mirror")
        self.done = True
        self.waits += 1


def test_unpinned_page_hits_until_its_block_is_reused(device):
    cache = make(device)
    for name in ("a", "b"):
        cache.reserve(name, 64, 1)
    k, v = append(cache, "a", 12)
    cache.storage.synchronize()
    page = cache.storage.pages["a", 0, 0]
    slot, host = page.slot, page.host_slot
    assert cache.allocator.slots[slot].ref_cnt == 1
    cache.reclaim_history("a", 0)
    assert cache.page_state(page.key)["residency"] == "clean_unpinned"
    assert page.slot == slot and cache.tables["a", 0].resident[0].item() == slot
    assert cache.allocator.slots[slot].ref_cnt == 0
    assert cache.snapshot()["allocatable_device_blocks"] == 4  # 3 empty + 1 readable
    q = torch.randn(2, 8, device=device)
    torch.testing.assert_close(row_attention(q, cache, "a", 0, positions(cache, [0])), dense_attention(q, k[:1], v[:1]))
    assert cache.snapshot()["row_stats"]["misses"] == 0
    append(cache, "b", 12)  # empty blocks go first
    assert page.slot == slot and cache.storage.stats["unpinned_block_reuses"] == 0
    append(cache, "b", 1)  # no empty block left: the readable block of "a" is reused
    assert page.slot is None and page.host_slot == host
    assert cache.tables["a", 0].resident[0].item() == -1
    assert cache.owners[slot] == ("b", 0, 3) and cache.allocator.slots[slot].ref_cnt == 1
    torch.testing.assert_close(row_attention(q, cache, "a", 0, positions(cache, [0])), dense_attention(q, k[:1], v[:1]))
    assert cache.snapshot()["row_stats"]["misses"] == 1
    cache.assert_invariants()


def test_a_reader_lease_protects_a_readable_unpinned_block(device):
    cache = make(device)
    for name in ("a", "b"):
        cache.reserve(name, 64, 1)
    k, _ = append(cache, "a", 12)
    cache.storage.synchronize()
    cache.reclaim_history("a", 0)
    page = cache.storage.pages["a", 0, 0]
    slot = page.slot
    with cache.resolve("a", 0, positions(cache, [0])) as lease:
        assert slot in cache.allocator.reclaimable and cache.allocator.slots[slot].ref_cnt == 1
        assert slot not in cache._available_blocks()
        with pytest.raises(RuntimeError, match="active references"):
            cache.allocator.reclaim(slot)
        assert all(cache.allocator.slots[i].ref_cnt == 2 for i in cache.tables["a", 0].blocks)
        cache.assert_invariants()
        if cache.storage.cuda:
            torch.cuda._sleep(2_000_000)
        seen = cache.pool[slot, 0, 0].clone()
        append(cache, "b", 13)  # "b" must reclaim its own history instead
        assert page.slot == slot and cache.tables["b", 0].blocks
        lease._validate()
    torch.testing.assert_close(seen, k[0])
    assert slot in cache._available_blocks() and cache.allocator.slots[slot].ref_cnt == 0
    assert all(cache.allocator.slots[i].ref_cnt == 1 for i in cache.tables["a", 0].blocks)
    with pytest.raises(RuntimeError, match="released"):
        lease.release()
    cache.assert_invariants()


def test_resident_window_triggers_the_hot_region(device):
    cache = make(device, pages=12, window=3)
    cache.reserve("a", 64, 1)
    append(cache, "a", 8)
    assert not cache.tables["a", 0].hot_required
    append(cache, "a", 4)
    tables = cache.tables["a", 0]
    assert tables.hot_required and tables.trigger == "window" and tables.blocks
    assert cache.storage.stats["evictions"] == 0 and len(cache.allocator.free) == 8
    cache.storage.synchronize()
    cache.collect()
    assert cache.page_state(("a", 0, 0))["residency"] == "clean_unpinned"
    assert cache.storage.pages["a", 0, 0].slot is not None
    cache.assert_invariants()


def test_watermark_counts_the_block_about_to_be_allocated(device):
    cache = make(device, pages=10, watermark=4)
    cache.reserve("a", 64, 1)
    append(cache, "a", 24)
    assert len(cache.allocator.free) == 4 and not cache.tables["a", 0].blocks
    append(cache, "a", 4)
    assert cache.tables["a", 0].trigger == "watermark" and cache.tables["a", 0].blocks
    assert len(cache.allocator.free) == 2 and cache.storage.stats["evictions"] == 0
    cache.assert_invariants()


def test_hot_demand_waits_out_a_busy_layer(device):
    cache = make(device, pages=6)
    cache.reserve("a", 64, 1)
    append(cache, "a", 12)
    resident = cache.tables["a", 0].resident.clone()
    with cache.resolve("a", 0, positions(cache, [0, 4, 8])):
        with pytest.raises(CapacityError, match="active row lease"):
            cache.transition_to_host("a", 0)
        assert cache.tables["a", 0].hot_required and not cache.tables["a", 0].blocks
        torch.testing.assert_close(resident, cache.tables["a", 0].resident)
        cache.collect()
        assert not cache.tables["a", 0].blocks
    cache.collect()
    assert cache.tables["a", 0].blocks
    cache.assert_invariants()


def test_both_active_tails_stay_resident_across_page_boundaries(device):
    assert ACTIVE_TAIL_PAGES == 2
    cache = make(device, pages=3, watermark=None)
    cache.reserve("a", 64, 1)
    append(cache, "a", 9)
    pages = cache.storage.pages
    assert pages["a", 0, 0].slot is None and pages["a", 0, 1].slot is not None and pages["a", 0, 2].slot is not None
    append(cache, "a", 3)  # page 2 seals; page 1 is still a tail
    assert pages["a", 0, 1].slot is not None
    append(cache, "a", 1)
    assert pages["a", 0, 1].slot is None and pages["a", 0, 2].slot is not None and pages["a", 0, 3].slot is not None
    cache.assert_invariants()
    tiny = make(device, pages=2)
    with pytest.raises(CapacityError, match="credits"):
        tiny.reserve("a", 64, 1)
    assert not tiny.storage.requests and not tiny.tables


def test_hot_rows_equal_to_the_union_progress_when_all_rows_miss(device):
    torch.manual_seed(29)
    cache = make(device, pages=3, watermark=None)  # one hot block and two tails
    cache.reserve("a", 64, 1)
    k, v = append(cache, "a", 32)
    cache.reset_stats()
    alternatives = ([0, 4, 8, 12], [1, 5, 9, 13])
    for step in range(16):
        nk, nv = append(cache, "a", 1)
        k, v = torch.cat((k, nk)), torch.cat((v, nv))
        chosen = alternatives[step % 2]
        assert all(cache.storage.pages["a", 0, t // 4].slot is None for t in chosen)
        q = torch.randn(2, 8, device=device)
        out = row_attention(q, cache, "a", 0, positions(cache, chosen))
        torch.testing.assert_close(out, dense_attention(q, k[chosen], v[chosen]), atol=3e-6, rtol=3e-5)
        tail = (len(k) - 1) // 4
        assert all(cache.storage.pages["a", 0, p].slot is not None for p in (tail - 1, tail))
        cache.assert_invariants()
    assert cache.row_stats.tolist() == [0, 0, 64]
    assert cache.storage.requests["a"].lengths == [48]
    assert cache.storage.stats["peak_device_pages"] <= 3
    cache.release_request("a")
    cache.assert_invariants()


def test_pending_mirror_is_dirty_and_a_policy_tick_does_not_wait(cpu_kernels):
    cache = make("cpu", pages=6)
    cache.reserve("a", 64, 1)
    append(cache, "a", 12)
    page = cache.storage.pages["a", 0, 0]
    completion = FakeCompletion()
    page.host_ready, page.host_committed_version = completion, 0
    cache.pending_clean.add(page.key)
    cache.reclaim_history("a", 0)
    assert cache.page_state(page.key)["residency"] == "dirty"
    assert page.slot not in cache.allocator.reclaimable
    cache.collect()
    assert page.slot not in cache.allocator.reclaimable
    completion.done = True
    cache.collect()
    assert cache.page_state(page.key)["residency"] == "clean_unpinned"
    page.host_ready = None
    cache.release_request("a")
    cache.assert_invariants()


def test_pressure_waits_for_one_eligible_mirror(cpu_kernels):
    cache = make("cpu", pages=3, watermark=0)
    cache.reserve("a", 64, 1)
    append(cache, "a", 12)
    completions = []
    for index in (0, 1):
        page = cache.storage.pages["a", 0, index]
        page.host_ready, page.host_committed_version = FakeCompletion(wait_completes=True), 0
        cache.pending_clean.add(page.key)
        completions.append(page.host_ready)
    original = cache.storage.wait
    cache.storage.wait = lambda stream, event: None  # the fakes are not stream events
    append(cache, "a", 1)
    assert sum(c.waits for c in completions) >= 1
    assert cache.storage.stats["pressure_mirror_waits"] >= 1
    for page in cache.storage.pages.values():
        page.host_ready = None
    cache.storage.wait = original
    cache.release_request("a")
    cache.assert_invariants()


def test_allocation_revisits_a_group_published_late(cpu_kernels, monkeypatch):
    cache = make("cpu", pages=4)
    cache.reserve("a", 64, 1)
    append(cache, "a", 12)
    cache.transition_to_host("a", 0)
    page = cache.storage.pages["a", 0, 0]
    slot = page.slot
    cache.allocator.reclaimable.pop(slot)
    cache.allocator.incref(slot)  # put the allocation reference back
    cache.allocator.group_pinned.setdefault(page.key[:2], {})[page.key] = slot  # and its index entry
    page.host_committed_version = 0
    assert not cache.allocator.free

    def publish_after_the_policy_tick(**kwargs):
        # the mirror completes only after the tick has visited the group
        cache.pending_clean.add(page.key)
        cache._publish_clean()

    monkeypatch.setattr(cache, "update_residency", publish_after_the_policy_tick)
    assert cache._slot() == slot
    assert page.slot is None and cache.tables["a", 0].resident[0].item() == -1
    cache.assert_invariants()


class HeldMirror:
    """A host mirror event that completes only when the test says so (the
    policy only queries mirror events on this path)."""

    def __init__(self):
        self.done = False

    def query(self):
        return self.done


def test_page_stays_pinned_until_its_mirror_event_completes(device):
    cache = make(device, pages=8)
    cache.reserve("a", 64, 1)
    k = torch.randn(12, 1, 8, device=cache.device)
    v = torch.randn(12, 1, 8, device=cache.device)
    cache.write("a", 0, k, v)
    cache.storage.synchronize()
    # a mirror still in flight: its event has not completed yet
    page = cache.storage.pages["a", 0, 0]
    held = HeldMirror()
    page.host_ready, page.host_committed_version = held, 0
    cache.pending_clean.add(page.key)
    cache.transition_to_host("a", 0)
    assert page.slot not in cache.allocator.reclaimable
    assert cache.page_state(page.key)["residency"] == "dirty"
    assert cache.storage.stats["pressure_mirror_waits"] == 0
    held.done = True
    cache.collect()
    assert cache.page_state(page.key)["residency"] == "clean_unpinned"
    page.host_ready = None
    cache.assert_invariants()
