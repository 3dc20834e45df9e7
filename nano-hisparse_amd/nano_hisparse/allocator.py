"""Device blocks of the KV pool: ownership, reference counts and reuse.

Reference: nano_hisparse/allocator.py:9-83. One pool tensor of
[gpu_pages, 2, page_size, kv_heads, head_dim] holds resident pages and hot
blocks alike. A block bound to an owner carries one allocation reference;
readers add temporary references. A block whose allocation reference was
given up (unpinned) stays readable until it is reclaimed, which runs the
owner's callback; `fence` is the event that must complete before the block's
bytes may be overwritten.

Besides the reference's structures the allocator keeps indexes that make the
residency policy independent of the pool size: the bound blocks of each
(request, layer) in binding order, the KV-page blocks of each (request,
layer) that still hold their allocation reference, a min-heap of empty
blocks (stale entries are skipped lazily) and the number of unpinned blocks
that readers still reference, so "allocatable blocks" is counted and
enumerated in order, and a layer's unpin candidates are found, without a
scan.
"""

from __future__ import annotations

import heapq
from collections import Counter, OrderedDict
from dataclasses import dataclass

import torch


@dataclass
class DeviceSlot:
    owner: tuple | None = None
    ref_cnt: int = 0
    fence: object = None


class DeviceAllocator:
    def __init__(self, config):
        from .row_kernels import padded_pool

        # on a GPU each block is followed by a few head slots of padding (padded_pool)
        self.storage = padded_pool(config.gpu_pages, config.page_size, config.kv_heads, config.head_dim,
                                   config.dtype, config.device)
        self.budget = config.gpu_pages
        self.slots = [DeviceSlot() for _ in range(config.gpu_pages)]
        self.free: set[int] = set(range(config.gpu_pages))
        # slot -> callback run when an unpinned (still readable) block is taken
        self.reclaimable: OrderedDict[int, object] = OrderedDict()
        # owner key -> slot, in binding order
        self.lru: OrderedDict[tuple, int] = OrderedDict()
        self.occupancy: Counter = Counter()
        # (request, layer) -> {owner key: slot} in binding order
        self.group_blocks: dict[tuple, OrderedDict] = {}
        # (request, layer) -> {owner key: slot} of KV pages (key[2] >= 0) not unpinned
        self.group_pinned: dict[tuple, dict] = {}
        self._empty_heap = list(range(config.gpu_pages))
        self.referenced_unpinned = 0  # reclaimable blocks with reader references

    def _allocation_refs(self, slot) -> int:
        return 0 if slot in self.reclaimable else 1

    def bind(self, slot, key):
        frame = self.slots[slot]
        assert slot in self.free and slot < self.budget
        assert frame.owner is None and frame.ref_cnt == 0
        self.free.discard(slot)
        frame.owner, frame.ref_cnt = key, 1
        self.lru[key] = slot
        self.occupancy[key[0]] += 1
        self.group_blocks.setdefault(key[:2], OrderedDict())[key] = slot
        if key[2] >= 0:
            self.group_pinned.setdefault(key[:2], {})[key] = slot

    def release(self, slot, fence):
        frame = self.slots[slot]
        assert frame.owner is not None
        if frame.ref_cnt != self._allocation_refs(slot):
            raise RuntimeError("cannot release a block with active references")
        owner = frame.owner
        self.reclaimable.pop(slot, None)
        del self.lru[owner]
        self.occupancy[owner[0]] -= 1
        group = self.group_blocks[owner[:2]]
        del group[owner]
        if not group:
            del self.group_blocks[owner[:2]]
        self._drop_pinned(owner)
        frame.owner, frame.ref_cnt, frame.fence = None, 0, fence
        self.free.add(slot)
        heapq.heappush(self._empty_heap, slot)
        if len(self._empty_heap) > 2 * len(self.slots) + 64:
            self._empty_heap = sorted(self.free)

    def unpin(self, slot, on_reuse):
        """Give up the allocation reference; contents stay readable."""
        frame = self.slots[slot]
        assert frame.owner is not None and slot not in self.free
        if slot in self.reclaimable:
            return
        assert frame.ref_cnt > 0
        frame.ref_cnt -= 1
        self.reclaimable[slot] = on_reuse
        self._drop_pinned(frame.owner)
        if frame.ref_cnt:
            self.referenced_unpinned += 1

    def _drop_pinned(self, key):
        pinned = self.group_pinned.get(key[:2])
        if pinned is not None and pinned.pop(key, None) is not None and not pinned:
            del self.group_pinned[key[:2]]

    def reclaim(self, slot):
        """Take an unpinned block: its owner callback detaches the old mapping."""
        if self.slots[slot].ref_cnt:
            raise RuntimeError("cannot reclaim a block with active references")
        callback = self.reclaimable[slot]
        callback(slot)
        assert slot in self.free and slot not in self.reclaimable

    def incref(self, slot):
        frame = self.slots[slot]
        if frame.owner is None:
            raise RuntimeError("cannot reference an unbound block")
        if frame.ref_cnt == 0 and slot in self.reclaimable:
            self.referenced_unpinned += 1
        frame.ref_cnt += 1

    def decref(self, slot):
        frame = self.slots[slot]
        if frame.owner is None or frame.ref_cnt <= self._allocation_refs(slot):
            raise RuntimeError("no reader reference to release")
        frame.ref_cnt -= 1
        if frame.ref_cnt == 0 and slot in self.reclaimable:
            self.referenced_unpinned -= 1

    # ---- allocatable blocks: empty ones ascending, then unreferenced unpinned
    # ---- ones in unpin order, all below the budget

    def _empty_prefix(self, count):
        """The `count` lowest empty blocks below the budget, ascending."""
        heap, out, seen = self._empty_heap, [], set()
        while heap and len(out) < count:
            slot = heap[0]
            if slot not in self.free or slot in seen:
                heapq.heappop(heap)
                continue
            if slot >= self.budget:
                break
            seen.add(heapq.heappop(heap))
            out.append(slot)
        for slot in out:
            heapq.heappush(heap, slot)
        return out

    def available(self, count=None):
        """Allocatable blocks in allocation order (the first `count`)."""
        limit = len(self.slots) if count is None else count
        out = self._empty_prefix(limit)
        if len(out) < limit:
            for slot in self.reclaimable:
                if slot < self.budget and self.slots[slot].ref_cnt == 0:
                    out.append(slot)
                    if len(out) == limit:
                        break
        return out

    def available_count(self):
        if self.budget >= len(self.slots):
            return len(self.free) + len(self.reclaimable) - self.referenced_unpinned
        return len(self.available())

    def pinned_pages(self, group):
        """{owner key: slot} of the layer's KV-page blocks that still hold
        their allocation reference (unordered)."""
        return self.group_pinned.get(group, {})

    def group_keys(self, group):
        """Owner keys bound for one (request, layer), in binding order."""
        blocks = self.group_blocks.get(group)
        return list(blocks) if blocks else []
