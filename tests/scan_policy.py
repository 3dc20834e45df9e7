"""The residency policy as a full sweep: every tick visits every layer and
every bound block, with no index. HybridKVCache visits only the layers that
can act and reads allocatable blocks from the allocator's indexes; the
differential tests drive both through the same operations and require the
same decisions (block ids, unpin order, counters, errors).
"""

from collections import Counter
from contextlib import suppress

import torch

from nano_hisparse.config import CapacityError
from nano_hisparse.hybrid import ACTIVE_TAIL_PAGES, HybridKVCache


class ScanningCache(HybridKVCache):
    def _available_blocks(self, count=None):
        alloc = self.allocator
        empty = sorted(i for i in alloc.free if i < self.budget)
        readable = [i for i in alloc.reclaimable if i < self.budget and alloc.slots[i].ref_cnt == 0]
        out = empty + readable
        return out if count is None else out[:count]

    def _historical_pages(self, group=None):
        alloc, pages = self.allocator, self.storage.pages
        tails, out = {}, []
        for key in alloc.lru:
            if key[2] < 0 or (group is not None and key[:2] != group):
                continue
            page = pages[key]
            g = key[:2]
            if g not in tails:
                tails[g] = self._tail_index(g)
            allocation_ref = int(page.slot not in alloc.reclaimable)
            if page.sealed and alloc.slots[page.slot].ref_cnt == allocation_ref and key[2] <= tails[g] - ACTIVE_TAIL_PAGES:
                out.append(page)
        return out

    def _publish_clean(self):
        for key in list(self.pending_clean):
            page = self.storage.pages.get(key)
            if page is None:
                self.pending_clean.discard(key)
            elif page.host_ready is None or page.host_ready.query():
                page.host_committed_version = page.host_enqueued_version
                self.pending_clean.discard(key)
                self.storage.stats["host_mirror_completions"] += 1

    def _unpin_clean_pages(self, group):
        if not self.tables[group].blocks:
            return
        for page in sorted(self._historical_pages(group), key=lambda p: -p.key[2]):
            if page.host_committed_version == page.content_version and page.slot not in self.allocator.reclaimable:
                self.allocator.unpin(page.slot, self._on_block_reused)
                self.storage.stats["clean_page_unpins"] += 1

    def update_residency(self, request_id=None, layer=None, *, upcoming_allocation=False):
        self.storage.check_stream()
        self._publish_clean()
        groups = [
            g for g in self.tables
            if g[0] in self.storage.requests
            and (request_id is None or g[0] == request_id)
            and (layer is None or g[1] == layer)
        ]
        for group in groups:
            self._unpin_clean_pages(group)
        for group in groups:
            tables = self.tables[group]
            residents = sum(p.slot is not None for p in self.storage.group_pages.get(group, ()))
            if not residents:
                continue
            if not tables.hot_required:
                free = len(self._available_blocks()) - int(upcoming_allocation)
                if free < self.transition_watermark:
                    self._require_hot(group, "watermark")
                elif residents >= self.hot_config.resident_window_pages:
                    self._require_hot(group, "window")
            if tables.hot_required and not tables.blocks and not tables.busy:
                with suppress(CapacityError):
                    self.transition_to_host(*group)
            self._unpin_clean_pages(group)

    def transition_to_host(self, request_id, layer):
        self.storage.check_stream()
        group = (request_id, layer)
        tables = self.tables[group]
        if tables.blocks:
            return
        self._require_hot(group, "explicit")
        if tables.busy:
            raise CapacityError("cannot transition an active row lease")
        self._publish_clean()
        free = self._available_blocks()
        victims = [
            p for p in self._historical_pages(group)
            if p.host_committed_version == p.content_version and p.slot not in free
        ]
        needed = max(0, self.hot_blocks - len(free))
        if len(victims) < needed:
            raise CapacityError("cannot acquire complete hot region while blocks are leased")
        for page in victims[:needed]:
            free.append(page.slot)
            self.allocator.unpin(page.slot, self._on_block_reused)
            self.storage.stats["clean_page_unpins"] += 1
        blocks = free[: self.hot_blocks]
        for i, block in enumerate(blocks):
            self._take_block(block)
            self.storage.wait(self.storage.transfer, self.allocator.slots[block].fence)
            self.allocator.bind(block, (request_id, layer, -i - 1))
        tables.blocks = blocks
        self._awaiting.discard(group)
        self._file(group)  # bookkeeping only; the sweeps here ignore it
        tables.hot.copy_(torch.tensor(blocks, dtype=torch.int32, device=self.device))
        tables.ready = self.storage.event(self.storage.transfer)
        self.storage.stats["hot_region_allocations"] += 1
        self._unpin_clean_pages(group)

    def _slot(self):
        while True:
            self.update_residency(upcoming_allocation=True)
            for group in self.tables:
                self._unpin_clean_pages(group)
            free = self._available_blocks()
            if free:
                return self._take_block(free[0])
            candidates = self._historical_pages()
            pending = [p for p in candidates if p.host_committed_version < p.content_version and p.host_ready is not None]
            for group, count in Counter(p.key[:2] for p in candidates).most_common():
                if count >= self.hot_blocks + 1 and not self.tables[group].blocks:
                    self._require_hot(group, "pressure")
                    try:
                        self.transition_to_host(*group)
                    except CapacityError:
                        continue
                    free = self._available_blocks()
                    if free:
                        return self._take_block(free[0])
            if not pending:
                raise CapacityError("no reclaimable resident block; tails/readers are protected")
            pending[0].host_ready.synchronize()
            self.storage.stats["pressure_mirror_waits"] += 1
