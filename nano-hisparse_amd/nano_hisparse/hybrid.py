"""Hybrid KV cache: resident pages and per-layer hot rows in one device pool.

Reference: nano_hisparse/hybrid.py:19-594. Every (request, layer) admitted
reserves credits for a hot region of ceil(hot_rows / page_size) blocks and
two active tail blocks; resident history borrows the remaining blocks until
pressure (free-block watermark, resident window, or an allocation that
cannot be served) makes the layer allocate its whole hot region and turn
history into host-backed pages that stay readable until their block is
reused. Attention resolves selected token positions to physical rows
(libnhs_hip.so resolver), gathers missed rows from pinned host memory into
hot rows on the transfer stream (libnhs_hip.so gather) and runs row
attention on the compute stream; events order the two streams.

The policy makes the reference's decisions in the reference's order, but
visits only the layers that can act: a layer is "dirty" from the moment one
of its pages may have become unpinnable (a mirror published, readers gone,
a page sealed or pushed out of the active tails, a hot region bound) until
its clean history is unpinned, and a layer "awaits" a hot region until it
has one. A policy tick sweeps dirty and awaiting layers in admission order;
every other layer would be a no-op in a full sweep. Allocatable blocks come
from the allocator's indexes, and finished mirrors are found by querying
pending events in recording order, stopping at the first incomplete event
of each stream.
"""

from __future__ import annotations

import bisect
import heapq
from collections import Counter
from contextlib import suppress
from dataclasses import dataclass, field
from math import ceil

import torch

from .allocator import DeviceAllocator
from .config import CapacityError
from .row_index import LogicalTopK, resolve_rows
from .storage import HostStore, Location, PageLease, upload

ACTIVE_TAIL_PAGES = 2


@dataclass(frozen=True)
class HotConfig:
    """max_union_rows bounds the distinct rows one selection may name (U);
    hot_rows (H, default 2U) is the per-layer hot row count, U <= H <= 32768."""

    max_union_rows: int
    hot_rows: int | None = None
    resident_window_pages: int = 64
    transition_watermark: int | None = None

    def __post_init__(self):
        if self.max_union_rows < 1:
            raise ValueError("max_union_rows must be positive")
        if self.hot_rows is None:
            object.__setattr__(self, "hot_rows", 2 * self.max_union_rows)
        if not self.max_union_rows <= self.hot_rows <= 32768:
            raise ValueError("hot_rows must cover max_union_rows and be <= 32768")
        if self.resident_window_pages < ACTIVE_TAIL_PAGES:
            raise ValueError("resident window must cover both active tail pages")
        if self.transition_watermark is not None and self.transition_watermark < 0:
            raise ValueError("transition watermark must be nonnegative")

    def admission_blocks(self, page_size, layers=1):
        return layers * (ceil(self.hot_rows / page_size) + ACTIVE_TAIL_PAGES)


@dataclass
class LayerTables:
    """Device tables of one (request, layer): page -> host page, page ->
    resident block, hot block table, hot row tags (host rows) and LRU order."""

    source: torch.Tensor
    resident: torch.Tensor
    hot: torch.Tensor
    tags: torch.Tensor
    lru: torch.Tensor
    blocks: list = field(default_factory=list)
    ready: object = None
    last_use: object = None
    busy: bool = False
    hot_required: bool = False
    trigger: str | None = None

    @property
    def nbytes(self):
        return sum(t.numel() * t.element_size() for t in (self.source, self.resident, self.hot, self.tags, self.lru))


class RowLease(PageLease):
    """Reader lease over a layer's resident pages and hot blocks; holds the
    resolved RowPlan in `.plan` and marks the layer's hot rows busy."""

    def __init__(self, cache, tables, pages):
        super().__init__(cache.storage, pages, extra_slots=tables.blocks)
        self.tables, self.plan = tables, None
        tables.busy = True

    def wait(self):
        self._validate()
        self.store.wait(self.store.compute, self.tables.ready)

    def release(self):
        super().release()
        self.tables.last_use = self.done
        self.tables.busy = False


class _OrderedKeys(dict):
    """Insertion-ordered set; re-adding a key moves it to the end."""

    def add(self, key):
        self.pop(key, None)
        self[key] = None

    def discard(self, key):
        self.pop(key, None)


def store_entry(table, index, value):
    """Write one entry of a device table on the current stream as a
    one-element fill (the value travels as a kernel argument; indexed
    assignment of a Python number costs about three times the host time)."""
    table[index : index + 1].fill_(value)


class HybridKVCache:
    def __init__(self, config, hot: HotConfig):
        if config.host_pages * config.page_size >= 2**31:
            raise ValueError("host row tags require int32 addresses")
        self.config = config
        self.hot_config = hot
        self.hot_blocks = ceil(hot.hot_rows / config.page_size)
        self.tables: dict = {}
        self.pending_clean = _OrderedKeys()  # pages whose host mirror is in flight
        self._writing_key = None
        self._rank: dict = {}  # (request, layer) -> admission order
        self._next_rank = 0
        self._dirty: set = set()  # layers that may hold unpinnable clean history
        self._awaiting: set = set()  # layers without a hot region
        # awaiting layers holding resident pages: "active" ones may act at any
        # tick (hot region demanded, or the resident window reached);
        # "dormant" ones act only while allocatable blocks are below the
        # transition watermark
        self._awaiting_active: set = set()
        self._dormant: set = set()
        self._sweep = None  # (heap, rank cursor, group filter) while a tick runs
        self._item_tables: dict = {}  # batch composition -> device nhs_layer_item table
        self.allocator = DeviceAllocator(config)
        self.storage = HostStore(config, self.allocator)
        self.storage.listener = self._candidate
        self.pool, self.device = self.allocator.storage, self.storage.device
        self.row_stats = torch.zeros(3, dtype=torch.int64, device=self.device)
        self._host_pointer = self.storage.host_alias

    # ---- capacity ---------------------------------------------------------------------

    @property
    def index_bytes(self):
        return self.storage.index_bytes

    @property
    def budget(self):
        return self.allocator.budget

    @property
    def owners(self):
        return self.storage.owners

    def index_reservation_bytes(self, max_tokens, layers):
        tables = ceil(max_tokens / self.config.page_size) * 8 + self.hot_blocks * 4 + self.hot_config.hot_rows * 12
        return self.storage.index_reservation_bytes(max_tokens, layers) + layers * tables

    def admission_blocks(self, layers):
        return self.hot_config.admission_blocks(self.config.page_size, layers)

    @property
    def transition_watermark(self):
        configured = self.hot_config.transition_watermark
        return max(self.hot_blocks, self.budget // 10) if configured is None else configured

    def _available_blocks(self, count=None):
        """Allocatable blocks: empty ones first (ascending), then readable
        unpinned blocks nobody references, in the order they were unpinned
        (the first `count` of them)."""
        return self.allocator.available(count)

    def _take_block(self, slot):
        if slot in self.allocator.reclaimable:
            self.allocator.reclaim(slot)
        return slot

    def _on_block_reused(self, slot):
        page = self.storage.pages[self.allocator.slots[slot].owner]
        assert self.allocator.slots[slot].ref_cnt == 0
        assert page.host_committed_version == page.content_version
        self._detach(page)
        self.storage.stats["unpinned_block_reuses"] += 1

    # ---- admission ----------------------------------------------------------------------

    def reserve(self, request_id, max_tokens, layers):
        self.collect()
        promised = sum(self.admission_blocks(r.layers) for r in self.storage.requests.values())
        if promised + self.admission_blocks(layers) > self.budget:
            raise CapacityError("hot-region + active-tail credits exhausted; defer admission")
        extra = self.index_reservation_bytes(max_tokens, layers) - self.storage.index_reservation_bytes(
            max_tokens, layers
        )
        self.storage.reserve(request_id, max_tokens, layers, extra_index_bytes=extra)
        n = self.storage.requests[request_id].page_count
        H = self.hot_config.hot_rows

        def unset(size):
            return torch.full((size,), -1, dtype=torch.int32, device=self.device)

        for layer in range(layers):
            group = (request_id, layer)
            self.tables[group] = LayerTables(
                unset(n), unset(n), unset(self.hot_blocks), unset(H),
                torch.arange(H, dtype=torch.int64, device=self.device),
            )
            self._rank[group] = self._next_rank
            self._next_rank += 1
            self._awaiting.add(group)

    # ---- policy bookkeeping ----------------------------------------------------------------

    def _mark(self, group):
        """A page of `group` may have become unpinnable."""
        if group not in self.tables:
            return
        self._dirty.add(group)
        sweep = self._sweep
        if sweep is not None and self._rank[group] > sweep[1] and sweep[2](group):
            heapq.heappush(sweep[0], (self._rank[group], group))

    def _candidate(self, page):
        """Marks the page's layer if the page now meets every unpin condition
        but the hot region (sealed, clean, pinned, past the active tails)."""
        group = page.key[:2]
        if (
            group in self.tables
            and page.sealed
            and page.slot is not None
            and page.host_committed_version == page.content_version
            and page.slot not in self.allocator.reclaimable
            and page.key[2] <= self._tail_index(group) - ACTIVE_TAIL_PAGES
        ):
            self._mark(group)

    def _in_order(self, groups):
        return sorted(groups, key=self._rank.__getitem__)

    def _selector(self, request_id, layer):
        if request_id is None and layer is None:
            return lambda g: True
        return lambda g: (request_id is None or g[0] == request_id) and (layer is None or g[1] == layer)

    # ---- placement ----------------------------------------------------------------------

    def _prepare_append(self, page):
        self._writing_key = page.key
        if not page.valid_tokens:  # a new page: the active tails move on
            self._mark(page.key[:2])
        if page.valid_tokens:  # appending to an existing tail page
            if page.slot is None:
                raise RuntimeError("active append tail lost its resident lease")
            self.storage.stats["resident_hits"] += 1
            self.storage.stats["append_resident_hits"] += 1
            return PageLease(self.storage, [page])
        slot = self._slot()
        store_entry(self.tables[page.key[:2]].source, page.key[2], page.host_slot)
        self.storage.wait(self.storage.compute, self.allocator.slots[slot].fence)
        self._bind(page, slot, Location.RESIDENT)
        return None

    def _bind(self, page, slot, location):
        self.storage.bind(page, slot, location)
        group = page.key[:2]
        store_entry(self.tables[group].resident, page.key[2], slot)
        if group in self._awaiting:
            self._file(group)

    def _detach(self, page):
        self.storage.detach(page)
        group = page.key[:2]
        store_entry(self.tables[group].resident, page.key[2], -1)
        if group in self._awaiting:
            self._file(group)

    def _file(self, group):
        """Re-file an awaiting layer as active, dormant or neither (no
        resident pages) after its residents or hot-region demand changed."""
        self._awaiting_active.discard(group)
        self._dormant.discard(group)
        residents = self.storage.resident_pages[group]
        if group not in self._awaiting or not residents:
            return
        if self.tables[group].hot_required or residents >= self.hot_config.resident_window_pages:
            self._awaiting_active.add(group)
        else:
            self._dormant.add(group)

    def _tail_index(self, group):
        """Last page of a layer's history (the page being written, if any)."""
        if self._writing_key is not None and self._writing_key[:2] == group:
            return self._writing_key[2]
        length = self.storage.requests[group[0]].lengths[group[1]]
        return (length - 1) // self.config.page_size

    def _historical_pages(self, group=None):
        """Sealed resident pages older than the two active tails whose block
        only carries its allocation reference, in block-binding order."""
        alloc, pages = self.allocator, self.storage.pages
        tails = {}
        out = []
        for key in alloc.lru if group is None else alloc.group_keys(group):
            if key[2] < 0:  # a hot block, not a KV page
                continue
            if group is not None and key[:2] != group:
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
        """Publish every pending mirror whose event has completed. Events of
        one stream complete in recording order and pending pages are kept in
        that order, so a stream's first incomplete event ends its queries."""
        blocked = set()
        for key in list(self.pending_clean):
            page = self.storage.pages.get(key)
            if page is None:
                self.pending_clean.discard(key)
                continue
            event = page.host_ready
            stream = getattr(event, "stream", None)
            if stream is not None and stream in blocked:
                continue
            if event is None or event.query():
                page.host_committed_version = page.host_enqueued_version
                self.pending_clean.discard(key)
                self.storage.stats["host_mirror_completions"] += 1
                self._candidate(page)
            elif stream is not None:
                blocked.add(stream)

    def _unpin_clean_pages(self, group):
        """Once a layer has its hot region, its clean history gives up the
        allocation reference (newest page first) and stays readable. Only
        the layer's still-pinned pages can qualify (historical, clean, not
        yet unpinned), so only those are checked."""
        self._dirty.discard(group)
        if not self.tables[group].blocks:
            return
        pinned = self.allocator.pinned_pages(group)
        if not pinned:
            return
        pages, slots = self.storage.pages, self.allocator.slots
        last = self._tail_index(group) - ACTIVE_TAIL_PAGES
        ready = []
        for key, slot in pinned.items():
            page = pages[key]
            if (key[2] <= last and page.sealed and slots[slot].ref_cnt == 1
                    and page.host_committed_version == page.content_version):
                ready.append(page)
        ready.sort(key=lambda p: -p.key[2])
        for page in ready:
            self.allocator.unpin(page.slot, self._on_block_reused)
            self.storage.stats["clean_page_unpins"] += 1

    def _require_hot(self, group, reason):
        tables = self.tables[group]
        if not tables.hot_required:
            tables.hot_required, tables.trigger = True, reason
            self.storage.stats[f"hot_trigger_{reason}"] += 1
            if group in self._awaiting:
                self._file(group)

    def update_residency(self, request_id=None, layer=None, *, upcoming_allocation=False):
        """Publish finished mirrors and raise or serve hot-region demand,
        without blocking (reference hybrid.py:256-294): first every selected
        layer unpins its clean history, then, layer by layer in admission
        order, hot-region demand is raised and served and the layer unpins
        again. Only layers that can act are visited, in the same order as a
        full sweep: dirty layers and active awaiting ones from a heap;
        dormant layers (awaiting, below the resident window, no demand yet)
        only where allocatable blocks are below the watermark when the sweep
        reaches them, since elsewhere serving one is a no-op. Layers neither
        dirty nor awaiting, or without resident pages, are no-ops too. A
        layer that a later layer's transition makes dirty is still visited
        in this tick if it comes after the one being served."""
        self.storage.check_stream()
        self._publish_clean()
        selected = self._selector(request_id, layer)
        for group in self._in_order([g for g in self._dirty if selected(g)]):
            self._unpin_clean_pages(group)
        rank_of = self._rank
        heap = [(rank_of[g], g) for g in self._awaiting_active | self._dirty if selected(g)]
        heapq.heapify(heap)
        visited = set()
        dormant, at = None, 0  # selected dormant layers in rank order, built on first need
        outer, self._sweep = self._sweep, [heap, -1, selected]
        try:
            while True:
                # dormant layers ranked before the next heap layer (a serve
                # may push one), visited while the sweep is below the watermark
                while self._dormant and self._below_watermark(upcoming_allocation):
                    if dormant is None:
                        dormant = sorted((rank_of[g], g) for g in self._dormant if selected(g))
                        at = bisect.bisect_right(dormant, (self._sweep[1], ()))
                    while at < len(dormant) and dormant[at][1] in visited:
                        at += 1
                    if at == len(dormant) or (heap and dormant[at][0] > heap[0][0]):
                        break
                    rank, group = dormant[at]
                    at += 1
                    if group in self.tables:
                        visited.add(group)
                        self._sweep[1] = rank
                        self._serve(group, upcoming_allocation)
                if not heap:
                    break
                rank, group = heapq.heappop(heap)
                if group in visited or group not in self.tables:
                    continue
                visited.add(group)
                self._sweep[1] = rank
                if dormant is not None:
                    at = bisect.bisect_right(dormant, (rank, ()), at)
                self._serve(group, upcoming_allocation)
        finally:
            self._sweep = outer

    def _below_watermark(self, upcoming_allocation):
        return self.allocator.available_count() - int(upcoming_allocation) < self.transition_watermark

    def _serve(self, group, upcoming_allocation):
        tables = self.tables[group]
        residents = self.storage.resident_pages[group]
        if not residents:
            return
        if not tables.hot_required:
            free = self.allocator.available_count() - int(upcoming_allocation)
            if free < self.transition_watermark:
                self._require_hot(group, "watermark")
            elif residents >= self.hot_config.resident_window_pages:
                self._require_hot(group, "window")
        if tables.hot_required and not tables.blocks and not tables.busy:
            with suppress(CapacityError):  # retried at the next policy tick
                self.transition_to_host(*group)
        self._unpin_clean_pages(group)

    def transition_to_host(self, request_id, layer):
        """Bind the layer's whole hot region at once, then make clean history
        reclaimable (reference hybrid.py:296-331)."""
        self.storage.check_stream()
        group = (request_id, layer)
        tables = self.tables[group]
        if tables.blocks:
            return
        self._require_hot(group, "explicit")
        if tables.busy:
            raise CapacityError("cannot transition an active row lease")
        self._publish_clean()
        free = self._available_blocks(self.hot_blocks)
        needed = self.hot_blocks - len(free)
        if needed:
            # historical pages already unpinned are allocatable, hence in `free`
            victims = [
                p for p in self._historical_pages(group)
                if p.host_committed_version == p.content_version and p.slot not in self.allocator.reclaimable
            ]
            if len(victims) < needed:
                raise CapacityError("cannot acquire complete hot region while blocks are leased")
            for page in victims[:needed]:  # every check precedes every mutation
                free.append(page.slot)
                self.allocator.unpin(page.slot, self._on_block_reused)
                self.storage.stats["clean_page_unpins"] += 1
        blocks = free
        for i, block in enumerate(blocks):
            self._take_block(block)
            self.storage.wait(self.storage.transfer, self.allocator.slots[block].fence)
            self.allocator.bind(block, (request_id, layer, -i - 1))
        tables.blocks = blocks
        self._awaiting.discard(group)
        self._file(group)
        tables.hot.copy_(upload(blocks, torch.int32, self.device))
        tables.ready = self.storage.event(self.storage.transfer)
        self.storage.stats["hot_region_allocations"] += 1
        self._mark(group)
        self._unpin_clean_pages(group)

    def _slot(self):
        """A block for a new page (reference hybrid.py:333-368)."""
        while True:
            self.update_residency(upcoming_allocation=True)
            # a later group's transition may have published an earlier group's
            # mirrors: refresh every group's reclaimable history
            for group in self._in_order(self._dirty):
                self._unpin_clean_pages(group)
            free = self._available_blocks(1)
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
                    free = self._available_blocks(1)
                    if free:
                        return self._take_block(free[0])
            if not pending:
                raise CapacityError("no reclaimable resident block; tails/readers are protected")
            pending[0].host_ready.synchronize()  # one useful mirror, never the device
            self.storage.stats["pressure_mirror_waits"] += 1

    def reclaim_history(self, request_id, layer, *, evict=False):
        """Make finished history allocatable but readable; evict=True also
        revokes the mappings (a diagnostic: pressure does that on reuse)."""
        self.transition_to_host(request_id, layer)
        self._unpin_clean_pages((request_id, layer))
        if evict:
            for page in self._historical_pages((request_id, layer)):
                if page.slot in self.allocator.reclaimable:
                    self._take_block(page.slot)

    def _after_write(self, page):
        self.pending_clean.add(page.key)
        self.update_residency(*page.key[:2])

    def write(self, request_id, layer, k, v):
        if self.tables[request_id, layer].busy:
            raise RuntimeError("cannot append during a row lease")
        try:
            self.storage.append(request_id, layer, k, v, self._prepare_append, self._after_write)
        finally:
            self._writing_key = None

    # ---- the sparse decode path -----------------------------------------------------------

    def attention(self, query, request_id, layer, selection, backend="auto"):
        from .attention import row_attention

        length = self.storage.requests[request_id].lengths[layer]
        if selection.length != length or selection.page_size != self.config.page_size:
            raise ValueError("selection has stale length or wrong page size")
        if selection.heads != query.shape[0]:
            raise ValueError("selection must have one row per query head")
        topk = LogicalTopK.from_selection(selection, query.device)
        return row_attention(query, self, request_id, layer, topk, backend)

    def resolve(self, request_id, layer, topk: LogicalTopK):
        """Resolve `topk` for one layer and gather its misses; returns a
        RowLease whose `.plan` holds the physical rows (reference
        hybrid.py:412-469)."""
        self.storage.check_stream()
        topk.validate(self.device, self.hot_config.max_union_rows)
        tables = self.tables[request_id, layer]
        if tables.busy:
            raise RuntimeError("hot contents already leased by this layer")
        length = self.storage.requests[request_id].lengths[layer]
        if length < 1:
            raise ValueError("cannot resolve an empty history")
        # every resident page of this layer is pinned: which ones are selected
        # is only known on the device
        pages = [p for p in self.storage.group_pages.get((request_id, layer), ()) if p.slot is not None]
        lease = RowLease(self, tables, pages)
        store = self.storage
        try:
            store.wait(store.compute, tables.ready)
            plan = resolve_rows(
                topk, tables.source, tables.resident, tables.hot, tables.tags, tables.lru, length,
                self.config.page_size,
            )
            self.row_stats.add_(plan.counts)
            resolved = store.event(store.compute)
            store.wait(store.transfer, resolved)
            store.wait(store.transfer, tables.last_use)
            # mirrors and earlier spills precede this gather on the one transfer stream
            with store.context(store.transfer):
                if store.cuda:
                    from .row_kernels import gather_rows

                    gather_rows(self._host_pointer, self.pool, plan, self.config)
                else:
                    from .row_kernels import cpu_provider

                    cpu_provider("gather_rows").gather_rows(store.host, self.pool, plan, self.config)
            tables.ready = store.event(store.transfer)
            if store.cuda:  # produced on compute, read on transfer
                plan.miss_host_rows.record_stream(store.transfer)
                plan.miss_device_rows.record_stream(store.transfer)
            lease.plan = plan
            return lease
        except Exception:
            lease.release()
            raise

    # ---- batched decode ---------------------------------------------------------------------

    def decode_batch(self, request_ids, overlap=False, lengths_buffer=None):
        """A BatchDecode step over `request_ids` (one new token each)."""
        from .batched import BatchDecode

        return BatchDecode(self, request_ids, overlap, lengths_buffer)

    def _layer_items(self, request_ids):
        """Device table [layers, B, nhs_layer_item] of the requests' tables,
        cached per batch composition until one of them is released."""
        key = tuple(request_ids)
        items = self._item_tables.get(key)
        if items is None:
            from .row_kernels import layer_items

            store = self.storage
            layers = store.requests[key[0]].layers
            rows = []
            for layer in range(layers):
                row = []
                for rid in key:
                    t, request = self.tables[rid, layer], store.requests[rid]
                    row.append({
                        "source": t.source, "resident": t.resident, "hot": t.hot, "tags": t.tags, "lru": t.lru,
                        "minimum": request.minimum[layer], "maximum": request.maximum[layer],
                        "summaries": request.summaries[layer], "n_pages": request.page_count,
                    })
                rows.append(row)
            if len(self._item_tables) >= 16:
                self._item_tables.pop(next(iter(self._item_tables)))
            items = self._item_tables[key] = layer_items(rows, self.device)
        return items

    # ---- lifetime --------------------------------------------------------------------------

    def release_request(self, request_id, wait=True):
        groups = [t for (name, _), t in self.tables.items() if name == request_id]
        if any(t.busy for t in groups) or any(
            self.storage.pages[key].pins for key in self.storage.requests[request_id].keys
        ):
            raise RuntimeError("cannot release a request with active row leases")
        store = self.storage
        for tables in groups:
            store.wait(store.transfer, tables.ready)
            store.wait(store.transfer, tables.last_use)
            fence = store.event(store.transfer)
            for block in tables.blocks:
                self.allocator.release(block, fence)
        for key in store.requests[request_id].keys:
            page = store.pages[key]
            if page.slot is not None:
                self._detach(page)
        for key in [k for k in self._item_tables if request_id in k]:
            del self._item_tables[key]  # its tensors go with the request
        store.retire(request_id, keepalive=groups)
        for key in [k for k in self.tables if k[0] == request_id]:
            del self.tables[key]
            del self._rank[key]
            self._dirty.discard(key)
            self._awaiting.discard(key)
            self._awaiting_active.discard(key)
            self._dormant.discard(key)
        self.collect(wait=wait)

    def collect(self, wait=False):
        self.storage.collect(wait)
        self.update_residency()

    def page_state(self, key):
        """Dict describing one page (reference hybrid.py:496-507); publishes
        the host mirror's completion when its event has finished."""
        state = self.storage.page_state(key)
        page = self.storage.pages[key]
        unpinned = page.slot in self.allocator.reclaimable
        clean = page.host_committed_version == page.content_version
        if page.slot is None:
            residency = "host_only"
        elif unpinned:
            residency = "clean_unpinned"
        else:
            residency = "clean_pinned" if clean else "dirty"
        state.update(allocation_pinned=page.slot is not None and not unpinned, residency=residency)
        return state

    def set_budget(self, pages):
        if pages != self.budget:
            raise CapacityError("hybrid block budget is fixed; hot leases need readmission to resize")

    def close(self):
        # GPU readers of pinned memory are not visible to torch's allocator:
        # drain at teardown only
        self.storage.synchronize()

    def __del__(self):
        with suppress(RuntimeError, AttributeError, TypeError):
            if getattr(getattr(self, "storage", None), "cuda", False):
                self.close()

    def reset_stats(self):
        self.storage.stats.clear()
        self.row_stats.zero_()

    def snapshot(self):
        result = self.storage.snapshot()
        resident, hot, misses = self.row_stats.cpu().tolist()
        result.update(
            cache_layout="hybrid_rows",
            eviction_policy="resident-reclaim + per-layer row-LRU",
            max_union_rows=self.hot_config.max_union_rows,
            hot_rows=self.hot_config.hot_rows,
            active_tail_pages=ACTIVE_TAIL_PAGES,
            resident_window_pages=self.hot_config.resident_window_pages,
            transition_watermark=self.transition_watermark,
            empty_device_blocks=len(self.allocator.free),
            readable_unpinned_blocks=len(self.allocator.reclaimable),
            allocatable_device_blocks=self.allocator.available_count(),
            pending_clean_pages=len(self.pending_clean),
            hot_pending_groups=sum(t.hot_required and not t.blocks for t in self.tables.values()),
            hot_leased_blocks=sum(len(t.blocks) for t in self.tables.values()),
            admission_block_credits=sum(self.admission_blocks(r.layers) for r in self.storage.requests.values()),
            row_stats={
                "resident_hits": resident,
                "hot_hits": hot,
                "misses": misses,
                "h2d_bytes": misses * self.storage.page_bytes // self.config.page_size,
            },
        )
        return result

    def assert_invariants(self):
        store, alloc = self.storage, self.allocator
        store.assert_invariants()
        assert alloc.available_count() == len(self._available_blocks())
        assert self._awaiting == {g for g, t in self.tables.items() if not t.blocks}
        window = self.hot_config.resident_window_pages
        live = {g for g in self._awaiting if store.resident_pages[g]}
        assert self._awaiting_active == {
            g for g in live if self.tables[g].hot_required or store.resident_pages[g] >= window
        }
        assert self._dormant == live - self._awaiting_active
        assert alloc.group_pinned == {
            g: {k: s for k, s in b.items() if k[2] >= 0 and s not in alloc.reclaimable}
            for g, b in alloc.group_blocks.items()
            if any(k[2] >= 0 and s not in alloc.reclaimable for k, s in b.items())
        }
        assert set(self._rank) == set(self.tables)
        for name, request in store.requests.items():
            assert request.extra_index_bytes == sum(t.nbytes for g, t in self.tables.items() if g[0] == name)
        assert not (alloc.free & alloc.reclaimable.keys())
        for slot in alloc.reclaimable:
            page = store.pages[self.owners[slot]]
            assert page.slot == slot and page.sealed
            assert page.host_committed_version == page.content_version
            assert self.tables[page.key[:2]].blocks
            length = store.requests[page.key[0]].lengths[page.key[1]]
            assert page.key[2] <= (length - 1) // self.config.page_size - ACTIVE_TAIL_PAGES
        assert sum(self.admission_blocks(r.layers) for r in store.requests.values()) <= self.budget
        for group, tables in self.tables.items():
            assert len(tables.blocks) in (0, self.hot_blocks)
            assert sorted(tables.lru.tolist()) == list(range(self.hot_config.hot_rows))
            tags = [t for t in tables.tags.tolist() if t >= 0]
            assert len(tags) == len(set(tags))
            if not tables.blocks:
                assert not tags
            else:
                assert tables.hot_required
            for i, block in enumerate(tables.blocks):
                assert self.owners[block] == (*group, -i - 1)
                assert alloc.slots[block].ref_cnt == 1 + int(tables.busy)
            resident = tables.resident.tolist()
            for index, host in enumerate(tables.source.tolist()):
                page = store.pages.get((*group, index))
                assert host == (-1 if page is None else page.host_slot)
                assert resident[index] == (-1 if page is None or page.slot is None else page.slot)
                if page is not None and page.slot is None:
                    assert tables.blocks
