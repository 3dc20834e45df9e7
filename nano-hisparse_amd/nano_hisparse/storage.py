"""Logical pages with pinned host backing, append mirrors and retirement.

Reference: nano_hisparse/storage.py:23-456. A request reserves host credits
for `ceil(max_tokens / page_size)` pages per layer. Appending K/V writes the
rows into the page's resident device block, updates the page's Quest bounds
(per-element min/max of its keys, in the KV dtype) and mean key (fp32), and
mirrors the new rows to the page's host block on the transfer stream. Events
order the compute stream (appends, attention) against the transfer stream
(mirrors, gathers); reference counts decide when blocks and host slots may be
reused. The store knows no residency policy: callers place pages.
"""

from __future__ import annotations

import contextlib

from collections import Counter
from contextlib import nullcontext
from dataclasses import dataclass, field
from enum import Enum
from math import ceil

import torch

from .allocator import DeviceAllocator
from .config import CacheConfig, CapacityError


def upload(values, dtype, device):
    """A host list as a tensor on `device`, enqueued on the current stream
    from pinned memory: a copy from pageable memory would block the host
    until the device's queue drains."""
    host = torch.tensor(values, dtype=dtype)
    if torch.device(device).type != "cuda":
        return host.to(device)
    return host.pin_memory().to(device, non_blocking=True)

PageKey = tuple  # (request_id, layer, page index)


class Location(str, Enum):
    HOST = "host"
    RESIDENT = "resident"


@dataclass
class Page:
    key: PageKey
    host_slot: int
    slot: int | None = None
    location: Location = Location.HOST
    valid_tokens: int = 0
    pins: int = 0
    ready: object = None  # compute-stream event: device contents written
    last_use: object = None  # compute-stream event: last reader done
    host_ready: object = None  # event after which the host mirror is written (the append kernel's on a GPU)
    content_version: int = 0
    host_enqueued_version: int = 0
    host_committed_version: int = 0
    sealed: bool = False


@dataclass
class RequestPages:
    max_tokens: int
    layers: int
    page_count: int
    lengths: list
    summaries: torch.Tensor  # [layers, pages, kv_heads, head_dim] fp32 mean key
    minimum: torch.Tensor  # [layers, pages, kv_heads, head_dim] KV dtype
    maximum: torch.Tensor
    host_credits: int
    keys: list = field(default_factory=list)
    extra_index_bytes: int = 0
    keepalive: tuple = ()


class PageLease:
    """Reader references on pages' blocks (and extra blocks) for one use.

    Construction takes a block reference per page and per extra slot and a
    reader pin per page; release() records a compute-stream event as every
    page's last use and returns the references.
    """

    def __init__(self, store: "HostStore", pages, *, extra_slots=()):
        store.check_stream()
        for p in pages:
            live = store.pages.get(p.key) is p and p.slot is not None
            if not live or store.allocator.slots[p.slot].owner != p.key:
                raise RuntimeError("cannot reference a detached or retired page")
        slots = [p.slot for p in pages] + list(extra_slots)
        if any(store.allocator.slots[s].owner is None for s in slots):
            raise RuntimeError("cannot reference an unbound block")
        self.store, self.pages, self.slots = store, list(pages), slots
        self.released, self.done = False, None
        for s in slots:
            store.allocator.incref(s)
        for p in self.pages:
            p.pins += 1
            store.pinned.add(p.key)

    def _validate(self):
        self.store.check_stream()
        if self.released:
            raise RuntimeError("lease already released")

    def wait(self):
        self._validate()
        for p in self.pages:
            self.store.wait(self.store.compute, p.ready)

    def release(self):
        self._validate()
        self.done = self.store.event(self.store.compute)
        for p in self.pages:
            p.last_use = self.done
            p.pins -= 1
            if not p.pins:
                self.store.pinned.discard(p.key)
        for s in self.slots:
            self.store.allocator.decref(s)
        self.released = True
        self.store.notify(self.pages)

    def __enter__(self):
        self.wait()
        return self

    def __exit__(self, *exc):
        self.release()


class HostStore:
    def __init__(self, config: CacheConfig, allocator: DeviceAllocator):
        self.config = config
        self.allocator = allocator
        self.pool = allocator.storage
        self.device = self.pool.device
        self.cuda = self.device.type == "cuda"
        if self.cuda and not torch.cuda.is_available():
            raise RuntimeError("CUDA unavailable; use device='cpu' for the reference path")
        shape = (config.host_pages, 2, config.page_size, config.kv_heads, config.head_dim)
        self.host = torch.empty(shape, dtype=config.dtype, pin_memory=self.cuda)
        self.host_alias = None
        if self.cuda:
            from .row_kernels import MappedHost

            self.host_alias = MappedHost(self.host)
        self.compute = torch.cuda.current_stream(self.device) if self.cuda else None
        self._capture_stream = None
        self.transfer = torch.cuda.Stream(device=self.device) if self.cuda else None
        self.pages: dict = {}
        self.group_pages: dict = {}  # (request_id, layer) -> pages in index order
        self.resident_pages: Counter = Counter()  # (request_id, layer) -> pages holding a block
        # (request_id, layer) -> compute event of the last batched read of the
        # layer's pages (a batched step fences reuse per layer, not per page)
        self.layer_reads: dict = {}
        # called with each page that lost its readers or published its host
        # mirror (a residency policy's unpin candidates)
        self.listener = None
        self.requests: dict = {}
        self.free_host = list(range(config.host_pages - 1, -1, -1))
        self.stats: Counter = Counter()
        self.pinned: set = set()
        self.retired: list = []  # (event, request, pages)

    # ---- views ------------------------------------------------------------------

    @property
    def budget(self):
        return self.allocator.budget

    @property
    def owners(self):
        return [slot.owner for slot in self.allocator.slots]

    @property
    def page_bytes(self):
        return self.pool[0].numel() * self.pool.element_size()

    @property
    def index_bytes(self):
        live = list(self.requests.values()) + [r for _, r, _ in self.retired]
        tensors = sum(
            t.numel() * t.element_size() for r in live for t in (r.summaries, r.minimum, r.maximum)
        )
        return tensors + sum(r.extra_index_bytes for r in live)

    def index_reservation_bytes(self, max_tokens, layers):
        cfg = self.config
        per_page = cfg.kv_heads * cfg.head_dim * (4 + 2 * self.pool.element_size())
        return ceil(max_tokens / cfg.page_size) * layers * per_page

    @property
    def available_host_credits(self):
        return len(self.free_host) - sum(r.host_credits for r in self.requests.values())

    # ---- streams and events ---------------------------------------------------------

    def context(self, stream):
        return torch.cuda.stream(stream) if self.cuda else nullcontext()

    def event(self, stream):
        """A recorded event; `.stream` names the stream it completes in order on."""
        if not self.cuda:
            return None
        ev = torch.cuda.Event()
        ev.record(stream)
        ev.stream = stream
        return ev

    def notify(self, pages):
        if self.listener is not None:
            for page in pages:
                self.listener(page)

    def wait(self, stream, event):
        if event is not None:
            stream.wait_event(event)

    def active_compute(self):
        """The stream cache work runs on now: the capture stream while a
        graph is being captured (capturing()), else the compute stream."""
        return self._capture_stream if self._capture_stream is not None else self.compute

    def check_stream(self):
        if self.cuda and torch.cuda.current_stream(self.device) not in (self.compute, self._capture_stream):
            raise RuntimeError("cache operations must use the construction compute stream")

    @contextlib.contextmanager
    def capturing(self, stream):
        """Within: cache operations may also run on `stream`, whose launches
        are being captured into a graph that is replayed on the compute
        stream (so the stream order of cache work is unchanged)."""
        previous, self._capture_stream = self._capture_stream, stream
        try:
            yield
        finally:
            self._capture_stream = previous

    def synchronize(self):
        if self.cuda:
            self.compute.synchronize()
            self.transfer.synchronize()

    # ---- request lifetime ---------------------------------------------------------------

    def reserve(self, request_id, max_tokens, layers, *, extra_index_bytes=0):
        """Reserve host backing and index bytes for the admitted lifetime."""
        self.check_stream()
        self.collect()
        if request_id in self.requests:
            raise ValueError(f"duplicate request {request_id}")
        if max_tokens < 1 or layers < 1:
            raise ValueError("max_tokens and layers must be positive")
        cfg = self.config
        n = ceil(max_tokens / cfg.page_size)
        if n * layers > self.available_host_credits:
            raise CapacityError(f"need {n * layers} host credits; have {self.available_host_credits}")
        need = self.index_reservation_bytes(max_tokens, layers) + extra_index_bytes
        if self.index_bytes + need > cfg.index_budget_bytes:
            raise CapacityError("GPU index budget exhausted; defer request admission")
        shape = (layers, n, cfg.kv_heads, cfg.head_dim)
        summaries = torch.zeros(shape, device=self.device, dtype=torch.float32)
        # bounds are extrema of actual keys, exactly representable in the KV dtype
        minimum = torch.full(shape, torch.inf, device=self.device, dtype=cfg.dtype)
        maximum = torch.full(shape, -torch.inf, device=self.device, dtype=cfg.dtype)
        request = RequestPages(max_tokens, layers, n, [0] * layers, summaries, minimum, maximum, n * layers)
        request.extra_index_bytes = extra_index_bytes
        self.requests[request_id] = request

    def materialize(self, request_id, layer, index):
        key = (request_id, layer, index)
        page = self.pages.get(key)
        if page is None:
            request = self.requests[request_id]
            assert request.host_credits > 0 and self.free_host
            request.host_credits -= 1
            request.keys.append(key)
            page = self.pages[key] = Page(key, self.free_host.pop())
            self.group_pages.setdefault(key[:2], []).append(page)
            self.stats["materialized_pages"] += 1
        return page

    def _unmaterialize(self, page: Page):
        """Undo materialize() of a page that never held data."""
        key = page.key
        assert page.slot is None and page.valid_tokens == 0 and self.pages[key] is page
        request = self.requests[key[0]]
        del self.pages[key]
        self.group_pages[key[:2]].remove(page)
        request.keys.remove(key)
        request.host_credits += 1
        self.free_host.append(page.host_slot)
        self.stats["materialized_pages"] -= 1

    def detach(self, page: Page):
        """Drop a page's device block; reuse of the block waits on its events."""
        assert self.pages.get(page.key) is page
        assert page.slot is not None and page.pins == 0
        assert page.host_enqueued_version == page.content_version
        for ev in (page.ready, page.last_use, page.host_ready, self.layer_reads.get(page.key[:2])):
            self.wait(self.transfer, ev)
        self.allocator.release(page.slot, self.event(self.transfer))
        page.slot, page.location = None, Location.HOST
        self.resident_pages[page.key[:2]] -= 1
        self.stats["evictions"] += 1

    def bind(self, page: Page, slot, location):
        page.slot, page.location, page.last_use = slot, location, None
        self.allocator.bind(slot, page.key)
        self.resident_pages[page.key[:2]] += 1
        self.stats["peak_device_pages"] = max(self.stats["peak_device_pages"], len(self.allocator.lru))

    @torch.inference_mode()
    def append(self, request_id, layer, k, v, prepare_page, after_write=None):
        """Append K/V rows [tokens, kv_heads, head_dim] to one layer.

        prepare_page(page) places the page (and may return a read lease on
        an existing tail); after_write(page) runs once the page's mirror is
        enqueued. The store never chooses a victim itself.
        """
        self.check_stream()
        request = self.requests[request_id]
        cfg = self.config
        if not 0 <= layer < request.layers:
            raise ValueError("invalid layer")
        expected = (cfg.kv_heads, cfg.head_dim)
        if k.ndim != 3 or k.shape != v.shape or tuple(k.shape[1:]) != expected:
            raise ValueError(f"expected matching [tokens, {expected[0]}, {expected[1]}] K/V")
        if k.device != self.pool.device or v.device != self.pool.device:
            raise ValueError("K/V must be on the cache device")
        if k.dtype != cfg.dtype or v.dtype != cfg.dtype:
            raise ValueError("K/V dtype must match the cache")
        start = request.lengths[layer]
        if start + len(k) > request.max_tokens:
            raise CapacityError("request exceeds its reserved host capacity")
        if any(key[0] == request_id and key[1] == layer for key in self.pinned):
            raise RuntimeError("cannot append while this layer has active attention leases")
        if len(self.pinned) >= self.budget:
            raise CapacityError("no slot available for append")
        P = cfg.page_size
        appender = None
        if self.cuda:
            from .row_kernels import PageAppender

            # one kernel per page: pool rows, host mirror rows, bounds and summary
            appender = PageAppender(k.contiguous(), v.contiguous(), self.pool, self.host_alias, request.summaries,
                                    request.minimum, request.maximum)
        done = 0
        while done < len(k):
            index, within = divmod(start + done, P)
            count = min(P - within, len(k) - done)
            fresh = (request_id, layer, index) not in self.pages
            page = self.materialize(request_id, layer, index)
            try:
                lease = prepare_page(page)
            except Exception:
                if fresh:  # a failed placement leaves no empty page behind
                    self._unmaterialize(page)
                raise
            if lease is not None:
                lease.wait()
            for ev in (page.ready, page.last_use, page.host_ready):
                self.wait(self.compute, ev)  # earlier readers and mirrors of this page
            page.valid_tokens = within + count
            page.content_version += 1
            page.sealed = page.valid_tokens == P
            page.location = Location.RESIDENT
            if appender is not None:
                appender(done, count, page.slot, within, page.host_slot, layer * request.page_count + index)
                page.ready = self.event(self.compute)
                page.host_ready = page.ready
                page.host_enqueued_version = page.content_version
            else:
                block = self.pool[page.slot]
                block[0, within : within + count].copy_(k[done : done + count])
                block[1, within : within + count].copy_(v[done : done + count])
                self._update_bounds(request, layer, index, block, within, count)
                page.ready = self.event(self.compute)
                self._mirror(page, block, within, count)
            self.stats["d2h_bytes"] += self.page_bytes * count // P
            if lease is not None:
                lease.release()
            done += count
            request.lengths[layer] = start + done  # pages written so far stay counted if a later one fails
            if after_write is not None:
                after_write(page)

    def _update_bounds(self, request, layer, index, block, within, count):
        """Page mean key (fp32) and running min/max of the new keys
        (reference storage.py:302-309); CPU caches only (a GPU cache does
        this inside nhs_append_page)."""
        valid = within + count
        request.summaries[layer, index].copy_(block[0, :valid].float().mean(0))
        new_keys = block[0, within:valid].float()
        lo, hi = request.minimum[layer, index], request.maximum[layer, index]
        lo.copy_(torch.minimum(lo, new_keys.amin(0)))
        hi.copy_(torch.maximum(hi, new_keys.amax(0)))

    def _mirror(self, page, block, within, count):
        """Copy the new rows to the page's host block (CPU caches; a GPU
        cache writes them inside nhs_append_page)."""
        self.wait(self.transfer, page.ready)
        with self.context(self.transfer):
            if within == 0 and count == self.config.page_size:
                self.host[page.host_slot].copy_(block, non_blocking=self.cuda)
            else:
                for plane in (0, 1):
                    rows = slice(within, within + count)
                    self.host[page.host_slot, plane, rows].copy_(block[plane, rows], non_blocking=self.cuda)
        page.host_ready = self.event(self.transfer)
        page.host_enqueued_version = page.content_version
        if not self.cuda:
            page.host_committed_version = page.content_version

    def retire(self, request_id, *, keepalive=()):
        self.check_stream()
        request = self.requests[request_id]
        if any(self.pages[key].pins for key in request.keys):
            raise RuntimeError("cannot free a request with active leases")
        retired, waited = [], set()
        for key in request.keys:
            page = self.pages[key]
            assert page.slot is None, "detach resident blocks before retiring host backing"
            for ev in (page.ready, page.last_use, page.host_ready):
                if ev is not None and id(ev) not in waited:  # pages of a batched step share events
                    waited.add(id(ev))
                    self.wait(self.transfer, ev)
            retired.append(self.pages.pop(key))
        del self.requests[request_id]
        for layer in range(request.layers):
            self.group_pages.pop((request_id, layer), None)
            self.resident_pages.pop((request_id, layer), None)
            self.wait(self.transfer, self.layer_reads.pop((request_id, layer), None))
        request.keepalive = tuple(keepalive)
        done = self.event(self.transfer)
        self.retired.append((done, request, retired))
        self.stats["retired_requests"] += 1
        return done

    def collect(self, wait=False):
        """Return host slots of retired requests whose users have finished.

        Polling never blocks; wait=True drains the retirement events.
        """
        still = []
        for ev, request, pages in self.retired:
            if wait and ev is not None:
                ev.synchronize()
            if ev is None or ev.query():
                self.free_host.extend(p.host_slot for p in pages)
                self.stats["reclaimed_requests"] += 1
            else:
                still.append((ev, request, pages))
        self.retired = still

    # ---- introspection ------------------------------------------------------------------

    def page_state(self, key):
        page = self.pages[key]
        backup_pending = page.host_ready is not None and not page.host_ready.query()
        if not backup_pending and page.host_committed_version != page.host_enqueued_version:
            page.host_committed_version = page.host_enqueued_version
            self.notify((page,))
        return {
            "location": page.location.value,
            "loading": page.ready is not None and not page.ready.query(),
            "backup_pending": backup_pending,
            "content_version": page.content_version,
            "host_committed_version": page.host_committed_version,
            "sealed": page.sealed,
            "reader_refs": page.pins,
            "ref_cnt": self.allocator.slots[page.slot].ref_cnt if page.slot is not None else None,
        }

    def host_kv(self, request_id, layer):
        """Blocking diagnostic read of one layer's K and V from host memory."""
        self.synchronize()
        request = self.requests[request_id]
        n = ceil(request.lengths[layer] / self.config.page_size)
        if n == 0:
            raise ValueError("layer has no KV")
        chunks = []
        for i in range(n):
            page = self.pages[(request_id, layer, i)]
            chunks.append(self.host[page.host_slot, :, : page.valid_tokens])
        kv = torch.cat(chunks, dim=1)
        return kv[0], kv[1]

    def snapshot(self):
        locations = Counter(p.location.value for p in self.pages.values() if p.valid_tokens)
        return {
            "budget_pages": self.budget,
            # the pool's whole allocation, its blocks' padding included (row_kernels.padded_pool)
            "allocated_device_bytes": self.pool.untyped_storage().nbytes(),
            "allocated_host_bytes": self.host.numel() * self.host.element_size(),
            "index_bytes": self.index_bytes,
            "index_budget_bytes": self.config.index_budget_bytes,
            "host_materialized_pages": len(self.pages),
            "host_unused_credits": sum(r.host_credits for r in self.requests.values()),
            "host_available_credits": self.available_host_credits,
            "retiring_requests": len(self.retired),
            "request_device_pages": dict(self.allocator.occupancy),
            "locations": dict(locations),
            "stats": dict(self.stats),
        }

    def assert_invariants(self):
        owners = self.owners
        occupied = [k for k in owners if k is not None]
        assert len(occupied) == len(set(occupied))
        assert all(k is None for k in owners[self.budget :])
        retired_pages = [p for _, _, pages in self.retired for p in pages]
        assert len(self.free_host) + len(self.pages) + len(retired_pages) == self.config.host_pages
        slots = [p.host_slot for p in list(self.pages.values()) + retired_pages]
        assert len(set(slots + self.free_host)) == self.config.host_pages
        assert self.available_host_credits >= 0
        assert self.pinned == {p.key for p in self.pages.values() if p.pins}
        assert set(self.allocator.lru) == set(occupied)
        by_group = {}
        for key, slot in self.allocator.lru.items():
            by_group.setdefault(key[:2], []).append((key, slot))
        assert {g: list(b.items()) for g, b in self.allocator.group_blocks.items()} == by_group
        assert self.allocator.referenced_unpinned == sum(
            1 for s in self.allocator.reclaimable if self.allocator.slots[s].ref_cnt
        )
        assert +self.resident_pages == Counter(p.key[:2] for p in self.pages.values() if p.slot is not None)
        assert self.allocator.free == {i for i, k in enumerate(owners) if k is None}
        assert +self.allocator.occupancy == Counter(k[0] for k in occupied)
        for slot in self.allocator.slots:
            assert slot.ref_cnt >= 0
            if slot.owner is None:
                assert slot.ref_cnt == 0
        assert self.index_bytes <= self.config.index_budget_bytes
        for request in self.requests.values():
            assert len(request.keys) + request.host_credits == request.layers * request.page_count
        for key, page in self.pages.items():
            assert page.pins >= 0 and 0 <= page.valid_tokens <= self.config.page_size
            if page.slot is None:
                assert page.location == Location.HOST
            else:
                assert owners[page.slot] == key and page.location == Location.RESIDENT
                alloc = int(page.slot not in self.allocator.reclaimable)
                assert self.allocator.slots[page.slot].ref_cnt == alloc + page.pins
            assert page.pins == 0 or page.slot is not None
            assert page.host_committed_version <= page.host_enqueued_version == page.content_version
