"""One decode token for a batch of requests, one launch per stage and layer.

The reference decodes request by request (engine.py:111-121, model.py:
182-221): per layer and request an append, a Quest selection, a resolve, a
gather and an attention. BatchDecode runs the same stages for every request
of the batch at once on a GPU cache: per layer one append launch
(nhs_append_items), one Quest scoring launch (nhs_quest_select_items,
scores only), one launch that selects the pages and resolves their rows
(nhs_select_resolve_items; beyond its sizes a selector launch and a
resolver launch, nhs_resolve_items), one gather of the concatenated miss
plans on the transfer stream and one attention launch over all requests'
rows. Each
request keeps its own tables; the kernels read them through a device table
of per-(request, layer) pointers built once per batch composition.

Host bookkeeping stays per request but is O(1) per request and layer.
Every layer's page for the new token is placed when the step starts (the
residency policy, which may reclaim blocks, runs only then and once more at
end()), so no block changes owner between a layer's resolve and its
attention: the step's reads need no per-block reader references and are
fenced per layer (HostStore.layer_reads) for later reuse. That also lets a
caller interleave two steps over disjoint request sets layer by layer,
each one's gather (transfer stream) running beside the other's compute.
"""

from __future__ import annotations

import torch

from . import row_kernels as rk
from .hybrid import store_entry


class BatchDecode:
    """Appends and attends one decode token per request, layer by layer.

    Usage: step = cache.decode_batch(ids); for each layer l in order:
    step.append(l, k, v); out = step.attend(l, q, top_pages) (or
    h = step.select(l, q, top_pages) ... out = step.finish(h), to run other
    work while the gather is in flight); then step.end(). Every layer must
    be appended before it is attended; lengths advance per layer.
    """

    def __init__(self, cache, request_ids, overlap=False, lengths_buffer=None):
        """overlap=True puts each layer's gather on the cache's transfer
        stream, ordered by events, for callers that run other work beside
        it; by default it runs in order on the compute stream (a gather
        that nothing runs beside gains nothing from a second queue and would
        pay two cross-queue event hops per layer). lengths_buffer: a device
        int64 [2, B] tensor that receives the step's lengths (the kernels
        read it), for a caller that replays captured launches reading it."""
        store = cache.storage
        if not store.cuda:
            raise RuntimeError("batched decode runs on a GPU cache (libnhs_hip.so)")
        store.check_stream()
        ids = list(request_ids)
        if not ids or len(set(ids)) != len(ids):
            raise ValueError("a batch needs distinct request IDs")
        lengths = []
        for rid in ids:
            request = store.requests.get(rid)
            if request is None:
                raise KeyError(f"unknown request {rid}")
            if len(set(request.lengths)) != 1 or request.lengths[0] == 0:
                raise ValueError("all layers must have the same nonempty history")
            if request.lengths[0] + 1 > request.max_tokens:
                raise ValueError("decode would exceed the request's reserved tokens")
            if any(cache.tables[rid, layer].busy for layer in range(request.layers)):
                raise RuntimeError("cannot decode during a row lease")
            lengths.append(request.lengths[0])
        if len({store.requests[r].layers for r in ids}) != 1:
            raise ValueError("requests of a batch must have the same layer count")
        self.cache, self.ids, self.lengths = cache, ids, lengths
        self.overlap = overlap
        self._written = []  # pages appended this step
        self.layers = store.requests[ids[0]].layers
        self.items = cache._layer_items(ids)
        self.max_pages = max(store.requests[r].page_count for r in ids)
        both = torch.tensor([lengths, [n + 1 for n in lengths]], dtype=torch.int64).pin_memory()
        if lengths_buffer is None:
            self.dev_lengths = both.to(cache.device, non_blocking=True)
        else:
            if lengths_buffer.shape != both.shape or lengths_buffer.dtype != torch.int64:
                raise ValueError("lengths_buffer must be int64 [2, B]")
            self.dev_lengths = lengths_buffer.copy_(both, non_blocking=True)
        self._appended = set()
        self._attended = set()
        self._pages = self._place_all()

    # ---- append --------------------------------------------------------------------------

    def _place_all(self):
        """Place every layer's page for each request's new token (layer
        major); returns pages[layer][b]. A failure rolls back the pages
        opened here."""
        cache, store = self.cache, self.cache.storage
        P = cache.config.page_size
        pages, opened = [], []
        try:
            for layer in range(self.layers):
                row = []
                for rid, length in zip(self.ids, self.lengths):
                    index = length // P
                    fresh = (rid, layer, index) not in store.pages
                    page = store.materialize(rid, layer, index)
                    if fresh:
                        opened.append(page)
                    if page.valid_tokens:  # the active tail keeps its allocation reference
                        if page.slot is None:
                            raise RuntimeError("active append tail lost its resident lease")
                        store.stats["resident_hits"] += 1
                        store.stats["append_resident_hits"] += 1
                    else:
                        try:
                            cache._prepare_append(page)
                        finally:
                            cache._writing_key = None
                    for ev in (page.ready, page.last_use, page.host_ready):
                        if ev is not None and getattr(ev, "stream", None) != store.compute:
                            store.wait(store.compute, ev)
                    row.append(page)
                pages.append(row)
        except Exception:
            for page in reversed(opened):
                if page.slot is not None:
                    cache._detach(page)
                    store_entry(cache.tables[page.key[:2]].source, page.key[2], -1)
                store._unmaterialize(page)
            raise
        return pages

    @torch.inference_mode()
    def append(self, layer, k, v):
        """k, v: [B, kv_heads, head_dim] in the cache dtype, on its device."""
        cache, store = self.cache, self.cache.storage
        cfg = cache.config
        B = len(self.ids)
        if layer in self._appended or not 0 <= layer < self.layers:
            raise ValueError("each layer is appended once per step")
        if k.shape != (B, cfg.kv_heads, cfg.head_dim) or v.shape != k.shape:
            raise ValueError(f"expected [{B}, {cfg.kv_heads}, {cfg.head_dim}] K/V")
        if k.dtype != cfg.dtype or v.dtype != cfg.dtype or k.device != cache.pool.device:
            raise ValueError("K/V dtype/device must match the cache")
        if not (k[0].is_contiguous() and v[0].is_contiguous() and k.stride() == v.stride()):
            k, v = k.contiguous(), v.contiguous()  # rows may be views of a fused projection
        rk.append_items(k, v, cache.pool, store.host_alias, self.items[layer], self.dev_lengths[0])
        self._account_append(layer)

    def _account_append(self, layer):
        """The host state of layer's append: page contents and versions,
        request lengths, the mirror byte count."""
        cache, store = self.cache, self.cache.storage
        P = cache.config.page_size
        pages = self._pages[layer]
        row_bytes = store.page_bytes // P
        for rid, length, page in zip(self.ids, self.lengths, pages):
            page.valid_tokens = length % P + 1
            page.content_version += 1
            page.sealed = page.valid_tokens == P
            page.host_enqueued_version = page.content_version
            store.requests[rid].lengths[layer] = length + 1
        self._written.extend(pages)
        store.stats["d2h_bytes"] += row_bytes * len(self.ids)
        self._appended.add(layer)

    def sync_tables(self):
        """Make the compute stream wait for every pending event of the batch's
        tables (all layers) now, so the layer launches that follow wait for
        none (as launches replayed from a captured graph cannot)."""
        store = self.cache.storage
        tables = [self.cache.tables[rid, layer] for layer in range(self.layers) for rid in self.ids]
        _wait_all(store, store.compute, (t.ready for t in tables))
        for t in tables:
            t.ready = None

    def clear_reads(self):
        """Make the compute and transfer streams wait now for the last read
        of every table of the batch (all layers) and drop those events, so
        that the launches that follow, gathers on the transfer stream
        included, wait for none (as launches captured into a graph cannot);
        end() records the step's own."""
        store = self.cache.storage
        tables = [self.cache.tables[rid, layer] for layer in range(self.layers) for rid in self.ids]
        for stream in (store.compute, store.transfer):
            _wait_all(store, stream, (t.last_use for t in tables))
        for t in tables:
            t.last_use = None

    def forget_capture_events(self):
        """Drop the events a captured (not executed) step left on the batch's
        tables: they belong to the graph and are never recorded."""
        for layer in range(self.layers):
            for rid in self.ids:
                t = self.cache.tables[rid, layer]
                t.ready = t.last_use = None

    def account_replayed(self):
        """Host state of a step whose launches were replayed from a captured
        graph of a step over the same batch: every layer appended and
        attended (the graph's gathers ran inside it, in its order)."""
        for layer in range(self.layers):
            self._account_append(layer)
            self._attended.add(layer)

    def end(self):
        """Close the step: one compute-stream event, recorded after every
        launch of the step, becomes the appended pages' write and mirror
        event and the read fence of every layer the step read (nothing
        changes blocks mid-step, so per-layer events would only add queue
        markers); then the residency policy tick (publishes mirrors, unpins
        clean history, serves hot-region demand)."""
        cache, store = self.cache, self.cache.storage
        done = store.event(store.compute)
        for page in self._written:
            page.ready = page.host_ready = done
            cache.pending_clean.add(page.key)
        for rid in self.ids:
            for layer in self._attended:
                cache.tables[rid, layer].last_use = done
                store.layer_reads[rid, layer] = done
        self._written = []
        cache.update_residency()

    # ---- attention -----------------------------------------------------------------------

    @torch.inference_mode()
    def attend(self, layer, query, top_pages, keep_sink=True):
        """query [B, q_heads, head_dim] -> [B, q_heads, head_dim]: Quest
        top_pages selection, resolve, gather and row attention for every
        request of the batch."""
        return self.finish(self.select(layer, query, top_pages, keep_sink))

    @torch.inference_mode()
    def select(self, layer, query, top_pages, keep_sink=True):
        """Quest selection and resolve on the compute stream, then the gather
        of the misses (on the transfer stream with overlap); returns the
        handle for finish()."""
        cache, store = self.cache, self.cache.storage
        cfg = cache.config
        if layer not in self._appended:
            raise ValueError("append the layer's token before attending")
        if query.ndim != 3 or query.shape[0] != len(self.ids) or query.shape[2] != cfg.head_dim:
            raise ValueError("query must be [B, q_heads, head_dim]")
        if query.shape[1] % cfg.kv_heads or query.device != cache.pool.device:
            raise ValueError("query GQA/device mismatch")
        if top_pages < 1:
            raise ValueError("top_pages must be positive")
        if top_pages * cfg.page_size > cache.hot_config.max_union_rows:
            raise ValueError("top-k width/union exceeds the admitted max_union_rows")
        if query.stride(2) != 1:
            query = query.contiguous()
        items, lengths = self.items[layer], self.dev_lengths[1]
        tables = [cache.tables[rid, layer] for rid in self.ids]
        # Quest scoring, then the selection and the resolve in one launch
        # where the shape fits (else the selector and the resolver)
        fused = rk.fused_select_fits(self.max_pages, top_pages, cfg.page_size)
        _, positions, scores = rk.quest_items(
            query, items, cfg.dtype, cfg.kv_heads, lengths, cfg.page_size, self.max_pages, top_pages, keep_sink,
            select=not fused,
        )
        _wait_all(store, store.compute, (t.ready for t in tables))
        hot_rows = cache.hot_config.hot_rows
        if fused:
            _, positions, physical, miss_host, miss_device, _ = rk.select_resolve_items(
                scores, items, hot_rows, lengths, cfg.page_size, top_pages, keep_sink, counts_total=cache.row_stats
            )
        else:
            physical, miss_host, miss_device, _ = rk.resolve_items(
                positions, items, hot_rows, lengths, cfg.page_size, counts_total=cache.row_stats
            )
        if not self.overlap:
            rk.gather_plan(store.host_alias, cache.pool, miss_host.view(-1), miss_device.view(-1), cfg.page_size)
            for t in tables:
                t.ready = None  # in order on the compute stream
            return layer, query, physical, None
        compute = store.active_compute()
        resolved = store.event(compute)
        store.wait(store.transfer, resolved)
        _wait_all(store, store.transfer, (t.last_use for t in tables))
        with store.context(store.transfer):
            rk.gather_plan(store.host_alias, cache.pool, miss_host.view(-1), miss_device.view(-1), cfg.page_size)
        miss_host.record_stream(store.transfer)
        miss_device.record_stream(store.transfer)
        gathered = store.event(store.transfer)
        for t in tables:
            t.ready = gathered
        return layer, query, physical, gathered

    @torch.inference_mode()
    def finish(self, handle):
        """Attention over the selected rows once their gather is done."""
        layer, query, physical, gathered = handle
        cache, store = self.cache, self.cache.storage
        store.wait(store.active_compute(), gathered)
        out = rk.attend_batched(query, cache.pool, physical, cache.config.page_size)
        self._attended.add(layer)
        return out


def _wait_all(store, stream, events):
    """Make `stream` wait for each distinct event not recorded on it."""
    seen = set()
    for ev in events:
        if ev is None or id(ev) in seen or getattr(ev, "stream", None) == stream:
            continue
        seen.add(id(ev))
        store.wait(stream, ev)
