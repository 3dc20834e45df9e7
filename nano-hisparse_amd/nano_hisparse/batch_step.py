"""Batched sparse decode step for one layer, pipelined across two streams.

The reference resolves, gathers and attends one (request, layer) at a time
(hybrid.py:412-469, attention.py:18-35). Here B requests whose layer tables
are stacked ([B, ...] tensors with a common stride) run as chunks of
requests: for every chunk the compute stream selects pages (Quest) and
resolves rows, the transfer stream gathers that chunk's missed rows from
pinned host memory, and the compute stream attends over the chunk once its
gather event has fired. The compute stream enqueues chunk c+1's selection
and resolution before chunk c's attention, so while the transfer stream is
busy with one chunk's host rows the compute stream works on its neighbours
(double buffering); HIP events order the two streams, and nothing is read
back to the host.

On MI355X the default is one chunk. Kernels that run while the gather
streams host rows over PCIe slow down 2-7x, even on CUs the gather does not
use (a CU-masked transfer stream of 16 CUs still saturates the link), so the
overlap costs more than it hides at the Llama-3-8B decode shape: 778 us per
step unchunked against 805-2073 us with 2-8 chunks. The chunked schedule
stays for shapes with little gather traffic per chunk. With one chunk there
is nothing to overlap, and each event hop between two queues costs ~10 us,
so the gather then runs on the compute stream unless a transfer stream is
passed (740 us against 760 us per step).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import row_kernels as rk


@dataclass
class BatchTables:
    """Stacked resolver tables and Quest bounds of B requests for one layer.

    source/resident [B, n_pages] int32 (host page / resident block per
    logical page, -1 none); hot [B, hot_blocks] int32; tags [B, H] int32 and
    lru [B, H] int64 (updated in place by every step); minimum/maximum
    [B, n_pages, Hkv, D] in the KV dtype; lengths [B] int64.
    """

    source: torch.Tensor
    resident: torch.Tensor
    hot: torch.Tensor
    tags: torch.Tensor
    lru: torch.Tensor
    minimum: torch.Tensor
    maximum: torch.Tensor
    lengths: torch.Tensor

    @property
    def batch(self):
        return self.source.shape[0]


@dataclass
class ChunkResult:
    requests: slice
    positions: torch.Tensor  # [b, top_pages * P] int32 selected token positions
    physical: torch.Tensor  # [b, top_pages * P] int64 pool rows (-1 padding)
    counts: torch.Tensor  # [b, 3] int64 resident / hot / miss
    events: dict | None = None


class SparseDecodeBatch:
    """One layer's sparse decode for B requests: Quest top-k -> resolve ->
    host-row gather (transfer stream) -> GQA row attention, in `chunks`
    pipelined groups of requests.

    pool: the device KV pool [blocks, 2, P, Hkv, D]; host: the pinned host
    store of the same page shape. Tensors live on one GPU. transfer: the
    stream of the gathers (default: the compute stream for one chunk, a new
    side stream for several).
    """

    def __init__(self, pool, host, tables: BatchTables, page_size, top_pages, keep_sink=True, chunks=1,
                 compute=None, transfer=None):
        if pool.device.type != "cuda":
            raise ValueError("SparseDecodeBatch runs on a GPU")
        if not 1 <= chunks <= tables.batch:
            raise ValueError("chunks must be between 1 and the batch size")
        self.pool, self.tables, self.page_size = pool, tables, page_size
        self.top_pages, self.keep_sink = top_pages, keep_sink
        self.alias = rk.MappedHost(host)
        device = pool.device
        self.compute = compute or torch.cuda.current_stream(device)
        B = tables.batch
        bounds = [round(i * B / chunks) for i in range(chunks + 1)]
        self.slices = [slice(a, b) for a, b in zip(bounds, bounds[1:]) if b > a]
        if transfer is None:
            transfer = self.compute if len(self.slices) == 1 else torch.cuda.Stream(device=device)
        self.transfer = transfer
        self._workspace = None

    def _attend(self, query, physical, out):
        lib = rk._hip.load()
        B, Hq, D = query.shape
        need = lib.nhs_attend_workspace_bytes(B, Hq, D, physical.shape[-1])
        if self._workspace is None or self._workspace.numel() < need:
            self._workspace = torch.zeros(max(need, 1 << 16), dtype=torch.uint8, device=query.device)
        rk.attend_batched(query, self.pool, physical, self.page_size, out=out, workspace=self._workspace)

    def timing_events(self):
        """Events for one timed step: per chunk, a (start, stop) pair for
        each of its four launchers (create them before a timed region)."""
        names = ("quest", "resolve", "gather", "attention")
        return [{n: rk.timing_events() for n in names} for _ in self.slices]

    def step(self, query, out=None, events=None):
        """Attend query [B, Hq, D] over each request's Quest selection.

        Returns (out [B, Hq, D] in the query dtype, [ChunkResult]). With
        `events` from timing_events(), each launcher's events are stamped by
        its dispatches themselves (begin of its first kernel, end of its
        last).
        """
        t = self.tables
        B = t.batch
        if query.shape[0] != B:
            raise ValueError("query batch differs from the tables")
        if out is None:
            out = torch.empty_like(query)
        compute, transfer = self.compute, self.transfer

        def mark(events, name):
            if events is not None:
                rk.set_launch_events(*events[name])

        results, waiting = [], []
        with torch.cuda.stream(compute):
            for i, s in enumerate(self.slices):
                chunk_events = events[i] if events is not None else None
                mark(chunk_events, "quest")
                _, positions, _ = rk.quest_batched(
                    query[s], t.minimum[s], t.maximum[s], t.lengths[s], self.page_size, self.top_pages,
                    self.keep_sink,
                )
                mark(chunk_events, "resolve")
                physical, miss_host, miss_device, counts = rk.resolve_batched(
                    positions, t.source[s], t.resident[s], t.hot[s], t.tags[s], t.lru[s], t.lengths[s],
                    self.page_size,
                )
                resolved = torch.cuda.Event()
                resolved.record(compute)
                transfer.wait_event(resolved)
                with torch.cuda.stream(transfer):
                    mark(chunk_events, "gather")
                    rk.gather_plan(self.alias, self.pool, miss_host, miss_device, self.page_size)
                    gathered = torch.cuda.Event()
                    gathered.record(transfer)
                miss_host.record_stream(transfer)
                miss_device.record_stream(transfer)
                result = ChunkResult(s, positions, physical, counts, chunk_events)
                results.append(result)
                if waiting:  # attend the previous chunk now that this one's plan is enqueued
                    self._finish(query, out, *waiting.pop())
                waiting.append((result, gathered))
            while waiting:
                self._finish(query, out, *waiting.pop())
        return out, results

    def _finish(self, query, out, result, gathered):
        compute = self.compute
        compute.wait_event(gathered)
        if result.events is not None:
            rk.set_launch_events(*result.events["attention"])
        s = result.requests
        self._attend(query[s], result.physical, out[s])


def gather_results(results):
    """Concatenate the per-chunk positions, rows and counts along the batch."""
    return (
        torch.cat([r.positions for r in results]),
        torch.cat([r.physical for r in results]),
        torch.cat([r.counts for r in results]),
    )
