"""Batched sparse decode step for one layer, with the host-row gather
double-buffered against attention on a side stream.

The reference resolves, gathers and attends one (request, layer) at a time
(hybrid.py:412-469, attention.py:18-35). Here B requests whose layer tables
are stacked ([B, ...] tensors with a common stride) take one Quest launch
and one resolver launch; their host-row gathers then run on the transfer
stream in `chunks` groups of requests, and the compute stream attends over
each group as soon as that group's gather event has fired, while the
transfer stream already copies the next group's rows. HIP events order the
two streams; nothing is read back to the host.

Measured on MI355X at the Llama-3-8B decode shape (16 requests, 2048 rows,
25% of them gathered): kernels that run beside the PCIe gather slow down
2-7x (the contention is in the shared L2/fabric path: it stays when the
gather is confined to 16 CUs, which alone still saturate the link), so only
the attention, not the selection or resolution, is overlapped with it. With
one chunk there is nothing to overlap and each event hop between two queues
costs ~10 us, so the gather then runs on the compute stream unless a
transfer stream is passed.
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
class StepResult:
    positions: torch.Tensor  # [B, top_pages * P] int32 selected token positions (-1 padding)
    physical: torch.Tensor  # [B, top_pages * P] int64 pool rows (-1 padding)
    counts: torch.Tensor  # [B, 3] int64 resident / hot / miss
    chunks: list  # slices of the batch gathered and attended together


class SparseDecodeBatch:
    """One layer's sparse decode for B requests: Quest top-k -> resolve ->
    host-row gather -> GQA row attention.

    pool: the device KV pool [blocks, 2, P, Hkv, D]; host: the pinned host
    store of the same page shape. Tensors live on one GPU. chunks: request
    groups whose gathers and attentions are pipelined. transfer: the stream
    of the gathers (default: the compute stream for one chunk, a new side
    stream for several).
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

    def timing_events(self):
        """Events for one timed step: a (start, stop) pair for the Quest and
        resolver launches and, per chunk, for its gather and its attention
        (create them before a timed region)."""
        return {
            "quest": [rk.timing_events()],
            "resolve": [rk.timing_events()],
            "gather": [rk.timing_events() for _ in self.slices],
            "attention": [rk.timing_events() for _ in self.slices],
        }

    def _attend(self, query, physical, out):
        lib = rk._hip.load()
        B, Hq, D = query.shape
        need = lib.nhs_attend_workspace_bytes(B, Hq, D, physical.shape[-1])
        if self._workspace is None or self._workspace.numel() < need:
            self._workspace = torch.zeros(max(need, 1 << 16), dtype=torch.uint8, device=query.device)
        rk.attend_batched(query, self.pool, physical, self.page_size, out=out, workspace=self._workspace)

    def step(self, query, out=None, events=None):
        """Attend query [B, Hq, D] over each request's Quest selection.

        Returns (out [B, Hq, D] in the query dtype, StepResult). With
        `events` from timing_events(), every launch stamps its pair with its
        kernels' own begin and end (a stage left out of the dict is not
        stamped; each stamped launch adds a few microseconds).
        """
        t = self.tables
        if query.shape[0] != t.batch:
            raise ValueError("query batch differs from the tables")
        if out is None:
            out = torch.empty_like(query)
        compute, transfer = self.compute, self.transfer
        side = transfer is not compute

        def mark(name, i=0):
            if events is not None and name in events:
                rk.set_launch_events(*events[name][i])

        with torch.cuda.stream(compute):
            # Quest scoring, then the selection and the resolve in one launch
            # where it fits (else the selector and the resolver separately)
            fused = rk.fused_select_fits(t.minimum.shape[1], self.top_pages, self.page_size)
            mark("quest")
            _, positions, scores = rk.quest_batched(
                query, t.minimum, t.maximum, t.lengths, self.page_size, self.top_pages, self.keep_sink,
                select=not fused,
            )
            mark("resolve")
            if fused:
                _, positions, physical, miss_host, miss_device, counts = rk.select_resolve_batched(
                    scores, t.source, t.resident, t.hot, t.tags, t.lru, t.lengths, self.page_size, self.top_pages,
                    self.keep_sink,
                )
            else:
                physical, miss_host, miss_device, counts = rk.resolve_batched(
                    positions, t.source, t.resident, t.hot, t.tags, t.lru, t.lengths, self.page_size
                )
            if side:
                resolved = torch.cuda.Event()
                resolved.record(compute)
                transfer.wait_event(resolved)
            gathered = []
            with torch.cuda.stream(transfer):
                for i, s in enumerate(self.slices):
                    mark("gather", i)
                    rk.gather_plan(self.alias, self.pool, miss_host[s], miss_device[s], self.page_size)
                    if side:
                        done = torch.cuda.Event()
                        done.record(transfer)
                        gathered.append(done)
            if side:
                miss_host.record_stream(transfer)
                miss_device.record_stream(transfer)
            for i, s in enumerate(self.slices):
                if side:
                    compute.wait_event(gathered[i])
                mark("attention", i)
                self._attend(query[s], physical[s], out[s])
        return out, StepResult(positions, physical, counts, list(self.slices))
