"""A CPU kernel provider for host-logic tests, computed by the C oracle.

The package computes only on the GPU; these tests run its host control plane
(admission, residency, leases, the engine) on CPU tensors by installing this
provider with row_kernels.set_cpu_provider. Each method has the contract of
the GPU launcher it stands in for.
"""

from __future__ import annotations

import numpy as np
import torch

import oracle
from nano_hisparse import row_kernels
from nano_hisparse.row_index import RowPlan


class OracleProvider:
    def resolve_rows(self, topk, source, resident, hot, tags, lru, length, page_size):
        tags_np = tags.numpy().astype(np.int64)
        lru_np = lru.numpy().astype(np.int64)
        physical, mh, md, counts = oracle.resolve_rows(
            topk.resolver_positions.numpy(), source.numpy(), resident.numpy(), hot.numpy(), tags_np, lru_np, length, page_size
        )
        tags.copy_(torch.from_numpy(tags_np))
        lru.copy_(torch.from_numpy(lru_np))
        rows = torch.from_numpy(physical)
        if topk.head_columns is not None:
            cols = topk.head_columns
            valid = (cols >= 0) & (cols < rows.numel())
            rows = torch.where(valid, rows[cols.clamp(0, max(rows.numel() - 1, 0))], torch.full_like(cols, -1))
        return RowPlan(rows, torch.from_numpy(mh), torch.from_numpy(md), torch.from_numpy(counts))

    def gather_rows(self, host, pool, plan, config):
        oracle.gather_rows(host, pool, plan.miss_host_rows, plan.miss_device_rows, config.page_size)

    def attend_rows(self, query, pool, rows, config):
        # [B=1, N] when every head shares one list, else [B=1, Hq, N]
        rows = rows[0][None] if rows.stride(0) == 0 else rows[None]
        out = oracle.attend_rows(query[None], pool.contiguous(), rows.contiguous(), config.page_size)
        return out[0].to(query.dtype)

    def quest_positions(self, query, minimum, maximum, length, page_size, top_pages, keep_sink):
        _, _, positions = oracle.quest_select(
            query[None], minimum[None], maximum[None], [length], page_size, top_pages, keep_sink
        )
        return positions[0]

    def mean_pages(self, query, summaries, length, page_size, top_pages):
        _, pages, _ = oracle.mean_select(query[None], summaries[None], [length], page_size, top_pages)
        return [p for p in pages[0].tolist() if p >= 0]


def install():
    row_kernels.set_cpu_provider(OracleProvider())


def uninstall():
    row_kernels.set_cpu_provider(None)
