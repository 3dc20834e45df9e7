"""Logical top-k positions and their resolution to physical pool rows.

Reference: nano_hisparse/row_index.py:15-140. resolve_rows runs the
libnhs_hip.so resolver: one workgroup sorts and deduplicates the positions,
looks rows up in the resident table, then in the hot tags (an LDS hash of
the wanted host rows probed by one pass over the tags), assigns misses to
unprotected LRU slots, updates tags and LRU order in place and writes the
compact miss plan, all on the device with no host round trip.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .selection import Selection

MAX_POSITIONS = 32768  # NHS_MAX_POSITIONS of include/nhs.h


class LogicalTopK:
    """Shared [K] token positions, with optional legacy per-head columns
    (reference row_index.py:15-51).

    For a selector's device output (ascending positions, -1 padding at the
    end) `positions` is the exact token list, as the reference builds it
    (row_index.py:22-23): the padding is cut off on first access, which
    reads its length back from the device once. The resolver reads the
    padded tensor (`resolver_positions`; padding resolves to -1) and never
    waits for that read.
    """

    __slots__ = ("_positions", "_padded", "head_columns")

    def __init__(self, positions, head_columns=None, *, padded=None):
        self._positions = positions
        self._padded = padded
        self.head_columns = head_columns

    @classmethod
    def from_selection(cls, selection: Selection, device):
        device = torch.device(device)
        shared = selection.shared_positions
        if shared is not None and shared.device == device:
            return cls(None, padded=shared)
        rows = selection.positions
        if all(row == rows[0] for row in rows):
            return cls(torch.tensor(rows[0], dtype=torch.int32, device=device))
        # explicit per-head rows: their union plus each head's columns in it
        union = sorted({t for row in rows for t in row})
        column = {t: i for i, t in enumerate(union)}
        width = max(map(len, rows))
        columns = [[column[t] for t in row] + [-1] * (width - len(row)) for row in rows]
        return cls(
            torch.tensor(union, dtype=torch.int32, device=device),
            torch.tensor(columns, dtype=torch.int64, device=device),
        )

    @property
    def positions(self):
        if self._positions is None:  # the valid entries of the padded output are a prefix
            self._positions = self._padded[: int((self._padded >= 0).sum())]
        return self._positions

    @property
    def resolver_positions(self):
        """The tensor the resolver reads: the padded selector output, or the
        exact positions."""
        return self._padded if self._padded is not None else self._positions

    def validate(self, device, maximum):
        p = self.resolver_positions
        if p.ndim != 1 or p.numel() < 1 or p.dtype not in (torch.int32, torch.int64) or p.device != device:
            raise ValueError("logical top-k must be a nonempty device integer vector")
        # padding never counts: the exact length is read back only when the
        # padded width exceeds the budget
        if p.numel() > maximum and self.positions.numel() > maximum:
            raise ValueError("top-k width/union exceeds the admitted max_union_rows")
        c = self.head_columns
        if c is not None and (c.ndim != 2 or c.device != device or c.dtype != torch.int64):
            raise ValueError("head columns must be a device int64 matrix")

    def __repr__(self):
        return f"LogicalTopK(positions={self.positions!r}, head_columns={self.head_columns!r})"


@dataclass
class RowPlan:
    physical_rows: torch.Tensor  # [K] (or [heads, W] for per-head columns) int64, -1 padding
    miss_host_rows: torch.Tensor  # [K] int64: compact prefix of missed host rows, then -1
    miss_device_rows: torch.Tensor  # [K] int64: their hot-row destinations, then -1
    counts: torch.Tensor  # [3] int64: unique resident hits, hot hits, misses


def _as(t, dtype):
    """A contiguous view of t in dtype, converting (and copying) only if needed."""
    return t if t.dtype == dtype and t.is_contiguous() else t.to(dtype).contiguous()


def resolve_rows(topk, source_table, resident_table, hot_table, tags, lru, length, page_size):
    """Resident lookup first; every selected hot hit is protected before any
    miss replaces a row; misses take the least recently used other slots.

    tags (host rows held by the hot slots, -1 empty) and lru (a permutation
    of the hot slots, least recent first) are updated in place. Duplicate,
    padding and out-of-range positions resolve to -1.
    """
    positions = topk.resolver_positions
    if positions.device.type != "cuda":
        from .row_kernels import cpu_provider

        return cpu_provider("resolve_rows").resolve_rows(
            topk, source_table, resident_table, hot_table, tags, lru, length, page_size
        )
    from . import row_kernels as rk

    if positions.numel() > MAX_POSITIONS:
        raise ValueError(f"the resolver takes at most {MAX_POSITIONS} positions per call")
    src, res, hot = (_as(t, torch.int32) for t in (source_table, resident_table, hot_table))
    tags32, lru64 = _as(tags, torch.int32), _as(lru, torch.int64)
    pos = positions if positions.is_contiguous() else positions.contiguous()
    physical, miss_host, miss_device, counts = rk.resolve_batched(
        pos[None], src[None], res[None], hot[None], tags32[None], lru64[None], int(length), int(page_size)
    )
    if tags32 is not tags:
        tags.copy_(tags32)
    if lru64 is not lru:
        lru.copy_(lru64)
    rows = physical[0]
    if topk.head_columns is not None:
        rows = rk.expand_columns(rows, topk.head_columns)
    return RowPlan(rows, miss_host[0], miss_device[0], counts[0])
