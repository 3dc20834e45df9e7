"""Token selections and the page selectors that produce them.

Reference: nano_hisparse/selection.py:11-153. A Selection is one shared set
of causal token positions (or one set per query head). The selectors run on
the GPU (libnhs_hip.so) and return selections backed by a device tensor of
positions, so the decode path never copies them to the host; `positions`
materializes Python tuples on first access only.
"""

from __future__ import annotations

from math import ceil, sqrt

import torch


class Selection:
    """Canonical per-head sorted unique token positions.

    Either `positions` (tuples, one per query head) is given, or a shared
    device tensor of positions (ascending, -1 padding) from a selector.
    """

    __slots__ = ("_positions", "_shared", "length", "page_size", "source", "heads")

    def __init__(self, positions, length, page_size, source, *, heads=None, shared=None):
        self._positions = positions
        self._shared = shared
        self.length, self.page_size, self.source = length, page_size, source
        self.heads = len(positions) if positions is not None else heads

    @classmethod
    def from_tokens(cls, rows, length, page_size, heads, source="external"):
        if length < 1 or page_size < 1 or heads < 1:
            raise ValueError("selection dimensions must be positive")
        if isinstance(rows, torch.Tensor):
            rows = rows.cpu().tolist()
        if rows and isinstance(rows[0], int):
            rows = [rows]
        if len(rows) == 1:
            rows = rows * heads
        if len(rows) != heads:
            raise ValueError("selection must be shared or have one row per query head")
        canonical = []
        for row in rows:
            if not isinstance(row, (list, tuple)):
                raise TypeError("selection rows must be integer sequences")
            if any(not isinstance(t, int) or t < -1 or t >= length for t in row):
                raise ValueError("token selection contains noncausal or invalid positions")
            values = tuple(sorted({t for t in row if t != -1}))
            if not values:
                raise ValueError("each query head must select at least one token")
            canonical.append(values)
        return cls(tuple(canonical), length, page_size, source)

    @classmethod
    def from_pages(cls, rows, length, page_size, heads, source="pages"):
        if isinstance(rows, torch.Tensor):
            rows = rows.cpu().tolist()
        if rows and isinstance(rows[0], int):
            rows = [rows]
        count = ceil(length / page_size)
        if any(p < 0 or p >= count for row in rows for p in row):
            raise ValueError("invalid logical page")
        tokens = [
            [t for p in row for t in range(p * page_size, min((p + 1) * page_size, length))] for row in rows
        ]
        return cls.from_tokens(tokens, length, page_size, heads, source)

    @classmethod
    def from_device(cls, positions: torch.Tensor, length, page_size, heads, source):
        """A shared selection held as an ascending position tensor with -1
        padding (selector output); nothing is copied to the host."""
        if positions.ndim != 1:
            raise ValueError("device positions must be a vector")
        return cls(None, length, page_size, source, heads=heads, shared=positions)

    @property
    def shared_positions(self):
        """The device position tensor of a selector-made selection, else None."""
        return self._shared

    @property
    def positions(self):
        if self._positions is None:  # materialize once (a device -> host copy)
            row = tuple(t for t in self._shared.tolist() if t >= 0)
            self._positions = (row,) * self.heads
        return self._positions

    @property
    def pages(self):
        return sorted({t // self.page_size for row in self.positions for t in row})

    def _key(self):
        return (self.positions, self.length, self.page_size, self.source)

    def __eq__(self, other):
        return isinstance(other, Selection) and self._key() == other._key()

    def __hash__(self):
        return hash(self._key())

    def __repr__(self):
        return (
            f"Selection(positions={self.positions!r}, length={self.length}, "
            f"page_size={self.page_size}, source={self.source!r})"
        )


def quest_selection(query, minimum, maximum, length, page_size, top_pages, keep_sink=True):
    """Quest page selection shared across heads (reference selection.py:69-91).

    Each page scores mean_h sum_d max(q[h,d] kmin[d], q[h,d] kmax[d]) over its
    per-element key bounds; the last page (and the first, with keep_sink and
    a budget above one page) is always kept; the top_pages pages are
    expanded to their causal tokens. query [q_heads, head_dim]; minimum and
    maximum [pages, kv_heads, head_dim] (a request's bounds for one layer).
    """
    count = ceil(length / page_size)
    if top_pages < 1 or query.shape[0] % minimum.shape[1]:
        raise ValueError("invalid page budget or GQA shape")
    heads = query.shape[0]
    if top_pages >= count:
        return Selection.from_pages(list(range(count)), length, page_size, heads, "quest")
    if query.device.type != "cuda":
        from .row_kernels import cpu_provider

        positions = cpu_provider("quest_selection").quest_positions(
            query, minimum, maximum, length, page_size, top_pages, keep_sink
        )
    else:
        from . import row_kernels as rk

        _, positions, _ = rk.quest_batched(
            query[None], minimum[None], maximum[None], int(length), page_size, top_pages, keep_sink
        )
        positions = positions[0]
    return Selection.from_device(positions, length, page_size, heads, "quest")


def select_pages(cache, request_id: str, layer: int, query: torch.Tensor, top_k: int | None) -> list[int]:
    """Page-mean selector for demonstrations (reference selection.py:119-145):
    the GQA-group mean query against each page's mean key; the first and last
    page (the last only, for a one-page budget) are always kept. None keeps
    the whole causal history."""
    request = cache.storage.requests[request_id]
    length = request.lengths[layer]
    count = ceil(length / cache.config.page_size)
    if count == 0:
        raise ValueError("cannot attend to empty KV")
    if top_k is None or top_k >= count:
        return list(range(count))
    if top_k < 1:
        raise ValueError("top_k must be positive or None")
    required = [count - 1] if top_k == 1 else [0, count - 1]
    if top_k == len(required):
        return sorted(required)
    if query.device.type != "cuda":
        from .row_kernels import cpu_provider

        return cpu_provider("select_pages").mean_pages(query, request.summaries[layer], length,
                                                       cache.config.page_size, top_k)
    from . import row_kernels as rk

    pages, _, _ = rk.mean_batched(query[None], request.summaries[layer][None], length, cache.config.page_size, top_k)
    return pages[0].tolist()  # a host list, as the reference returns


def selection_oracle(query, k, v, selection):
    """Offline diagnostic: sparse attention over the selection next to full
    attention, and how much of the attention mass the selection keeps
    (reference selection.py:94-116)."""
    groups = query.shape[0] // k.shape[1]
    keys = k.repeat_interleave(groups, 1).float()
    values = v.repeat_interleave(groups, 1).float()
    scores = torch.einsum("hd,thd->ht", query.float(), keys) / query.shape[-1] ** 0.5
    probability = scores.softmax(-1)
    full = torch.einsum("ht,thd->hd", probability, values)
    mask = torch.zeros_like(scores, dtype=torch.bool)
    for head, positions in enumerate(selection.positions):
        mask[head, list(positions)] = True
    sparse = torch.einsum("ht,thd->hd", scores.masked_fill(~mask, -torch.inf).softmax(-1), values)
    recalls = []
    for head, positions in enumerate(selection.positions):
        best = set(scores[head].topk(len(positions)).indices.tolist())
        recalls.append(len(best & set(positions)) / len(best))
    metrics = {
        "retained_attention_mass": (probability * mask).sum(-1).mean().item(),
        "oracle_token_recall": sum(recalls) / len(recalls),
        "relative_output_l2": ((sparse - full).norm() / full.norm().clamp_min(1e-12)).item(),
        "selected_token_fraction": mask.float().mean().item(),
        "union_pages": len(selection.pages),
    }
    return sparse.to(query.dtype), metrics


def dense_attention(query: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
    """Full softmax attention of query [heads, dim] over k/v [tokens, kv_heads,
    dim] in fp32 (a diagnostic; reference selection.py:148-153)."""
    groups = query.shape[0] // k.shape[1]
    k, v = k.repeat_interleave(groups, 1), v.repeat_interleave(groups, 1)
    scores = torch.einsum("hd,thd->ht", query.float(), k.float()) / sqrt(query.shape[-1])
    return torch.einsum("ht,thd->hd", scores.softmax(-1), v.float()).to(query.dtype)
