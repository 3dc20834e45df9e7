"""Cache dimensions and capacity errors (reference: nano_hisparse/config.py:8-30)."""

from __future__ import annotations

from dataclasses import dataclass

import torch


class CapacityError(RuntimeError):
    """Admission or allocation cannot proceed with the capacity left."""


_KV_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


@dataclass(frozen=True)
class CacheConfig:
    """Dimensions of the device pool and the pinned host store.

    gpu_pages blocks of [2, page_size, kv_heads, head_dim] make the device
    pool; host_pages blocks of the same shape make the host store.
    index_budget_bytes bounds the per-request index tensors (page bounds,
    summaries and the resolver tables) on the device.
    """

    gpu_pages: int = 16
    host_pages: int = 1024
    page_size: int = 16
    kv_heads: int = 2
    head_dim: int = 32
    device: str = "cuda"
    dtype: torch.dtype = torch.float32
    index_budget_bytes: int = 64 * 1024 * 1024

    def __post_init__(self):
        for name in ("gpu_pages", "host_pages", "page_size", "kv_heads", "head_dim"):
            if getattr(self, name) < 1:
                raise ValueError(f"{name} must be positive")
        if self.dtype not in _KV_DTYPES:
            raise ValueError("KV dtype must be float32, float16 or bfloat16")
        if self.index_budget_bytes < 1:
            raise ValueError("index budget must be positive")

    @property
    def row_bytes(self) -> int:
        """Bytes of one token row: K and V for every KV head."""
        return 2 * self.kv_heads * self.head_dim * torch.empty((), dtype=self.dtype).element_size()
