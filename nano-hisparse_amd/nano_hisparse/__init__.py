"""nano_hisparse on MI355X: the sparse decode step of nano-hisparse on gfx950.

Quest page selection, the row resolver, the host-row gather and physical-row
GQA attention run as hand-written HIP kernels (libnhs_hip.so, C ABI in
include/nhs.h); the Python modules keep the reference's engine and cache API.
"""

from .config import CacheConfig, CapacityError
from .hybrid import HotConfig, HybridKVCache
from .row_index import LogicalTopK

__all__ = ["CacheConfig", "CapacityError", "HotConfig", "HybridKVCache", "LogicalTopK"]
