"""ctypes binding of libnhs_hip.so, the gfx950 kernel library (include/nhs.h).

Loaded lazily on first GPU use, after torch: the library links the HIP
runtime that ships with torch, so the process keeps a single HIP runtime and
torch's stream handles are valid library arguments. There is no fallback: a
missing or unloadable library raises.
"""

from __future__ import annotations

import ctypes
import os
import re

_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_DIR, "libnhs_hip.so")
HEADER_PATH = os.path.normpath(os.path.join(_DIR, "..", "..", "include", "nhs.h"))

NHS_F32, NHS_F16, NHS_BF16 = 0, 1, 2
ABI_VERSION = 2

_i32, _i64, _p = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p

# argument types of every entry point, in include/nhs.h order
SIGNATURES = {
    "nhs_abi_version": ([], ctypes.c_int),
    "nhs_last_error": ([], ctypes.c_char_p),
    "nhs_set_launch_events": ([_p, _p], ctypes.c_int),
    "nhs_append_page": ([_p, _p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _p, ctypes.c_int64,
                         ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, _p, ctypes.c_int64, _p, _p, _p, _p],
                        ctypes.c_int),
    "nhs_host_device_ptr": ([_p, ctypes.POINTER(ctypes.c_void_p)], ctypes.c_int),
    "nhs_gather_rows": ([_p, _p, _p, _p, _i64, _i32, _i64, _i64, _p], ctypes.c_int),
    "nhs_set_gather_workgroups": ([_i32], ctypes.c_int),
    "nhs_attend_workspace_bytes": ([_i32, _i32, _i32, _i32], ctypes.c_int64),
    "nhs_attend_rows": (
        [_p, _i32, _i64, _i64, _p, _i32, _i64, _p, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _p, _i64,
         _i64, _p, _i64, _p],
        ctypes.c_int,
    ),
    "nhs_attend_rows_noalloc": (
        [_p, _i32, _i64, _i64, _p, _i32, _i64, _p, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _p, _i64,
         _i64, _p],
        ctypes.c_int,
    ),
    "nhs_resolve_rows": (
        [_i32, _i32, _p, _i32, _i64, _p, _p, _i64, _i32, _p, _i64, _p, _i64, _p, _i64, _i32, _p, _i64, _i32, _p,
         _p, _p, _i64, _p, _p, _p],
        ctypes.c_int,
    ),
    "nhs_quest_select": (
        [_i32, _p, _i32, _i64, _i64, _p, _p, _i32, _i64, _i32, _i32, _i32, _p, _i64, _i32, _i32, _i32, _i32, _p,
         _p, _p, _p],
        ctypes.c_int,
    ),
    "nhs_mean_select": (
        [_i32, _p, _i32, _i64, _i64, _p, _i64, _i32, _i32, _i32, _p, _i64, _i32, _i32, _i32, _p, _p, _p, _p],
        ctypes.c_int,
    ),
    "nhs_append_items": ([_i32, _p, _p, _i64, _i32, _i32, _i32, _p, _i64, _p, _p, _p, _p], ctypes.c_int),
    "nhs_quest_select_items": (
        [_i32, _p, _i32, _i64, _i64, _p, _i32, _i32, _i32, _i32, _p, _i32, _i32, _i32, _i32, _p, _p, _p, _p],
        ctypes.c_int,
    ),
    "nhs_resolve_items": (
        [_i32, _i32, _p, _i32, _i64, _p, _i32, _p, _i32, _p, _p, _p, _i64, _p, _p, _p],
        ctypes.c_int,
    ),
    "nhs_select_resolve_rows": (
        [_i32, _p, _i32, _i32, _i32, _i32, _p, _p, _i64, _i32, _p, _i64, _p, _i64, _p, _i64, _i32, _p, _i64, _i32,
         _p, _p, _p, _p, _p, _i64, _p, _p, _p],
        ctypes.c_int,
    ),
    "nhs_select_resolve_items": (
        [_i32, _p, _i32, _i32, _i32, _i32, _p, _i32, _p, _i32, _p, _p, _p, _p, _p, _i64, _p, _p, _p],
        ctypes.c_int,
    ),
    "nhs_add_rmsnorm": ([_i32, _i32, _i32, _p, _p, _i32, _p, ctypes.c_float, _p, _p], ctypes.c_int),
    "nhs_rope": ([_i32, _i32, _i32, _i32, _p, _i64, _p, _p, _p], ctypes.c_int),
    "nhs_silu_mul": ([_i32, _i32, _i32, _p, _p, _p], ctypes.c_int),
    "nhs_linear_small_m": ([_p, _i64, _p, _i64, _p, _i32, _i32, _i32, _i32, _p, _i64, _p], ctypes.c_int),
    "nhs_linear_silu_mul": ([_p, _i64, _p, _i64, _i32, _i32, _i32, _i32, _p, _i64, _p], ctypes.c_int),
    "nhs_linear_rope": (
        [_p, _i64, _p, _i64, _p, _i32, _i32, _i32, _i32, _i32, _i32, _p, _p, _p, _i64, _p], ctypes.c_int),
    "nhs_prefill_attention": (
        [_p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _p, _i64, _i64, _p],
        ctypes.c_int,
    ),
    "nhs_expand_columns": ([_p, _i64, _p, _i64, _i64, _p, _p], ctypes.c_int),
}

# nhs_layer_item: eight pointers and n_pages, 72 bytes
LAYER_ITEM_FIELDS = ("source", "resident", "hot", "tags", "lru", "minimum", "maximum", "summaries", "n_pages")

_lib = None


def header_symbols(path: str = HEADER_PATH) -> list[str]:
    """Names of the functions declared in include/nhs.h."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nhs_[a-z0-9_]+)\s*\(", text)))


def _hip_runtimes() -> set[str]:
    with open("/proc/self/maps") as maps:
        return {line.split()[-1] for line in maps if "libamdhip64" in line}


def load(check_runtime: bool = True):
    """Return the loaded library; raises RuntimeError when it is unavailable."""
    global _lib
    if _lib is not None:
        return _lib
    import torch  # noqa: F401  (loads torch's HIP runtime before the library binds to it)

    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `make -C nano-hisparse_amd/csrc` "
            "(or __graft_entry__.build()); nano_hisparse has no non-HIP kernel path"
        )
    lib = ctypes.CDLL(LIB_PATH)
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes, fn.restype = args, res
    if lib.nhs_abi_version() != ABI_VERSION:
        raise RuntimeError(f"libnhs_hip.so ABI {lib.nhs_abi_version()} != {ABI_VERSION}; rebuild it")
    if check_runtime and len(_hip_runtimes()) > 1:
        raise RuntimeError(f"two HIP runtimes are loaded: {sorted(_hip_runtimes())}")
    _lib = lib
    return lib


def check(status: int, what: str) -> None:
    if status != 0:
        message = _lib.nhs_last_error().decode(errors="replace") if _lib is not None else ""
        raise RuntimeError(f"{what} failed with status {status}: {message}")
