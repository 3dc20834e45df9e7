"""CPU oracle for the sparse decode step -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker (or the timed CPU baseline);
the product (the nano_hisparse package and libnhs_hip.so) never uses it.

It wraps the C restatement in nhs_oracle.c (built as libnhs_oracle.so by the
Makefile beside it) and adds two independent pure-Python formulations used to
pin it:

- resolve_rows_bruteforce: the resolver as a dictionary/list simulation of
  resident lookup, hot-tag lookup and LRU replacement, with no sorting or
  searchsorted (cross-checks oracle_resolve_rows, which follows the
  reference's sort formulation, nano_hisparse/row_index.py:62-140);
- attend_rows_float64: masked softmax attention in numpy float64
  (cross-checks oracle_attend_rows, nano_hisparse/attention.py:26-35).

Functions accept CPU torch tensors or numpy arrays; bf16 data is passed as
torch.bfloat16 tensors (or raw uint16 with an explicit dtype code).
"""

from __future__ import annotations

import ctypes
import os
from math import ceil

import numpy as np

F32, F16, BF16 = 0, 1, 2

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libnhs_oracle.so")
_lib = None


def build():
    """Compile libnhs_oracle.so with the Makefile beside this file."""
    import subprocess

    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"{_LIB_PATH} is missing; run `make -C {_HERE}`")
        _lib = ctypes.CDLL(_LIB_PATH)
        i32, i64, p, f32p = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p
        _lib.oracle_gather_rows.argtypes = [p, p, p, p, i64, i32, i64]
        _lib.oracle_attend_rows.argtypes = [
            p, i32, i64, i64, p, i32, p, i64, i64, i64, i32, i32, i32, i32, i32, i32, f32p,
        ]
        _lib.oracle_attend_rows_f32.argtypes = _lib.oracle_attend_rows.argtypes
        _lib.oracle_quest_select.argtypes = [
            i32, p, i32, i64, i64, p, p, i32, i64, i32, i32, i32, p, i32, i32, i32, i32, p, p, p,
        ]
        _lib.oracle_mean_select.argtypes = [
            i32, p, i32, i64, i64, p, i64, i32, i32, i32, p, i32, i32, i32, p, p, p,
        ]
        _lib.oracle_resolve_rows.argtypes = [p, i64, p, p, i64, p, p, p, i64, i64, i64, p, p, p, p]
        _lib.oracle_append_bounds.argtypes = [p, i32, i32, i32, i32, p, p, p]
        for name in (
            "oracle_gather_rows",
            "oracle_attend_rows",
            "oracle_attend_rows_f32",
            "oracle_quest_select",
            "oracle_mean_select",
            "oracle_resolve_rows",
            "oracle_append_bounds",
        ):
            getattr(_lib, name).restype = None
    return _lib


def _dtype_code(t):
    import torch

    if isinstance(t, torch.Tensor):
        return {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}[t.dtype]
    return {np.dtype(np.float32): F32, np.dtype(np.float16): F16}[t.dtype]


def _ptr(t):
    import torch

    if isinstance(t, torch.Tensor):
        assert t.device.type == "cpu" and t.is_contiguous(), "oracle inputs must be contiguous CPU tensors"
        return ctypes.c_void_p(t.data_ptr())
    assert isinstance(t, np.ndarray) and t.flags["C_CONTIGUOUS"]
    return ctypes.c_void_p(t.ctypes.data)


def _i64(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.int64))


# ---- gather (hybrid.py:452-459) ------------------------------------------------


def gather_rows(host, pool, miss_host, miss_device, page_size):
    """Copy plan rows host -> pool in place (both [blocks, 2, P, Hkv, D])."""
    if not (pool.is_contiguous() and host.is_contiguous()):
        raise ValueError("oracle gather_rows: host and pool must be contiguous (copy a padded pool first)")
    mh, md = _i64(miss_host).ravel(), _i64(miss_device).ravel()
    plane_bytes = int(np.prod(pool.shape[3:])) * pool.element_size()
    lib().oracle_gather_rows(_ptr(host), _ptr(pool), _ptr(mh), _ptr(md), mh.size, page_size, plane_bytes)


# ---- attention (attention.py:26-35) ----------------------------------------------


def attend_rows(query, pool, rows, page_size, arithmetic="float64"):
    """query [B, Hq, D]; rows [B, Hq, N] int64 (or [B, N] shared); fp32 out.
    arithmetic "float64": the masked softmax accumulated in double (the
    checker); "float32": the reference CPU path's own float32 arithmetic
    (oracle_attend_rows_f32, the CPU baseline's attention)."""
    import torch

    B, Hq, D = query.shape
    kv_heads = pool.shape[3]
    rows = torch.as_tensor(rows, dtype=torch.int64)
    if rows.ndim == 2:
        rows = rows[:, None, :].expand(B, Hq, rows.shape[-1])
    if tuple(rows.shape[:2]) != (B, Hq) or tuple(pool.shape[3:]) != (kv_heads, D) or Hq % kv_heads:
        raise ValueError("oracle attend_rows: query, rows and pool shapes disagree")
    rows = rows.contiguous()
    out = torch.empty(B, Hq, D, dtype=torch.float32)
    query, pool = query.contiguous(), pool.contiguous()
    fn = {"float64": lib().oracle_attend_rows, "float32": lib().oracle_attend_rows_f32}[arithmetic]
    fn(
        _ptr(query), _dtype_code(query), Hq * D, D, _ptr(pool), _dtype_code(pool), _ptr(rows),
        Hq * rows.shape[-1], rows.shape[-1], 1, B, rows.shape[-1], Hq, kv_heads, D, page_size, _ptr(out),
    )
    return out


def attend_rows_float64(query, pool, rows, page_size):
    """Independent numpy float64 masked softmax; same contract as attend_rows."""
    q = np.asarray(query.float().numpy(), dtype=np.float64)
    kv = np.asarray(pool.float().numpy(), dtype=np.float64)
    rows = np.asarray(rows, dtype=np.int64)
    B, Hq, D = q.shape
    kv_heads = kv.shape[3]
    if rows.ndim == 2:
        rows = np.broadcast_to(rows[:, None, :], (B, Hq, rows.shape[-1]))
    out = np.zeros((B, Hq, D))
    for b in range(B):
        for h in range(Hq):
            r = rows[b, h]
            r = r[r >= 0]
            if r.size == 0:
                continue
            kh = h // (Hq // kv_heads)
            k = kv[r // page_size, 0, r % page_size, kh]
            v = kv[r // page_size, 1, r % page_size, kh]
            s = k @ q[b, h] / np.sqrt(D)
            w = np.exp(s - s.max())
            out[b, h] = (w / w.sum()) @ v
    return out


# ---- selectors (selection.py:69-91, :119-145) -----------------------------------------


def quest_select(query, minimum, maximum, lengths, page_size, top_pages, keep_sink=True):
    """query [B, Hq, D]; minimum/maximum [B, max_pages, Hkv, D]. Returns
    (scores [B, max_pages] fp32, pages [B, top_pages], positions [B, top_pages*P])."""
    import torch

    query, minimum, maximum = (t.contiguous() for t in (query, minimum, maximum))
    B, Hq, D = query.shape
    max_pages, kv_heads = minimum.shape[1], minimum.shape[2]
    lengths = _i64(lengths).reshape(B)
    scores = torch.full((B, max_pages), float("nan"), dtype=torch.float32)
    pages = torch.empty(B, top_pages, dtype=torch.int32)
    positions = torch.empty(B, top_pages * page_size, dtype=torch.int32)
    lib().oracle_quest_select(
        B, _ptr(query), _dtype_code(query), Hq * D, D, _ptr(minimum), _ptr(maximum), _dtype_code(minimum),
        max_pages * kv_heads * D, Hq, kv_heads, D, _ptr(lengths), page_size, max_pages, top_pages,
        int(keep_sink), _ptr(scores), _ptr(pages), _ptr(positions),
    )
    return scores, pages, positions


def mean_select(query, summaries, lengths, page_size, top_pages):
    import torch

    query, summaries = query.contiguous(), summaries.contiguous().float()
    B, Hq, D = query.shape
    max_pages, kv_heads = summaries.shape[1], summaries.shape[2]
    lengths = _i64(lengths).reshape(B)
    scores = torch.full((B, max_pages), float("nan"), dtype=torch.float32)
    pages = torch.empty(B, top_pages, dtype=torch.int32)
    positions = torch.empty(B, top_pages * page_size, dtype=torch.int32)
    lib().oracle_mean_select(
        B, _ptr(query), _dtype_code(query), Hq * D, D, _ptr(summaries), max_pages * kv_heads * D, Hq,
        kv_heads, D, _ptr(lengths), page_size, max_pages, top_pages, _ptr(scores), _ptr(pages), _ptr(positions),
    )
    return scores, pages, positions


# ---- resolver (row_index.py:62-140) ------------------------------------------------


def resolve_rows(positions, source, resident, hot, tags, lru, length, page_size):
    """One item. tags/lru are int64 numpy arrays updated in place. Returns
    (physical, miss_host, miss_device, counts) as int64 numpy arrays."""
    raw = _i64(positions).ravel()
    source, resident, hot = _i64(source), _i64(resident), _i64(hot)
    assert tags.dtype == np.int64 and lru.dtype == np.int64 and tags.flags["C_CONTIGUOUS"]
    n, H = raw.size, tags.size
    physical, mh, md = (np.empty(n, np.int64) for _ in range(3))
    counts = np.empty(3, np.int64)
    lib().oracle_resolve_rows(
        _ptr(raw), n, _ptr(source), _ptr(resident), source.size, _ptr(hot), _ptr(tags), _ptr(lru), H,
        int(length), int(page_size), _ptr(physical), _ptr(mh), _ptr(md), _ptr(counts),
    )
    return physical, mh, md, counts


def resolve_rows_bruteforce(positions, source, resident, hot, tags, lru, length, page_size):
    """Dictionary/list simulation of the resolver contract (no sorts, no
    searchsorted). tags/lru are Python lists updated in place."""
    P, H = page_size, len(tags)
    raw = [int(t) for t in positions]
    n_pages = len(source)
    phys_of = {}
    counts = [0, 0, 0]
    needs_hot = []  # (token, host) ascending by token
    for t in sorted({t for t in raw if 0 <= t < length}):
        page = min(t // P, n_pages - 1)
        src, res = int(source[page]), int(resident[page])
        if src < 0:
            phys_of[t] = -1
            continue
        if res >= 0:
            phys_of[t] = res * P + t % P
            counts[0] += 1
        else:
            needs_hot.append((t, src * P + t % P))
    slot_of = {}
    for s, tag in enumerate(tags):
        if tag >= 0:
            slot_of[int(tag)] = s
    wanted = {host for _, host in needs_hot}
    protected = {s for s, tag in enumerate(tags) if tag >= 0 and int(tag) in wanted}
    victims = [s for s in lru if s not in protected] + [s for s in lru if s in protected]

    def hot_row(slot):
        return int(hot[slot // P]) * P + slot % P

    inserted = set()
    plan = []
    for t, host in needs_hot:
        if host in slot_of:
            phys_of[t] = hot_row(slot_of[host])
            counts[1] += 1
        else:
            slot = victims[min(len(plan), H - 1)]
            phys_of[t] = hot_row(slot)
            plan.append((host, hot_row(slot), slot))
            counts[2] += 1
    for host, _, slot in plan:
        tags[slot] = host
        inserted.add(slot)

    def category(s):
        return (s in inserted) + 2 * (s in protected)

    lru[:] = [s for c in range(4) for s in lru if category(s) == c]
    seen = set()
    physical = []
    for t in raw:
        if 0 <= t < length and t not in seen:
            seen.add(t)
            physical.append(phys_of[t])
        else:
            physical.append(-1)
    n = len(raw)
    miss_host = [h for h, _, _ in plan] + [-1] * (n - len(plan))
    miss_device = [d for _, d, _ in plan] + [-1] * (n - len(plan))
    return physical, miss_host[:n], miss_device[:n], counts


# ---- bounds producer (storage.py:302-309) --------------------------------------------------


def append_bounds(page_keys, within, count, summary, minimum, maximum):
    """page_keys [P, Hkv, D] (KV dtype); summary/minimum/maximum fp32 [Hkv, D]
    updated in place."""
    page_keys = page_keys.contiguous()
    row_elems = int(np.prod(page_keys.shape[1:]))
    lib().oracle_append_bounds(
        _ptr(page_keys), _dtype_code(page_keys), within, count, row_elems, _ptr(summary), _ptr(minimum),
        _ptr(maximum),
    )


def page_count(length, page_size):
    return ceil(length / page_size)
