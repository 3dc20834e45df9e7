"""Launchers for the gfx950 kernels of libnhs_hip.so, on torch tensors.

These replace nano_hisparse/row_kernels.py of the reference (Triton `_gather`
and `_attend`, and `MappedHost` through libcuda) and add batched launchers
for the selectors and the resolver. Every launcher validates shapes, dtypes
and devices, then enqueues on the current torch stream of the tensors'
device without synchronising. Tensors must live on a GPU: there is no CPU
kernel path. Host-logic tests that run without a GPU install a CPU kernel
provider explicitly (set_cpu_provider); the library never installs one.
"""

from __future__ import annotations

import ctypes

import torch
from torch._C import _cuda_getCurrentRawStream as _raw_stream

from . import _hip

_DTYPES = {torch.float32: _hip.NHS_F32, torch.float16: _hip.NHS_F16, torch.bfloat16: _hip.NHS_BF16}

_cpu_provider = None


def set_cpu_provider(provider):
    """Install (or clear, with None) the object that computes for CPU tensors.

    Only test harnesses use this, to run the host control plane without a GPU.
    It must offer resolve_rows(topk, source, resident, hot, tags, lru, length,
    page_size) -> RowPlan, gather_rows(host, pool, plan, config),
    attend_rows(query, pool, rows, config), quest_positions(query, minimum,
    maximum, length, page_size, top_pages, keep_sink) -> position tensor and
    mean_pages(query, summaries, length, page_size, top_pages) -> page list.
    """
    global _cpu_provider
    _cpu_provider = provider


def cpu_provider(what: str):
    if _cpu_provider is None:
        raise RuntimeError(
            f"{what}: nano_hisparse computes on the GPU through libnhs_hip.so; "
            "CPU tensors are not supported (no CPU kernel provider is installed)"
        )
    return _cpu_provider


def dtype_code(dtype) -> int:
    try:
        return _DTYPES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}") from None


def _ptr(t: torch.Tensor | None):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _stream(device) -> ctypes.c_void_p:
    """The calling thread's current stream on `device` as a raw handle (what
    torch.cuda.current_stream(device).cuda_stream returns, without building
    a Stream object: every launch from Python asks for it)."""
    return ctypes.c_void_p(_raw_stream(_device_index(device)))


def _device_index(device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def _require_gpu(what, *tensors):
    device = tensors[0].device
    if device.type != "cuda":
        raise ValueError(f"{what}: tensors must be on a GPU")
    for t in tensors:
        if t is not None and t.device != device:
            raise ValueError(f"{what}: all tensors must be on {device}")
    return device


def timing_events():
    """A (start, stop) pair of timing events usable with set_launch_events."""
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()  # creates the underlying hipEvent_t now
    stop.record()
    return start, stop


def set_launch_events(start, stop):
    """The next launcher called on this thread stamps `start` with the begin
    of its first kernel and `stop` with the end of its last kernel (events
    from timing_events(); either may be None)."""
    lib = _hip.load()
    lib.nhs_set_launch_events(
        ctypes.c_void_p(start.cuda_event if start is not None else 0),
        ctypes.c_void_p(stop.cuda_event if stop is not None else 0),
    )


class MappedHost:
    """Device alias of pinned host memory that torch allocated.

    The library only queries the alias (hipHostGetDevicePointer); it never
    registers or unregisters the allocation, which torch owns.
    Replaces MappedHost of the reference (row_kernels.py:10-32).
    """

    def __init__(self, tensor: torch.Tensor):
        if not tensor.is_pinned():
            raise ValueError("row gather requires pinned host backing")
        lib = _hip.load()
        alias = ctypes.c_void_p()
        _hip.check(lib.nhs_host_device_ptr(_ptr(tensor), ctypes.byref(alias)), "nhs_host_device_ptr")
        self.tensor, self.dtype, self.pointer = tensor, tensor.dtype, alias.value

    def data_ptr(self):
        return self.pointer


# ---- gather ----------------------------------------------------------------------


POOL_PAD_SLOTS = 3  # head slots of padding after each block of a GPU pool


def padded_pool(blocks, page_size, kv_heads, head_dim, dtype, device):
    """A pool [blocks, 2, page_size, kv_heads, head_dim] whose blocks are each
    followed by POOL_PAD_SLOTS head slots (head_dim elements each) of
    padding on a GPU (a strided view of a flat buffer; contiguous
    elsewhere). Consecutive blocks then shift every KV head's bytes by three
    head slots in the address, so over a request's pages each head's bytes
    take every offset within the rows. With contiguous blocks a head's bytes
    always sit at the same offset, and HBM served the heads whose offsets
    share address bits 8-10 (heads 1 and 5 of 8) ~20% slower, which the
    attention launch waited for."""
    shape = (blocks, 2, page_size, kv_heads, head_dim)
    block = 2 * page_size * kv_heads * head_dim
    esize = torch.empty((), dtype=dtype).element_size()
    if torch.device(device).type != "cuda" or kv_heads < 2 or (head_dim * esize) % 16:
        return torch.empty(shape, dtype=dtype, device=device)
    pad = POOL_PAD_SLOTS * head_dim
    flat = torch.empty(blocks * (block + pad), dtype=dtype, device=device)
    return flat.as_strided(shape, (block + pad, page_size * kv_heads * head_dim, kv_heads * head_dim, head_dim, 1))


def pool_block_stride(pool):
    """Bytes between consecutive blocks of a pool [blocks, 2, P, Hkv, D]: each
    block must be contiguous; a gap may follow it (stride(0) above
    2 * P * Hkv * D elements), as in the cache's padded pool."""
    if pool.ndim != 5:
        raise ValueError("the pool must be [blocks, 2, page_size, kv_heads, head_dim]")
    _, _, P, Hkv, D = pool.shape
    if tuple(pool.stride()[1:]) != (P * Hkv * D, Hkv * D, D, 1) or pool.stride(0) < 2 * P * Hkv * D:
        raise ValueError("the pool's blocks must be contiguous [2, P, Hkv, D] (a gap after each is allowed)")
    return pool.stride(0) * pool.element_size()


def gather_plan(host: MappedHost, pool, miss_host, miss_device, page_size):
    """Copy plan rows from the pinned host store into pool rows.

    miss_host / miss_device: int64 device tensors of equal numel (any shape,
    contiguous); -1 entries are skipped.
    """
    device = _require_gpu("gather_rows", pool, miss_host, miss_device)
    if miss_host.dtype != torch.int64 or miss_device.dtype != torch.int64:
        raise ValueError("gather plans must be int64")
    if miss_host.numel() != miss_device.numel() or not (miss_host.is_contiguous() and miss_device.is_contiguous()):
        raise ValueError("gather plans must be contiguous and of equal size")
    if host.dtype != pool.dtype:
        raise ValueError("host and pool dtypes differ")
    plane_bytes = pool[0, 0, 0].numel() * pool.element_size()
    stride = pool_block_stride(pool)
    lib = _hip.load()
    status = lib.nhs_gather_rows(
        ctypes.c_void_p(host.data_ptr()), _ptr(pool), _ptr(miss_host), _ptr(miss_device), miss_host.numel(),
        page_size, plane_bytes, stride, _stream(device),
    )
    _hip.check(status, "nhs_gather_rows")


def set_gather_workgroups(workgroups):
    """Cap the gather's grid (process-wide; 0 = uncapped)."""
    _hip.check(_hip.load().nhs_set_gather_workgroups(int(workgroups)), "nhs_set_gather_workgroups")


def gather_rows(host, pool, plan, config):
    """Reference signature (row_kernels.py:58-70): gather one RowPlan's misses."""
    gather_plan(host, pool, plan.miss_host_rows, plan.miss_device_rows, config.page_size)


# ---- append ----------------------------------------------------------------------


def append_page(k, v, pool, block, within, host, host_page, summary, minimum, maximum):
    """Write K/V rows [count, Hkv, D] into rows within.. of pool block `block`
    and, when `host` (a MappedHost) is given, of host block `host_page`; fold
    the new keys into the page's minimum/maximum [Hkv, D] and recompute its
    fp32 summary [Hkv, D] (mean key over every valid row)."""
    device = _require_gpu("append_page", k, v, pool, summary, minimum, maximum)
    if k.shape != v.shape or k.ndim != 3 or tuple(k.shape[1:]) != tuple(pool.shape[3:]):
        raise ValueError("append_page: K/V must be [tokens, kv_heads, head_dim] of the pool")
    if k.dtype != pool.dtype or v.dtype != pool.dtype or minimum.dtype != pool.dtype or maximum.dtype != pool.dtype:
        raise ValueError("append_page: K/V and bounds must have the pool dtype")
    if summary.dtype != torch.float32:
        raise ValueError("append_page: the summary is float32")
    for t in (summary, minimum, maximum):
        if not t.is_contiguous() or t.numel() != pool[0, 0, 0].numel():
            raise ValueError("append_page: summary and bounds are contiguous [kv_heads, head_dim]")
    if k.stride(2) != 1 or k.stride(1) != k.shape[2] or k.stride(0) != v.stride(0) or v.stride(2) != 1 \
            or v.stride(1) != v.shape[2]:
        raise ValueError("append_page: K/V rows must be contiguous with equal token strides")
    stride = pool_block_stride(pool)
    count, row_elems, P = k.shape[0], k.shape[1] * k.shape[2], pool.shape[2]
    if host is not None and host.dtype != pool.dtype:
        raise ValueError("append_page: host and pool dtypes differ")
    lib = _hip.load()
    status = lib.nhs_append_page(
        _ptr(k), _ptr(v), k.stride(0), dtype_code(pool.dtype), row_elems, P, _ptr(pool), stride, int(block),
        int(within),
        count, ctypes.c_void_p(host.data_ptr() if host is not None else 0), int(host_page if host is not None else 0),
        _ptr(summary), _ptr(minimum), _ptr(maximum), _stream(device),
    )
    _hip.check(status, "nhs_append_page")


class PageAppender:
    """append_page for the pages of one multi-page write (a prompt's K/V):
    the operands that stay fixed over the write (K/V rows, pool, host alias,
    the request's bounds [layers, pages, kv_heads, head_dim], the stream) are
    checked and turned into launch arguments once, so that each page costs
    one library call."""

    def __init__(self, k, v, pool, host, summaries, minimum, maximum):
        device = _require_gpu("append_page", k, v, pool, summaries, minimum, maximum)
        if k.shape != v.shape or k.ndim != 3 or tuple(k.shape[1:]) != tuple(pool.shape[3:]):
            raise ValueError("append_page: K/V must be [tokens, kv_heads, head_dim] of the pool")
        if k.dtype != pool.dtype or v.dtype != pool.dtype or minimum.dtype != pool.dtype or maximum.dtype != pool.dtype:
            raise ValueError("append_page: K/V and bounds must have the pool dtype")
        if summaries.dtype != torch.float32:
            raise ValueError("append_page: the summary is float32")
        row_elems = k.shape[1] * k.shape[2]
        for t in (summaries, minimum, maximum):
            if not t.is_contiguous() or t.shape[-2:] != k.shape[1:]:
                raise ValueError("append_page: summaries and bounds are contiguous [..., kv_heads, head_dim]")
        if k.stride(2) != 1 or k.stride(1) != k.shape[2] or k.stride(0) != v.stride(0) or v.stride(2) != 1 \
                or v.stride(1) != v.shape[2]:
            raise ValueError("append_page: K/V rows must be contiguous with equal token strides")
        if host is not None and host.dtype != pool.dtype:
            raise ValueError("append_page: host and pool dtypes differ")
        self.lib = _hip.load()
        self.k, self.v = k, v  # held for the write
        self.esize = k.element_size()
        self.k_ptr, self.v_ptr, self.token_stride = k.data_ptr(), v.data_ptr(), k.stride(0)
        self.dtype, self.row_elems, self.page_size = dtype_code(pool.dtype), row_elems, pool.shape[2]
        self.pool_ptr, self.pool_stride = pool.data_ptr(), pool_block_stride(pool)
        self.host_ptr = host.data_ptr() if host is not None else 0
        self.sum_ptr, self.min_ptr, self.max_ptr = summaries.data_ptr(), minimum.data_ptr(), maximum.data_ptr()
        self.stream = _stream(device)

    def __call__(self, first, count, block, within, host_page, bounds_index):
        """Rows first..first+count-1 of the write into rows within.. of pool
        block `block` (and host block `host_page`); bounds_index is the
        page's index in the flattened [layers, pages] bounds."""
        if not (0 <= first and count >= 1 and first + count <= self.k.shape[0]):
            raise ValueError("append_page: rows outside the write")
        off = bounds_index * self.row_elems
        status = self.lib.nhs_append_page(
            ctypes.c_void_p(self.k_ptr + first * self.token_stride * self.esize),
            ctypes.c_void_p(self.v_ptr + first * self.token_stride * self.esize), self.token_stride, self.dtype,
            self.row_elems, self.page_size, ctypes.c_void_p(self.pool_ptr), self.pool_stride, int(block), int(within),
            int(count), ctypes.c_void_p(self.host_ptr), int(host_page if self.host_ptr else 0),
            ctypes.c_void_p(self.sum_ptr + off * 4), ctypes.c_void_p(self.min_ptr + off * self.esize),
            ctypes.c_void_p(self.max_ptr + off * self.esize), self.stream,
        )
        _hip.check(status, "nhs_append_page")


# ---- attention ------------------------------------------------------------------

_workspaces: dict = {}


def attend_workspace(device, nbytes):
    """Zero-initialised attention workspace for the current stream of `device`.

    The kernel's split-arrival counters live at the front of the workspace;
    they must be zero before a launch and every launch leaves them at zero,
    so one buffer serves every call on a stream (calls on one stream never
    overlap). A larger request replaces the buffer.
    """
    index = _device_index(device)
    key = (index, _raw_stream(index))
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws



def attend_batched(query, pool, rows, page_size, out=None, workspace=None):
    """GQA attention of query [B, Hq, D] over rows [B, N] (shared by all heads
    of a request) or [B, Hq, N] (one list per head), int64 pool rows with -1
    masked. Returns out [B, Hq, D] in the query's dtype."""
    device = _require_gpu("attend_rows", query, pool, rows)
    if query.ndim != 3 or pool.ndim != 5 or rows.ndim not in (2, 3) or rows.dtype != torch.int64:
        raise ValueError("attend_rows: expected query [B, Hq, D], pool [blocks, 2, P, Hkv, D], int64 rows")
    B, Hq, D = query.shape
    kv_heads = pool.shape[3]
    if pool.shape[4] != D or pool.shape[2] != page_size or Hq % kv_heads:
        raise ValueError("attend_rows: query/pool head shape mismatch")
    if query.stride(2) != 1:
        raise ValueError("attend_rows: query rows must be contiguous")
    stride = pool_block_stride(pool)
    if rows.shape[0] != B or (rows.ndim == 3 and rows.shape[1] != Hq):
        raise ValueError("attend_rows: rows do not match the query batch/heads")
    if pool.shape[0] * page_size >= 2**31:
        raise ValueError("attend_rows: pool rows must be < 2^31")
    n_rows = rows.shape[-1]
    r_bs, r_cs = rows.stride(0), rows.stride(-1)
    r_hs = rows.stride(1) if rows.ndim == 3 else 0
    if rows.ndim == 3 and r_hs == 0:
        rows = rows[:, 0]  # an expanded shared list
    lib = _hip.load()
    if out is None:
        out = torch.empty(B, Hq, D, dtype=query.dtype, device=device)
    if n_rows == 0:
        return out.zero_()
    need = lib.nhs_attend_workspace_bytes(B, Hq, D, n_rows)
    if workspace is None:
        workspace = attend_workspace(device, need)
    elif workspace.numel() * workspace.element_size() < need:
        raise ValueError(f"attend_rows: workspace holds {workspace.numel() * workspace.element_size()} < {need} bytes")
    status = lib.nhs_attend_rows(
        _ptr(query), dtype_code(query.dtype), query.stride(0), query.stride(1), _ptr(pool), dtype_code(pool.dtype),
        stride, _ptr(rows), r_bs, r_hs, r_cs, B, n_rows, Hq, kv_heads, D, page_size, _ptr(out), out.stride(0),
        out.stride(1), _ptr(workspace), workspace.numel() * workspace.element_size(), _stream(device),
    )
    _hip.check(status, "nhs_attend_rows")
    return out


def attend_rows(query, pool, rows, config):
    """Reference signature (row_kernels.py:116-135): query [Hq, D], rows
    [Hq, N] (a stride-0 expansion when shared) -> [Hq, D]."""
    return attend_batched(query.unsqueeze(0), pool, rows.unsqueeze(0), config.page_size)[0]


# ---- resolver ---------------------------------------------------------------------


def _lengths_arg(lengths, device):
    if isinstance(lengths, torch.Tensor):
        return lengths.to(device=device, dtype=torch.int64).contiguous(), 0
    return None, int(lengths)


def _check_tables(B, source, resident, hot, tags, lru, page_size):
    """Validates the strided per-item tables; returns the hot row count."""
    for name, t, dt in (("source", source, torch.int32), ("resident", resident, torch.int32),
                        ("hot", hot, torch.int32), ("tags", tags, torch.int32), ("lru", lru, torch.int64)):
        if t.dtype != dt or t.ndim != 2 or t.shape[0] != B or t.stride(1) != 1:
            raise ValueError(f"{name} must be a [B, n] {dt} tensor with unit stride")
    if source.shape != resident.shape or source.stride(0) != resident.stride(0):
        raise ValueError("source and resident tables must have the same shape and strides")
    H = tags.shape[1]
    if lru.shape[1] != H or hot.shape[1] * page_size < H:
        raise ValueError("tags/lru/hot table sizes disagree")
    return H


def _plan_outputs(B, K, device):
    physical = torch.empty(B, K, dtype=torch.int64, device=device)
    return physical, torch.empty_like(physical), torch.empty_like(physical), torch.empty(
        B, 3, dtype=torch.int64, device=device)


def resolve_batched(positions, source, resident, hot, tags, lru, lengths, page_size, counts_total=None):
    """Resolve B items at once; every table has a leading batch dimension.

    positions [B, K] int32/int64; source/resident [B, n_pages] int32;
    hot [B, blocks] int32; tags [B, H] int32 and lru [B, H] int64 (updated in
    place); lengths: int, or int64 tensor [B]. Returns (physical, miss_host,
    miss_device, counts[B, 3]) as int64 device tensors; counts_total [3] is
    incremented when given.
    """
    device = _require_gpu("resolve_rows", positions, source, resident, hot, tags, lru)
    B, K = positions.shape
    if positions.dtype not in (torch.int32, torch.int64) or positions.stride(1) != 1:
        raise ValueError("positions must be a [B, K] int32/int64 tensor with unit stride")
    H = _check_tables(B, source, resident, hot, tags, lru, page_size)
    lengths_t, length = _lengths_arg(lengths, device)
    physical, miss_host, miss_device, counts = _plan_outputs(B, K, device)
    lib = _hip.load()
    status = lib.nhs_resolve_rows(
        B, K, _ptr(positions), int(positions.dtype == torch.int64), positions.stride(0), _ptr(source),
        _ptr(resident), source.stride(0), source.shape[1], _ptr(hot), hot.stride(0), _ptr(tags), tags.stride(0),
        _ptr(lru), lru.stride(0), H, _ptr(lengths_t), length, page_size, _ptr(physical), _ptr(miss_host),
        _ptr(miss_device), K, _ptr(counts), _ptr(counts_total), _stream(device),
    )
    _hip.check(status, "nhs_resolve_rows")
    return physical, miss_host, miss_device, counts


def expand_columns(shared_rows, columns):
    """out[h, c] = shared_rows[columns[h, c]] for 0 <= column < n, else -1."""
    device = _require_gpu("expand_columns", shared_rows, columns)
    shared_rows, columns = shared_rows.contiguous(), columns.contiguous()
    out = torch.empty(columns.shape, dtype=torch.int64, device=device)
    lib = _hip.load()
    status = lib.nhs_expand_columns(
        _ptr(shared_rows), shared_rows.numel(), _ptr(columns), columns.shape[0], columns.shape[1], _ptr(out),
        _stream(device),
    )
    _hip.check(status, "nhs_expand_columns")
    return out


# ---- selectors ---------------------------------------------------------------------


def quest_batched(query, minimum, maximum, lengths, page_size, top_pages, keep_sink=True, select=True):
    """Quest selection for B requests: query [B, Hq, D]; minimum/maximum
    [B, n_pages, Hkv, D] (the per-page bounds of each request). Returns
    (pages [B, top_pages] int32 ascending with -1 padding, positions
    [B, top_pages*P] int32 ascending with -1 padding, scores [B, n_pages]);
    select=False computes the scores only (pages and positions None), for
    select_resolve_batched."""
    device = _require_gpu("quest_selection", query, minimum, maximum)
    B, Hq, D = query.shape
    if minimum.shape != maximum.shape or minimum.ndim != 4 or minimum.shape[0] != B or minimum.shape[3] != D:
        raise ValueError("quest bounds must be [B, n_pages, Hkv, D]")
    if minimum.dtype != maximum.dtype or minimum.stride() != maximum.stride():
        raise ValueError("minimum and maximum must share dtype and layout")
    if not minimum[0].is_contiguous() or query.stride(2) != 1:
        raise ValueError("quest bounds of a request and query rows must be contiguous")
    n_pages, kv_heads = minimum.shape[1], minimum.shape[2]
    lengths_t, length = _lengths_arg(lengths, device)
    scores = torch.empty(B, n_pages, dtype=torch.float32, device=device)
    pages, positions = _selection_outputs(B, top_pages, page_size, device, select)
    lib = _hip.load()
    status = lib.nhs_quest_select(
        B, _ptr(query), dtype_code(query.dtype), query.stride(0), query.stride(1), _ptr(minimum), _ptr(maximum),
        dtype_code(minimum.dtype), minimum.stride(0), Hq, kv_heads, D, _ptr(lengths_t), length, page_size,
        n_pages, top_pages, int(bool(keep_sink)), _ptr(scores), _ptr(pages), _ptr(positions), _stream(device),
    )
    _hip.check(status, "nhs_quest_select")
    return pages, positions, scores


def _selection_outputs(B, top_pages, page_size, device, select):
    if not select:
        return None, None
    return (torch.empty(B, top_pages, dtype=torch.int32, device=device),
            torch.empty(B, top_pages * page_size, dtype=torch.int32, device=device))


def mean_batched(query, summaries, lengths, page_size, top_pages, select=True):
    """Page-mean selection for B requests; summaries [B, n_pages, Hkv, D] fp32.
    select=False computes the scores only, as in quest_batched."""
    device = _require_gpu("select_pages", query, summaries)
    B, Hq, D = query.shape
    if summaries.ndim != 4 or summaries.dtype != torch.float32 or summaries.shape[0] != B:
        raise ValueError("summaries must be [B, n_pages, Hkv, D] float32")
    if not summaries[0].is_contiguous() or query.stride(2) != 1:
        raise ValueError("summaries of a request and query rows must be contiguous")
    n_pages, kv_heads = summaries.shape[1], summaries.shape[2]
    lengths_t, length = _lengths_arg(lengths, device)
    scores = torch.empty(B, n_pages, dtype=torch.float32, device=device)
    pages, positions = _selection_outputs(B, top_pages, page_size, device, select)
    lib = _hip.load()
    status = lib.nhs_mean_select(
        B, _ptr(query), dtype_code(query.dtype), query.stride(0), query.stride(1), _ptr(summaries),
        summaries.stride(0), Hq, kv_heads, D, _ptr(lengths_t), length, page_size, n_pages, top_pages,
        _ptr(scores), _ptr(pages), _ptr(positions), _stream(device),
    )
    _hip.check(status, "nhs_mean_select")
    return pages, positions, scores


# ---- batched decode over per-item tables (nhs_layer_item) ---------------------------------


def layer_items(rows, device):
    """Device table of nhs_layer_item entries: `rows` is a list of layers,
    each a list of per-request dicts with the tensors named by
    _hip.LAYER_ITEM_FIELDS (n_pages an int). Returns int64 [layers, B, 9];
    the tensors must outlive the table."""
    fields = _hip.LAYER_ITEM_FIELDS
    table = []
    for layer in rows:
        for item in layer:
            for name in fields[:-1]:
                t = item[name]
                if t.device != device or not t.is_contiguous():
                    raise ValueError(f"layer item {name} must be a contiguous tensor on {device}")
            table.append([item[name].data_ptr() for name in fields[:-1]] + [int(item["n_pages"])])
    out = torch.tensor(table, dtype=torch.int64).view(len(rows), -1, len(fields))
    return out.pin_memory().to(device, non_blocking=True)


def append_items(k, v, pool, host, items, lengths):
    """One token per item: k/v [B, Hkv, D] rows appended at lengths[b] of
    each item's layer (nhs_append_items)."""
    device = _require_gpu("append_items", k, v, pool, items, lengths)
    B = k.shape[0]
    if k.shape != v.shape or k.dtype != v.dtype or k.dtype != pool.dtype or k.stride() != v.stride():
        raise ValueError("k and v must match each other and the pool")
    row_elems = k[0].numel()
    if row_elems != pool.shape[3] * pool.shape[4] or not k[0].is_contiguous():
        raise ValueError("k/v rows must be contiguous [Hkv, D] rows of the pool's shape")
    if items.shape[0] != B or lengths.shape[0] != B or lengths.dtype != torch.int64:
        raise ValueError("one item and one int64 length per row")
    stride = pool_block_stride(pool)
    lib = _hip.load()
    status = lib.nhs_append_items(
        B, _ptr(k), _ptr(v), k.stride(0), dtype_code(k.dtype), row_elems, pool.shape[2], _ptr(pool), stride,
        ctypes.c_void_p(host.data_ptr()) if host is not None else None, _ptr(items), _ptr(lengths),
        _stream(device),
    )
    _hip.check(status, "nhs_append_items")


def quest_items(query, items, bounds_dtype, kv_heads, lengths, page_size, max_pages, top_pages, keep_sink=True,
                select=True):
    """quest_batched over per-item bounds; returns (pages, positions, scores)
    (select=False: scores only)."""
    device = _require_gpu("quest_items", query, items, lengths)
    B, Hq, D = query.shape
    if query.stride(2) != 1 or items.shape[0] != B or lengths.shape[0] != B:
        raise ValueError("query rows must be contiguous, with one item and one length per request")
    scores = torch.empty(B, max_pages, dtype=torch.float32, device=device)
    pages, positions = _selection_outputs(B, top_pages, page_size, device, select)
    lib = _hip.load()
    status = lib.nhs_quest_select_items(
        B, _ptr(query), dtype_code(query.dtype), query.stride(0), query.stride(1), _ptr(items),
        dtype_code(bounds_dtype), Hq, kv_heads, D, _ptr(lengths), page_size, max_pages, top_pages,
        int(bool(keep_sink)), _ptr(scores), _ptr(pages), _ptr(positions), _stream(device),
    )
    _hip.check(status, "nhs_quest_select_items")
    return pages, positions, scores


def resolve_items(positions, items, hot_rows, lengths, page_size, counts_total=None):
    """resolve_batched over per-item tables; returns (physical, miss_host,
    miss_device, counts)."""
    device = _require_gpu("resolve_items", positions, items, lengths)
    B, K = positions.shape
    if positions.dtype not in (torch.int32, torch.int64) or positions.stride(1) != 1:
        raise ValueError("positions must be a [B, K] int32/int64 tensor with unit stride")
    if items.shape[0] != B or lengths.shape[0] != B:
        raise ValueError("one item and one length per request")
    physical = torch.empty(B, K, dtype=torch.int64, device=device)
    miss_host = torch.empty_like(physical)
    miss_device = torch.empty_like(physical)
    counts = torch.empty(B, 3, dtype=torch.int64, device=device)
    lib = _hip.load()
    status = lib.nhs_resolve_items(
        B, K, _ptr(positions), int(positions.dtype == torch.int64), positions.stride(0), _ptr(items), hot_rows,
        _ptr(lengths), page_size, _ptr(physical), _ptr(miss_host), _ptr(miss_device), K, _ptr(counts),
        _ptr(counts_total), _stream(device),
    )
    _hip.check(status, "nhs_resolve_items")
    return physical, miss_host, miss_device, counts


# ---- fused selection + resolution ---------------------------------------------------

FUSED_WAVE_PAGES = 1024  # pages one wave ranks (nhs_select_resolve_*)
FUSED_MAX_PAGES = 4096  # pages four waves rank, choosing at most FUSED_MAX_TOP
FUSED_MAX_TOP = 256
FUSED_MAX_POSITIONS = 4096  # top_pages * page_size held in LDS
MODES = {"quest": 0, "mean": 1}


def fused_select_fits(max_pages, top_pages, page_size):
    """Whether nhs_select_resolve_* takes this shape (else a selector launch
    and a resolver launch do the same work)."""
    pages = max(max_pages, top_pages)
    ranked = pages <= FUSED_WAVE_PAGES or (pages <= FUSED_MAX_PAGES and top_pages <= FUSED_MAX_TOP)
    return ranked and top_pages * page_size <= FUSED_MAX_POSITIONS


def select_resolve_batched(scores, source, resident, hot, tags, lru, lengths, page_size, top_pages, keep_sink=True,
                           mode="quest", counts_total=None):
    """The selection of quest_batched / mean_batched (mode) on their
    scores-only output, then resolve_batched on the chosen positions, in one
    launch. Returns (pages, positions, physical, miss_host, miss_device,
    counts), bit-identical to the two calls."""
    device = _require_gpu("select_resolve", scores, source, resident, hot, tags, lru)
    B, max_pages = scores.shape
    if scores.dtype != torch.float32 or not scores.is_contiguous():
        raise ValueError("scores must be a contiguous [B, max_pages] float32 tensor")
    H = _check_tables(B, source, resident, hot, tags, lru, page_size)
    lengths_t, length = _lengths_arg(lengths, device)
    K = top_pages * page_size
    pages, positions = _selection_outputs(B, top_pages, page_size, device, True)
    physical, miss_host, miss_device, counts = _plan_outputs(B, K, device)
    lib = _hip.load()
    status = lib.nhs_select_resolve_rows(
        B, _ptr(scores), max_pages, MODES[mode], top_pages, int(bool(keep_sink)), _ptr(source), _ptr(resident),
        source.stride(0), source.shape[1], _ptr(hot), hot.stride(0), _ptr(tags), tags.stride(0), _ptr(lru),
        lru.stride(0), H, _ptr(lengths_t), length, page_size, _ptr(pages), _ptr(positions), _ptr(physical),
        _ptr(miss_host), _ptr(miss_device), K, _ptr(counts), _ptr(counts_total), _stream(device),
    )
    _hip.check(status, "nhs_select_resolve_rows")
    return pages, positions, physical, miss_host, miss_device, counts


def select_resolve_items(scores, items, hot_rows, lengths, page_size, top_pages, keep_sink=True, mode="quest",
                         counts_total=None):
    """select_resolve_batched over per-item tables (nhs_select_resolve_items)."""
    device = _require_gpu("select_resolve_items", scores, items, lengths)
    B, max_pages = scores.shape
    if scores.dtype != torch.float32 or not scores.is_contiguous():
        raise ValueError("scores must be a contiguous [B, max_pages] float32 tensor")
    if items.shape[0] != B or lengths.shape[0] != B:
        raise ValueError("one item and one length per request")
    K = top_pages * page_size
    pages, positions = _selection_outputs(B, top_pages, page_size, device, True)
    physical, miss_host, miss_device, counts = _plan_outputs(B, K, device)
    lib = _hip.load()
    status = lib.nhs_select_resolve_items(
        B, _ptr(scores), max_pages, MODES[mode], top_pages, int(bool(keep_sink)), _ptr(items), hot_rows,
        _ptr(lengths), page_size, _ptr(pages), _ptr(positions), _ptr(physical), _ptr(miss_host),
        _ptr(miss_device), K, _ptr(counts), _ptr(counts_total), _stream(device),
    )
    _hip.check(status, "nhs_select_resolve_items")
    return pages, positions, physical, miss_host, miss_device, counts


# ---- elementwise stages of the batched decode layer -------------------------------------


def add_rmsnorm(x, delta, weight, eps, write_back=True):
    """x [rows, width] (+ delta, written back into x when write_back) ->
    RMSNorm(h) * weight, a new tensor."""
    device = _require_gpu("add_rmsnorm", x, weight)
    if x.ndim != 2 or not x.is_contiguous() or weight.shape != (x.shape[1],) or weight.dtype != x.dtype:
        raise ValueError("add_rmsnorm: x [rows, width] contiguous, weight [width] of x's dtype")
    if delta is not None and (delta.shape != x.shape or delta.dtype != x.dtype or not delta.is_contiguous()):
        raise ValueError("add_rmsnorm: delta must match x")
    out = torch.empty_like(x)
    lib = _hip.load()
    status = lib.nhs_add_rmsnorm(x.shape[0], x.shape[1], dtype_code(x.dtype), _ptr(x), _ptr(delta),
                                 int(bool(write_back)), _ptr(weight), float(eps), _ptr(out), _stream(device))
    _hip.check(status, "nhs_add_rmsnorm")
    return out


def rope_(t, heads, head_dim, cos, sin):
    """Rotary embedding in place on t [rows, >= heads*head_dim] (row stride
    t.stride(0)); cos/sin [rows, head_dim/2] in t's dtype."""
    device = _require_gpu("rope", t, cos, sin)
    rows = t.shape[0]
    if t.stride(-1) != 1 or cos.shape != (rows, head_dim // 2) or sin.shape != cos.shape:
        raise ValueError("rope: unit-stride rows and [rows, head_dim/2] cos/sin")
    if cos.dtype != t.dtype or sin.dtype != t.dtype or not (cos.is_contiguous() and sin.is_contiguous()):
        raise ValueError("rope: cos/sin must be contiguous in t's dtype")
    lib = _hip.load()
    status = lib.nhs_rope(rows, heads, head_dim, dtype_code(t.dtype), _ptr(t), t.stride(0), _ptr(cos), _ptr(sin),
                          _stream(device))
    _hip.check(status, "nhs_rope")


def silu_mul(gate_up):
    """gate_up [rows, 2*inter] -> silu(gate) * up [rows, inter]."""
    device = _require_gpu("silu_mul", gate_up)
    if gate_up.ndim != 2 or gate_up.shape[1] % 2 or not gate_up.is_contiguous():
        raise ValueError("silu_mul: gate_up [rows, 2*inter] contiguous")
    rows, inter = gate_up.shape[0], gate_up.shape[1] // 2
    out = torch.empty(rows, inter, dtype=gate_up.dtype, device=device)
    lib = _hip.load()
    status = lib.nhs_silu_mul(rows, inter, dtype_code(gate_up.dtype), _ptr(gate_up), _ptr(out), _stream(device))
    _hip.check(status, "nhs_silu_mul")
    return out


# ---- prefill attention ---------------------------------------------------------------------


def prefill_attention(q, k, v, out=None):
    """Causal GQA attention of one prompt: q [S, Hq, D], k/v [S, Hkv, D]
    (bf16 or fp16, rows may be views of a fused projection) -> [S, Hq, D]."""
    device = _require_gpu("prefill_attention", q, k, v)
    if q.ndim != 3 or k.ndim != 3 or k.shape != v.shape or q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2]:
        raise ValueError("prefill_attention: q [S, Hq, D], k and v [S, Hkv, D]")
    if q.dtype != k.dtype or q.dtype != v.dtype or q.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("prefill_attention: bf16 or fp16 q/k/v of one dtype")
    if any(t.stride(2) != 1 for t in (q, k, v)):
        raise ValueError("prefill_attention: head dims must be contiguous")
    S, Hq, D = q.shape
    if out is None:
        out = torch.empty(S, Hq, D, dtype=q.dtype, device=device)
    lib = _hip.load()
    status = lib.nhs_prefill_attention(
        _ptr(q), q.stride(0), q.stride(1), _ptr(k), k.stride(0), k.stride(1), _ptr(v), v.stride(0), v.stride(1),
        dtype_code(q.dtype), S, Hq, k.shape[1], D, _ptr(out), out.stride(0), out.stride(1), _stream(device),
    )
    _hip.check(status, "nhs_prefill_attention")
    return out


# ---- decode linear layers --------------------------------------------------------------------


def linear_small_m(x, weight, bias=None, out=None):
    """y = x @ weight.T (+ bias) for x [m <= 16, k], weight [n, k] (bf16 or
    fp16, one dtype); the weight stream of a decode projection."""
    device = _require_gpu("linear_small_m", x, weight)
    if x.ndim != 2 or weight.ndim != 2 or x.shape[1] != weight.shape[1]:
        raise ValueError("linear_small_m: x [m, k], weight [n, k]")
    if x.dtype != weight.dtype or x.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("linear_small_m: bf16 or fp16 x and weight of one dtype")
    if x.stride(1) != 1 or weight.stride(1) != 1:
        raise ValueError("linear_small_m: rows must be contiguous")
    m, k = x.shape
    n = weight.shape[0]
    if bias is not None and (bias.shape != (n,) or bias.dtype != x.dtype or not bias.is_contiguous()):
        raise ValueError("linear_small_m: bias must be a contiguous [n] vector of the same dtype")
    if out is None:
        out = torch.empty(m, n, dtype=x.dtype, device=device)
    elif out.shape != (m, n) or out.dtype != x.dtype or out.stride(1) != 1:
        raise ValueError("linear_small_m: out must be [m, n] with contiguous rows")
    lib = _hip.load()
    status = lib.nhs_linear_small_m(
        _ptr(x), x.stride(0), _ptr(weight), weight.stride(0), _ptr(bias),
        dtype_code(x.dtype), m, n, k, _ptr(out), out.stride(0), _stream(device),
    )
    _hip.check(status, "nhs_linear_small_m")
    return out


def _linear_operands(who, x, weight):
    if x.ndim != 2 or weight.ndim != 2 or x.shape[1] != weight.shape[1]:
        raise ValueError(f"{who}: x [m, k], weight [n, k]")
    if x.dtype != weight.dtype or x.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"{who}: bf16 or fp16 x and weight of one dtype")
    if x.stride(1) != 1 or weight.stride(1) != 1:
        raise ValueError(f"{who}: rows must be contiguous")


def linear_silu_mul(x, gate_up_weight):
    """silu(x @ gate.T) * (x @ up.T) for the fused [gate; up] weight
    [2 * inter, k]: linear_small_m then silu_mul in one launch, bit-identical
    to the two."""
    device = _require_gpu("linear_silu_mul", x, gate_up_weight)
    _linear_operands("linear_silu_mul", x, gate_up_weight)
    if gate_up_weight.shape[0] % 2:
        raise ValueError("linear_silu_mul: gate_up_weight [2 * inter, k]")
    m, k = x.shape
    inter = gate_up_weight.shape[0] // 2
    out = torch.empty(m, inter, dtype=x.dtype, device=device)
    lib = _hip.load()
    status = lib.nhs_linear_silu_mul(_ptr(x), x.stride(0), _ptr(gate_up_weight), gate_up_weight.stride(0),
                                     dtype_code(x.dtype), m, inter, k, _ptr(out), out.stride(0), _stream(device))
    _hip.check(status, "nhs_linear_silu_mul")
    return out


def linear_rope(x, weight, bias, rope_heads, head_dim, cos, sin):
    """x @ weight.T (+ bias) with the rotary embedding applied to the first
    rope_heads heads of head_dim of each row (cos/sin [m, head_dim / 2] in
    x's dtype): linear_small_m then rope_ in one launch, bit-identical to the
    two."""
    device = _require_gpu("linear_rope", x, weight, cos, sin)
    _linear_operands("linear_rope", x, weight)
    m, k = x.shape
    n = weight.shape[0]
    if bias is not None and (bias.shape != (n,) or bias.dtype != x.dtype or not bias.is_contiguous()):
        raise ValueError("linear_rope: bias must be a contiguous [n] vector of the same dtype")
    if cos.shape != (m, head_dim // 2) or sin.shape != cos.shape or cos.dtype != x.dtype or sin.dtype != x.dtype:
        raise ValueError("linear_rope: cos/sin [m, head_dim/2] in x's dtype")
    if not (cos.is_contiguous() and sin.is_contiguous()):
        raise ValueError("linear_rope: cos/sin must be contiguous")
    out = torch.empty(m, n, dtype=x.dtype, device=device)
    lib = _hip.load()
    status = lib.nhs_linear_rope(_ptr(x), x.stride(0), _ptr(weight), weight.stride(0), _ptr(bias),
                                 dtype_code(x.dtype), m, n, k, head_dim, rope_heads, _ptr(cos), _ptr(sin), _ptr(out),
                                 out.stride(0), _stream(device))
    _hip.check(status, "nhs_linear_rope")
    return out
