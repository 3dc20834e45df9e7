"""Attention over selected physical rows (reference nano_hisparse/attention.py:6-35).

The row lease resolves the selection and gathers the missed rows; the
attention itself is libnhs_hip.so's split-K GQA row kernel on the compute
stream. `backend` keeps the reference's argument: "auto", "hip" and
"triton" all name the HIP kernels on a GPU cache; "torch", the reference's
torch path, is not part of this build on the GPU. CPU caches compute only
through a CPU kernel provider that a test harness installs.
"""

import torch

BACKENDS = ("auto", "hip", "torch", "triton")


@torch.inference_mode()
def row_attention(query, cache, request_id, layer, topk, backend="auto"):
    if backend not in BACKENDS:
        raise ValueError("invalid attention backend")
    if query.ndim != 2 or query.shape[1] != cache.config.head_dim:
        raise ValueError("invalid query shape")
    if query.shape[0] % cache.config.kv_heads or query.device != cache.pool.device:
        raise ValueError("query GQA/device mismatch")
    if topk.head_columns is not None and topk.head_columns.shape[0] != query.shape[0]:
        raise ValueError("selection must have one row per query head")
    if backend == "triton" and not cache.storage.cuda:
        raise ValueError("Triton requires CUDA")
    if backend == "torch" and cache.storage.cuda:
        raise ValueError("backend 'torch' is the reference's CPU path; on the GPU use 'auto' (libnhs_hip.so)")
    with cache.resolve(request_id, layer, topk) as lease:
        rows = lease.plan.physical_rows
        if rows.ndim == 1:
            rows = rows[None, :].expand(query.shape[0], -1)
        if cache.storage.cuda:
            from .row_kernels import attend_rows

            return attend_rows(query, cache.pool, rows, cache.config)
        from .row_kernels import cpu_provider

        return cpu_provider("row_attention").attend_rows(query, cache.pool, rows, cache.config)
