"""Attention over selected physical rows (reference nano_hisparse/attention.py:6-35).

The row lease resolves the selection and gathers the missed rows; the
attention itself is libnhs_hip.so's split-K GQA row kernel on the compute
stream. `backend` keeps the reference's argument (`auto|torch|triton`,
reference attention.py:8-9, cli.py:48, engine.py:30) plus "hip": on a GPU
cache every one of them runs the HIP kernel, so a caller that asks for the
reference's torch path or its Triton kernels gets the same masked softmax
over the same rows from the one GPU implementation (no second code path).
CPU caches compute only through a CPU kernel provider that a test harness
installs.
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
    with cache.resolve(request_id, layer, topk) as lease:
        rows = lease.plan.physical_rows
        if rows.ndim == 1:
            rows = rows[None, :].expand(query.shape[0], -1)
        if cache.storage.cuda:
            from .row_kernels import attend_rows

            return attend_rows(query, cache.pool, rows, cache.config)
        from .row_kernels import cpu_provider

        return cpu_provider("row_attention").attend_rows(query, cache.pool, rows, cache.config)
