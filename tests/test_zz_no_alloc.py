"""nhs_attend_rows_noalloc (no workspace argument, no allocation) against
nhs_attend_rows with a caller workspace, through the C ABI: two calls in a
row on the one scratch array, the second with a smaller input, each equal
bit for bit to the workspace entry point and within tolerance of the oracle.
The first call reads the cache's padded pool (a gap after each block), the
second a contiguous one.
"""

import ctypes
import re

import pytest
import torch

import oracle
from nano_hisparse import _hip
from nano_hisparse import row_kernels as rk

pytestmark = pytest.mark.gpu

NHS_ERR_WORKSPACE = -3


def _max_bytes():
    """NHS_ATTEND_NOALLOC_BYTES of include/nhs.h."""
    text = open(_hip.HEADER_PATH).read()
    m = re.search(r"#define NHS_ATTEND_NOALLOC_BYTES \((\d+)ll << (\d+)\)", text)
    return int(m.group(1)) << int(m.group(2))


def _case(seed, B, Hq, Hkv, D, P, blocks, n_rows):
    g = torch.Generator().manual_seed(seed)
    pool = torch.randn(blocks, 2, P, Hkv, D, generator=g).to(torch.bfloat16)
    q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16)
    rows = torch.randint(0, blocks * P, (B, n_rows), generator=g)
    rows[:, ::7] = -1  # masked rows
    return q, pool, rows


def _noalloc(lib, q, pool, rows, P, out, stream):
    B, Hq, D = q.shape
    Hkv = pool.shape[3]
    return lib.nhs_attend_rows_noalloc(
        q.data_ptr(), _hip.NHS_BF16, q.stride(0), q.stride(1), pool.data_ptr(), _hip.NHS_BF16,
        rk.pool_block_stride(pool), rows.data_ptr(),
        rows.stride(0), 0, rows.stride(1), B, rows.shape[1], Hq, Hkv, D, P, out.data_ptr(), out.stride(0),
        out.stride(1), stream,
    )


def test_noalloc_attention_equals_the_workspace_entry_point():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    lib = _hip.load()
    dev = torch.device("cuda:0")
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    shapes = [  # the second call is smaller: fewer requests, rows and heads
        dict(seed=1, B=16, Hq=32, Hkv=8, D=128, P=64, blocks=600, n_rows=2048),
        dict(seed=2, B=3, Hq=28, Hkv=4, D=128, P=32, blocks=300, n_rows=500),
    ]
    for k, shape in enumerate(shapes):
        print("case:", shape, flush=True)
        q, pool, rows = _case(**shape)
        gq, grows = q.to(dev), rows.to(dev)
        if k == 0:  # the cache's padded pool (a gap after each block)
            blocks, _, P, Hkv, D = pool.shape
            gpool = rk.padded_pool(blocks, P, Hkv, D, pool.dtype, dev)
            gpool.copy_(pool.to(dev))
            assert rk.pool_block_stride(gpool) > pool[0].numel() * pool.element_size()
        else:
            gpool = pool.to(dev)
        need = lib.nhs_attend_workspace_bytes(q.shape[0], q.shape[1], q.shape[2], rows.shape[1])
        assert 0 < need <= _max_bytes()
        expected = rk.attend_batched(gq, gpool, grows, shape["P"])  # the workspace entry point
        out = torch.full_like(gq, float("nan"))
        status = _noalloc(lib, gq, gpool, grows, shape["P"], out, stream)
        _hip.check(status, "nhs_attend_rows_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(out.cpu().view(torch.int16), expected.cpu().view(torch.int16))
        want = oracle.attend_rows(q, pool, rows, shape["P"])
        assert (out.cpu().float() - want).abs().max().item() <= 2e-2


def test_noalloc_attention_rejects_shapes_beyond_its_scratch():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    lib = _hip.load()
    dev = torch.device("cuda:0")
    q = torch.zeros(256, 64, 128, dtype=torch.bfloat16, device=dev)
    pool = torch.zeros(4, 2, 64, 8, 128, dtype=torch.bfloat16, device=dev)
    rows = torch.zeros(256, 4096, dtype=torch.int64, device=dev)
    need = lib.nhs_attend_workspace_bytes(256, 64, 128, 4096)
    assert need > _max_bytes()
    out = torch.empty_like(q)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    assert _noalloc(lib, q, pool, rows, 64, out, stream) == NHS_ERR_WORKSPACE  # rejected on the host, nothing runs
    assert b"maximum" in lib.nhs_last_error()
