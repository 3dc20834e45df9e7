"""Decode linear layers (nhs_linear_small_m) against an fp32 reference of
torch's nn.Linear on the same bf16/fp16 inputs: within 2 units in the last
place of the output dtype relative to the largest output magnitude of the row
(the kernel rounds one fp32 sum once; the order of the K sum differs), at the
Llama-3-8B decode shapes (q/k/v fused with bias, o, gate/up fused, down,
lm_head) and ragged token counts."""

import pytest
import torch

from nano_hisparse import row_kernels as rk


def log_case(**kw):
    print("case:", kw, flush=True)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,n,k,bias", [(8, 6144, 4096, True), (8, 4096, 4096, False), (8, 28672, 4096, False),
                                        (8, 4096, 14336, False), (3, 4096, 2048, True), (1, 16, 2048, False),
                                        (16, 512, 6144, True), (13, 2064, 4096, False)])
def test_linear_small_m_matches_fp32_reference(gpu, dtype, m, n, k, bias):
    log_case(test="linear", dtype=str(dtype), m=m, n=n, k=k, bias=bias)
    g = torch.Generator(device=gpu).manual_seed(n + k + m)
    x = torch.randn(m, k, generator=g, device=gpu).to(dtype)
    w = (torch.randn(n, k, generator=g, device=gpu) / k ** 0.5).to(dtype)
    b = torch.randn(n, generator=g, device=gpu).to(dtype) if bias else None
    y = rk.linear_small_m(x, w, b)
    ref = x.float() @ w.float().t().contiguous()
    if bias:
        ref = ref + b.float()
    eps = torch.finfo(dtype).eps
    scale = ref.abs().amax(1, keepdim=True).clamp_min(1e-3)
    assert ((y.float() - ref).abs() / scale).max().item() <= 2 * eps


@pytest.mark.gpu
def test_linear_small_m_strided_rows_and_out(gpu):
    """x and out as row slices of wider buffers (the fused projection layout)."""
    log_case(test="linear-strided")
    g = torch.Generator(device=gpu).manual_seed(1)
    big = torch.randn(5, 2048 + 64, generator=g, device=gpu).to(torch.bfloat16)
    x = big[:, 32:32 + 2048]
    w = (torch.randn(256, 2048, generator=g, device=gpu) / 45).to(torch.bfloat16)
    out_big = torch.zeros(5, 256 + 16, device=gpu, dtype=torch.bfloat16)
    out = out_big[:, 16:]
    rk.linear_small_m(x, w, out=out)
    ref = x.float() @ w.float().t().contiguous()
    assert ((out.float() - ref).abs() / ref.abs().amax(1, keepdim=True)).max().item() <= 2 * torch.finfo(torch.bfloat16).eps
    assert torch.equal(out_big[:, :16], torch.zeros_like(out_big[:, :16]))


@pytest.mark.gpu
def test_linear_small_m_rejects_unsupported_shapes(gpu):
    x = torch.zeros(17, 2048, device=gpu, dtype=torch.bfloat16)
    w = torch.zeros(16, 2048, device=gpu, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="m <= 16"):
        rk.linear_small_m(x, w)
    with pytest.raises(RuntimeError, match="multiple"):
        rk.linear_small_m(x[:4, :1024], w[:, :1024])


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,inter,k", [(8, 14336, 4096), (3, 256, 2048), (16, 64, 6144), (1, 8, 2048)])
def test_linear_silu_mul_equals_the_projection_then_silu_mul(gpu, dtype, m, inter, k):
    """The fused gate/up projection + SiLU * up is bit-identical to
    linear_small_m followed by silu_mul (same K sums, same rounding steps)."""
    log_case(test="linear-silu-mul", dtype=str(dtype), m=m, inter=inter, k=k)
    g = torch.Generator(device=gpu).manual_seed(inter + k + m)
    x = (2 * torch.randn(m, k, generator=g, device=gpu)).to(dtype)
    w = (torch.randn(2 * inter, k, generator=g, device=gpu) / k ** 0.5).to(dtype)
    fused = rk.linear_silu_mul(x, w)
    two = rk.silu_mul(rk.linear_small_m(x, w))
    assert fused.shape == (m, inter)
    assert torch.equal(fused, two)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,heads,rope_heads,head_dim,k,bias", [
    (8, 48, 40, 128, 4096, True),   # Llama-3-8B fused q/k/v: 32 q + 8 k heads rotate, 8 v heads do not
    (5, 6, 4, 64, 2048, False),
    (16, 3, 3, 32, 2048, True),
    (1, 2, 1, 16, 2048, False),
    (4, 4, 0, 128, 2048, True),     # no head rotates: the plain projection
])
def test_linear_rope_equals_the_projection_then_rope(gpu, dtype, m, heads, rope_heads, head_dim, k, bias):
    """The fused q/k/v projection + RoPE is bit-identical to linear_small_m
    followed by rope_ on the first rope_heads heads."""
    log_case(test="linear-rope", dtype=str(dtype), m=m, heads=heads, rope_heads=rope_heads, head_dim=head_dim, k=k)
    g = torch.Generator(device=gpu).manual_seed(heads * head_dim + k + m)
    n = heads * head_dim
    x = torch.randn(m, k, generator=g, device=gpu).to(dtype)
    w = (torch.randn(n, k, generator=g, device=gpu) / k ** 0.5).to(dtype)
    b = torch.randn(n, generator=g, device=gpu).to(dtype) if bias else None
    angle = 1000 * torch.rand(m, head_dim // 2, generator=g, device=gpu)
    cos, sin = angle.cos().to(dtype).contiguous(), angle.sin().to(dtype).contiguous()
    fused = rk.linear_rope(x, w, b, rope_heads, head_dim, cos, sin)
    two = rk.linear_small_m(x, w, b)
    if rope_heads:
        rk.rope_(two, rope_heads, head_dim, cos, sin)
    assert torch.equal(fused, two)


@pytest.mark.gpu
def test_fused_linear_forms_reject_unsupported_shapes(gpu):
    x = torch.zeros(4, 2048, device=gpu, dtype=torch.bfloat16)
    cos = torch.zeros(4, 8, device=gpu, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="multiple of 8"):
        rk.linear_silu_mul(x, torch.zeros(12, 2048, device=gpu, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="multiple of 16"):
        rk.linear_rope(x, torch.zeros(48, 2048, device=gpu, dtype=torch.bfloat16), None, 1, 24,
                       torch.zeros(4, 12, device=gpu, dtype=torch.bfloat16), torch.zeros(4, 12, device=gpu,
                                                                                           dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="rope_heads"):
        rk.linear_rope(x, torch.zeros(32, 2048, device=gpu, dtype=torch.bfloat16), None, 3, 16, cos, cos)
    with pytest.raises(RuntimeError, match="multiple of 2048"):
        rk.linear_silu_mul(x[:, :1024], torch.zeros(16, 1024, device=gpu, dtype=torch.bfloat16))
