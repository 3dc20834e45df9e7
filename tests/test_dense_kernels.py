"""The batched decode layer's fused elementwise kernels against the torch
expressions they replace (reference model.py:43-71, 140-158), and the fused
batched model step against per-request decoding.

RoPE and the residual adds reproduce torch's roundings exactly (bit-exact);
RMSNorm's mean and SiLU's exp may differ from torch's by their last fp32
bits. For SiLU that shows as at most one unit in the last place after
rounding to bf16/fp16; RMSNorm rounds twice after the mean
(round(round(h * r) * weight)), so a flip of the inner rounding by one unit
can become two units of the output (seen at fp16, 4 x 8192: 0.46 * r rounds
one unit apart, times a weight of 1.06 two units apart). fp32: a relative
1e-6.
"""

import pytest
import torch
from torch.nn import functional as F

from nano_hisparse import row_kernels as rk
from nano_hisparse.config import CacheConfig
from nano_hisparse.hybrid import HotConfig, HybridKVCache
from nano_hisparse.model import Model, ModelConfig, RMSNorm

DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def ulp_close(a, b, units=1):
    """|a - b| within `units` units in the last place of b's dtype (fp32: a
    relative 1e-6 per unit, the spread of the mean's reduction order over
    rows of thousands)."""
    a, b = a.float(), b.float()
    eps = units * {torch.float32: 1e-6, torch.float16: 2.0**-10, torch.bfloat16: 2.0**-7}[ULP_DTYPE[0]]
    tiny = {torch.float32: 1e-30, torch.float16: 6e-8, torch.bfloat16: 1e-30}[ULP_DTYPE[0]]
    return bool(((a - b).abs() <= eps * b.abs() + tiny).all())


ULP_DTYPE = [torch.float32]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
def test_add_rmsnorm_matches_torch(gpu, dtype):
    ULP_DTYPE[0] = dtype
    g = torch.Generator(device=gpu).manual_seed(1)
    for rows, width in ((8, 4096), (16, 3584), (2, 512), (4, 8192), (3, 96), (1, 1000), (2, 8704), (3, 1004)):
        x = torch.randn(rows, width, generator=g, device=gpu).to(dtype)
        delta = torch.randn(rows, width, generator=g, device=gpu).to(dtype)
        norm = RMSNorm(width, 1e-6).to(gpu)
        norm.weight.data = (1 + 0.1 * torch.randn(width, generator=g, device=gpu)).to(dtype)
        want_h = x + delta
        want = norm(want_h)
        got_x = x.clone()
        got = rk.add_rmsnorm(got_x, delta, norm.weight, 1e-6)
        assert torch.equal(got_x, want_h)  # the residual add is exact
        assert ulp_close(got, want, units=2), (rows, width)
        plain = rk.add_rmsnorm(x.clone(), None, norm.weight, 1e-6)
        assert ulp_close(plain, norm(x), units=2), (rows, width)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
def test_rope_matches_the_torch_rotation_bit_exactly(gpu, dtype):
    g = torch.Generator(device=gpu).manual_seed(2)
    rows, heads, D, extra = 5, 12, 64, 3 * 64
    t = torch.randn(rows, heads * D + extra, generator=g, device=gpu).to(dtype)
    angle = torch.rand(rows, D // 2, generator=g, device=gpu) * 1000
    cos, sin = angle.cos().to(dtype), angle.sin().to(dtype)
    # the model's expression: t * cos + cat(-hi, lo) * sin with cos/sin repeated
    view = t[:, : heads * D].view(rows, heads, D)
    c2, s2 = torch.cat((cos, cos), -1)[:, None, :], torch.cat((sin, sin), -1)[:, None, :]
    lo, hi = view.chunk(2, -1)
    want = view * c2 + torch.cat((-hi, lo), -1) * s2
    tail = t[:, heads * D:].clone()
    rk.rope_(t, heads, D, cos.contiguous(), sin.contiguous())
    assert torch.equal(t[:, : heads * D].view(rows, heads, D), want)
    assert torch.equal(t[:, heads * D:], tail)  # v columns untouched


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
def test_silu_mul_matches_torch(gpu, dtype):
    ULP_DTYPE[0] = dtype
    g = torch.Generator(device=gpu).manual_seed(3)
    gu = (3 * torch.randn(8, 2 * 1000, generator=g, device=gpu)).to(dtype)
    want = F.silu(gu[:, :1000]) * gu[:, 1000:]
    assert ulp_close(rk.silu_mul(gu), want)


@pytest.mark.gpu
# (2048, 16, 4): q/k/v and o take nhs_linear_small_m in bf16
@pytest.mark.parametrize("hidden,heads,kv_heads", [(128, 8, 2), (2048, 16, 4)])
@pytest.mark.parametrize("micro_batches", [1, 2])
@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 0.15)])
def test_fused_batched_step_matches_per_request_decode(gpu, dtype, tol, micro_batches, hidden, heads, kv_heads):
    print("case:", dict(dtype=str(dtype), micro_batches=micro_batches, hidden=hidden), flush=True)
    torch.manual_seed(7)
    cfg = ModelConfig(hidden_size=hidden, intermediate_size=2 * hidden, num_hidden_layers=2,
                      num_attention_heads=heads, num_key_value_heads=kv_heads, vocab_size=100)
    model = Model(cfg).eval().to(gpu).to(dtype)
    caches = [
        HybridKVCache(CacheConfig(gpu_pages=64, host_pages=256, page_size=4, kv_heads=kv_heads,
                                  head_dim=hidden // heads, dtype=dtype, device=gpu),
                      HotConfig(16, 32, resident_window_pages=4))
        for _ in range(2)
    ]
    prompts = {"a": list(range(3, 40)), "b": list(range(1, 23)), "c": list(range(9, 60))}
    tokens = {}
    for c in caches:
        for name, prompt in prompts.items():
            c.reserve(name, len(prompt) + 16, cfg.num_hidden_layers)
            tokens[name] = int(model.prefill(prompt, c, name).argmax())
    for _ in range(6):
        batch = model.decode_batch([tokens[n] for n in prompts], list(prompts), caches[1], 4, micro_batches)
        for i, name in enumerate(prompts):
            single = model.decode(tokens[name], name, caches[0], top_k=4)
            scale = single.abs().max().item()
            assert (batch[i] - single).abs().max().item() <= tol * max(scale, 1.0), name
        tokens = {n: int(batch[i].argmax()) for i, n in enumerate(prompts)}
    for c in caches:
        c.assert_invariants()
