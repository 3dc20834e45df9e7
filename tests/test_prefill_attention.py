"""Causal GQA prefill attention (nhs_prefill_attention) against an fp32
reference of the dense causal softmax attention that Model.prefill computes
(reference model.py:170-180): bf16 within 2e-2 and fp16 within 1e-2 max-abs,
over ragged lengths (not multiples of the 64-row tiles), GQA groups of 1, 4
and 7, head_dim 64 and 128, and strided q/k/v views of one fused projection."""

import pytest
import torch

from nano_hisparse import row_kernels as rk


def reference(q, k, v):
    S, Hq, D = q.shape
    g = Hq // k.shape[1]
    qf = q.float().transpose(0, 1)  # [Hq, S, D]
    kf = k.float().repeat_interleave(g, 1).transpose(0, 1).contiguous()
    vf = v.float().repeat_interleave(g, 1).transpose(0, 1).contiguous()
    scores = torch.matmul(qf, kf.transpose(1, 2).contiguous()) / D**0.5
    mask = torch.ones(S, S, dtype=torch.bool, device=q.device).triu(1)
    scores.masked_fill_(mask, float("-inf"))
    return torch.matmul(scores.softmax(-1), vf).transpose(0, 1)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 2e-2), (torch.float16, 1e-2)])
@pytest.mark.parametrize("S,Hq,Hkv,D", [(1, 8, 8, 128), (7, 4, 1, 64), (64, 8, 2, 128), (65, 28, 4, 128),
                                          (200, 32, 8, 128), (1000, 8, 2, 64), (513, 4, 4, 128)])
def test_prefill_attention_matches_fp32_reference(gpu, dtype, tol, S, Hq, Hkv, D):
    print("case:", dict(S=S, Hq=Hq, Hkv=Hkv, D=D, dtype=str(dtype)), flush=True)
    g = torch.Generator(device=gpu).manual_seed(S * 31 + Hq)
    fused = torch.randn(S, (Hq + 2 * Hkv) * D, generator=g, device=gpu).to(dtype)
    q = fused[:, : Hq * D].view(S, Hq, D)
    k = fused[:, Hq * D: (Hq + Hkv) * D].view(S, Hkv, D)
    v = fused[:, (Hq + Hkv) * D:].view(S, Hkv, D)
    out = rk.prefill_attention(q, k, v)
    want = reference(q, k, v)
    err = (out.float() - want).abs().max().item()
    assert err <= tol, err


@pytest.mark.gpu
def test_prefill_attention_rejects_unsupported_inputs(gpu):
    q = torch.randn(8, 4, 96, device=gpu, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="head_dim"):
        rk.prefill_attention(q, q[:, :2], q[:, :2])
    with pytest.raises(ValueError, match="bf16 or fp16"):
        x = torch.randn(8, 4, 64, device=gpu)
        rk.prefill_attention(x, x, x)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_model_prefill_runs_the_flash_kernel(gpu, dtype, monkeypatch):
    """A bf16/fp16 GPU model's prefill calls nhs_prefill_attention; its
    logits match the same model with the attention swapped for the fp32
    reference (rounded to the model dtype)."""
    from nano_hisparse.model import Model, ModelConfig

    print("case:", dict(test="model-prefill", dtype=str(dtype)), flush=True)
    torch.manual_seed(3)
    cfg = ModelConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                      num_key_value_heads=2, vocab_size=128)
    model = Model(cfg).to(gpu, dtype).eval()
    tokens = list(torch.randint(0, 128, (150,)).tolist())
    calls = []
    kernel = rk.prefill_attention

    def counted(q, k, v):
        calls.append(q.shape)
        return kernel(q, k, v)

    monkeypatch.setattr(rk, "prefill_attention", counted)
    got = model.prefill(tokens)
    assert len(calls) == cfg.num_hidden_layers
    monkeypatch.setattr(rk, "prefill_attention", lambda q, k, v: reference(q, k, v).to(q.dtype))
    want = model.prefill(tokens)
    err = (got - want).abs().max().item()
    assert err <= 5e-2 * max(1.0, want.abs().max().item()), err
