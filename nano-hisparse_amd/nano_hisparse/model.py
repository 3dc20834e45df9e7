"""A small Qwen2-shaped decoder that drives the sparse decode path.

Reference: nano_hisparse/model.py:19-221. Dense layers (projections, RoPE,
RMSNorm, SwiGLU) are torch operations, the prefill's causal attention of a
bf16/fp16 GPU model is the MFMA flash kernel (nhs_prefill_attention); each
decode step appends K/V through the cache, selects pages with Quest on the
GPU and attends over the selected rows with the HIP kernels. The module tree
(names and construction order) is the reference's, which is HF Qwen2's, so
state dicts load either way and a seeded random init draws the same weights.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import nn
from torch.nn import functional as F

from .selection import Selection, quest_selection, select_pages
from .storage import upload


@dataclass
class ModelConfig:
    vocab_size: int = 256
    hidden_size: int = 128
    intermediate_size: int = 256
    num_hidden_layers: int = 2
    num_attention_heads: int = 4
    num_key_value_heads: int = 2
    rms_norm_eps: float = 1e-6
    rope_theta: float = 10000.0

    @property
    def head_dim(self):
        return self.hidden_size // self.num_attention_heads

    def __post_init__(self):
        if (
            self.hidden_size % self.num_attention_heads
            or self.num_attention_heads % self.num_key_value_heads
            or self.head_dim % 2
        ):
            raise ValueError("model dimensions must support grouped-query attention and RoPE")


class RMSNorm(nn.Module):
    def __init__(self, width, eps):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(width))
        self.eps = eps

    def forward(self, x):
        xf = x.float()
        return (xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + self.eps)).to(x.dtype) * self.weight


class Projections(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        kv_width = cfg.num_key_value_heads * cfg.head_dim
        self.q_proj = nn.Linear(cfg.hidden_size, cfg.hidden_size, bias=True)
        self.k_proj = nn.Linear(cfg.hidden_size, kv_width, bias=True)
        self.v_proj = nn.Linear(cfg.hidden_size, kv_width, bias=True)
        self.o_proj = nn.Linear(cfg.hidden_size, cfg.hidden_size, bias=False)


class MLP(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.gate_proj = nn.Linear(cfg.hidden_size, cfg.intermediate_size, bias=False)
        self.up_proj = nn.Linear(cfg.hidden_size, cfg.intermediate_size, bias=False)
        self.down_proj = nn.Linear(cfg.intermediate_size, cfg.hidden_size, bias=False)

    def forward(self, x):
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class Block(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.input_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.self_attn = Projections(cfg)
        self.mlp = MLP(cfg)


class Decoder(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.layers = nn.ModuleList(Block(cfg) for _ in range(cfg.num_hidden_layers))
        self.norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)


class Model(nn.Module):
    def __init__(self, config: ModelConfig | None = None):
        super().__init__()
        self.config = config or ModelConfig()
        self.model = Decoder(self.config)
        self.lm_head = nn.Linear(self.config.hidden_size, self.config.vocab_size, bias=False)

    @classmethod
    def from_pretrained(cls, name: str, device="cuda", dtype=torch.bfloat16):
        """Qwen2/Qwen2.5 weights with standard RoPE from a local directory or
        an already-cached hub name (no network is assumed)."""
        from transformers import AutoConfig, AutoModelForCausalLM

        hf_cfg = AutoConfig.from_pretrained(name)
        rope = getattr(hf_cfg, "rope_parameters", None) or getattr(hf_cfg, "rope_scaling", None) or {}
        if hf_cfg.model_type != "qwen2" or rope.get("rope_type", rope.get("type", "default")) != "default":
            raise ValueError("only Qwen2/Qwen2.5 with standard RoPE are supported")
        if getattr(hf_cfg, "use_sliding_window", False) or hf_cfg.hidden_act != "silu":
            raise ValueError("sliding window / non-SiLU models are unsupported")
        hf = AutoModelForCausalLM.from_pretrained(name, torch_dtype=dtype).eval().to(device)
        model = cls.__new__(cls)
        nn.Module.__init__(model)
        fields = {f: getattr(hf_cfg, f) for f in ModelConfig.__dataclass_fields__ if f != "rope_theta"}
        fields["rope_theta"] = rope.get("rope_theta", getattr(hf_cfg, "rope_theta", 10000.0))
        model.config = ModelConfig(**fields)
        model.model, model.lm_head = hf.model, hf.lm_head
        return model.eval()

    @property
    def device(self):
        return self.model.embed_tokens.weight.device

    @property
    def dtype(self):
        return self.model.embed_tokens.weight.dtype

    def _project(self, layer, x, start):
        """RMSNorm, q/k/v projections and rotary embedding for tokens at
        positions start .. start + len(x) - 1."""
        return self._project_at(layer, x, torch.arange(start, start + len(x), device=x.device))

    def _project_at(self, layer, x, positions):
        """_project for rows at arbitrary positions (an int tensor [len(x)])."""
        cfg, n = self.config, len(x)
        h = layer.input_layernorm(x)
        attn = layer.self_attn
        q = attn.q_proj(h).view(n, cfg.num_attention_heads, cfg.head_dim)
        k = attn.k_proj(h).view(n, cfg.num_key_value_heads, cfg.head_dim)
        v = attn.v_proj(h).view(n, cfg.num_key_value_heads, cfg.head_dim)
        inv_freq = cfg.rope_theta ** (-torch.arange(0, cfg.head_dim, 2, device=x.device).float() / cfg.head_dim)
        angle = positions.float()[:, None] * inv_freq[None, :]
        angle = torch.cat((angle, angle), -1)[:, None, :]
        cos, sin = angle.cos().to(x.dtype), angle.sin().to(x.dtype)

        def rope(t):
            lo, hi = t.chunk(2, -1)
            return t * cos + torch.cat((-hi, lo), -1) * sin

        return rope(q), rope(k), v

    @staticmethod
    def _finish(layer, residual, attention):
        x = residual + layer.self_attn.o_proj(attention.reshape(len(residual), -1))
        return x + layer.mlp(layer.post_attention_layernorm(x))

    @torch.inference_mode()
    def prefill(self, tokens: list[int], cache=None, request_id=None):
        """Dense causal forward over the prompt, writing K/V to the cache;
        returns the last position's logits (fp32)."""
        if not tokens:
            raise ValueError("prompt cannot be empty")
        if cache is not None and any(cache.storage.requests[request_id].lengths):
            raise ValueError("prefill is allowed exactly once per request")
        cfg = self.config
        groups = cfg.num_attention_heads // cfg.num_key_value_heads
        # bf16/fp16 models on a GPU run the causal attention as the MFMA
        # flash kernel (nhs_prefill_attention): O(S) memory where the dense
        # path materialises S x S scores per head; fp32 and CPU models keep
        # the dense causal attention.
        flash = (self.device.type == "cuda" and self.dtype in (torch.bfloat16, torch.float16)
                 and cfg.head_dim in (64, 128))
        if flash:
            from . import row_kernels as rk
        x = self.model.embed_tokens(upload(tokens, torch.int64, self.device))
        for index, layer in enumerate(self.model.layers):
            q, k, v = self._project(layer, x, 0)
            if cache is not None:
                cache.write(request_id, index, k, v)
            if flash:
                attention = rk.prefill_attention(q, k, v)
            else:
                attention = F.scaled_dot_product_attention(
                    q.transpose(0, 1),
                    k.repeat_interleave(groups, 1).transpose(0, 1),
                    v.repeat_interleave(groups, 1).transpose(0, 1),
                    is_causal=True,
                ).transpose(0, 1)
            x = self._finish(layer, x, attention)
        return self.lm_head(self.model.norm(x[-1])).float()

    @torch.inference_mode()
    def decode(self, token: int, request_id, cache, top_k=None, backend="auto", selector="quest"):
        """One decode step: per layer append K/V, select (Quest top_k pages,
        or the page-mean selector, or everything for top_k=None) and attend
        over the selected rows. Returns fp32 logits."""
        lengths = cache.storage.requests[request_id].lengths
        if len(set(lengths)) != 1 or lengths[0] == 0:
            raise ValueError("all layers must have the same nonempty history")
        position = lengths[0]
        P = cache.config.page_size
        x = self.model.embed_tokens(upload([token], torch.int64, self.device))
        for index, layer in enumerate(self.model.layers):
            q, k, v = self._project(layer, x, position)
            cache.write(request_id, index, k, v)
            request = cache.storage.requests[request_id]
            if selector == "quest" and top_k is not None:
                selection = quest_selection(
                    q[0], request.minimum[index], request.maximum[index], request.lengths[index], P, top_k
                )
            elif selector in ("quest", "mean"):
                pages = select_pages(cache, request_id, index, q[0], top_k)
                selection = Selection.from_pages(pages, request.lengths[index], P, q.shape[1])
            else:
                raise ValueError("selector must be quest or mean")
            attention = cache.attention(q[0], request_id, index, selection, backend)
            x = self._finish(layer, x, attention.unsqueeze(0))
        return self.lm_head(self.model.norm(x[0])).float()

    def _fused_projections(self):
        """Per layer: the q/k/v weights and biases and the gate/up weights as
        one tensor each, for one GEMM apiece in the batched decode. The
        module parameters become views of the fused tensors (names, state
        dicts and the per-request path are unchanged); fusing again happens
        only if a parameter was replaced since (e.g. by .to())."""
        fused = getattr(self, "_fused", None)
        if fused is not None and fused[0] == self._projection_pointers():
            return fused[1]
        layers = []
        for layer in self.model.layers:
            attn, mlp = layer.self_attn, layer.mlp
            qkv = (attn.q_proj, attn.k_proj, attn.v_proj)
            layers.append((_fuse(qkv, "weight"), _fuse(qkv, "bias"), _fuse((mlp.gate_proj, mlp.up_proj), "weight")))
        self._fused = (self._projection_pointers(), layers)
        return layers

    def _projection_pointers(self):
        out = []
        for layer in self.model.layers:
            attn, mlp = layer.self_attn, layer.mlp
            for m in (attn.q_proj, attn.k_proj, attn.v_proj, mlp.gate_proj, mlp.up_proj):
                out.append(m.weight.data_ptr())
        return out

    @torch.inference_mode()
    def decode_batch(self, tokens: list[int], request_ids: list, cache, top_k: int, micro_batches: int = 1,
                     graph: bool = False):
        """One decode step for several requests at once (Quest top_k pages).

        Dense layers run on the batch with fused projections (one q/k/v
        GEMM, one gate/up GEMM) and libnhs_hip.so's fused residual-add +
        RMSNorm, RoPE (cos/sin computed once per step) and SiLU * up
        kernels; the sparse stages run once per layer for all requests
        (cache.decode_batch). With micro_batches=2 the requests form two
        groups that run half a layer apart, so each group's host-row gather
        (transfer stream) runs beside the other group's layer compute; the
        gather's grid is capped meanwhile to leave compute units to that
        work. Returns fp32 logits [B, vocab]; row b equals decode(tokens[b],
        request_ids[b]) up to the order of the dense layers' reductions.

        graph=True (one group) replays the step's launches from a HIP graph
        captured at the first step of this batch composition (see
        _decode_batch_graph): the same kernels on the same buffers, with no
        per-launch host work."""
        from . import row_kernels as rk

        if len(tokens) != len(request_ids):
            raise ValueError("one token per request")
        if top_k is None or top_k < 1:
            raise ValueError("batched decode needs a positive Quest top_k")
        if micro_batches not in (1, 2):
            raise ValueError("micro_batches must be 1 or 2")
        n = len(tokens)
        if n < 2:
            micro_batches = 1
        cuts = [0, n] if micro_batches == 1 else [0, (n + 1) // 2, n]
        if graph:
            return self._decode_batch_graph(tokens, request_ids, cache, top_k, cuts)
        overlap = len(cuts) > 2
        groups = [_Group(self, tokens[a:b], request_ids[a:b], cache, overlap) for a, b in zip(cuts, cuts[1:])]
        logits = self._run_groups(groups, top_k)
        for g in groups:
            g.step.end()
        return logits

    def _run_groups(self, groups, top_k):
        """Every layer of one group, or of two groups half a layer apart (each
        group's gather on the transfer stream beside the other's compute,
        with the gather's grid capped meanwhile), then the final norm and the
        lm_head; returns the logits."""
        from . import row_kernels as rk

        fused = self._fused_projections()
        layers = self.model.layers
        if len(groups) == 1:
            g = groups[0]
            for index, layer in enumerate(layers):
                g.pre(index, layer, fused[index], top_k)
                g.post(layer)
        else:
            a, b = groups
            rk.set_gather_workgroups(32)
            try:
                a.pre(0, layers[0], fused[0], top_k)
                b.pre(0, layers[0], fused[0], top_k)
                for index, layer in enumerate(layers):
                    following = index + 1 < len(layers)
                    a.post(layer)
                    if following:
                        a.pre(index + 1, layers[index + 1], fused[index + 1], top_k)
                    b.post(layer)
                    if following:
                        b.pre(index + 1, layers[index + 1], fused[index + 1], top_k)
            finally:
                rk.set_gather_workgroups(0)
        x = groups[0].x + groups[0].delta if len(groups) == 1 else torch.cat([g.x + g.delta for g in groups])
        return _linear(self.model.norm(x), self.lm_head.weight, self.lm_head.bias).float()


    def clear_decode_graphs(self):
        """Drops every captured decode-step graph, with the cache, buffers and
        graph memory each one holds."""
        self.__dict__.pop("_decode_graphs", None)

    def _decode_batch_graph(self, tokens, request_ids, cache, top_k, cuts):
        """decode_batch with the step's launches (every layer of every group,
        the final norm and the lm_head) captured once per batch composition
        into a HIP graph and replayed from then on. With two groups (cuts
        [0, m, n]) the capture holds both groups' schedule: each gather is a
        branch forked from the capture stream by an event and joined back by
        the attention that waits for it, so the replay runs it beside the
        other group's compute as the eager steps do.

        Per step, outside the graph: the page placement and residency policy
        (BatchDecode's constructor; its table writes precede the replay on
        the compute stream), the upload of the lengths and token ids into the
        buffers the graph reads, the waits for the tables' pending events,
        and after the replay the pages' host state and the policy tick
        (end()). Every launch's shape depends only on the batch, the budget
        and the requests' reserved pages, so the replayed step is the eager
        one. A graph is reused only while the cache's device item tables of
        the groups are the same objects (they hold the pointers the graph
        read); otherwise it is captured again."""
        store = cache.storage
        store.check_stream()
        graphs = self.__dict__.setdefault("_decode_graphs", {})
        # graphs captured against another cache hold that cache (its pool),
        # their buffers and their private memory: drop them
        for stale in [k for k, e in graphs.items() if e["cache"] is not cache]:
            del graphs[stale]
        spans = list(zip(cuts, cuts[1:]))
        overlap = len(spans) > 1
        key = (tuple(request_ids), top_k, len(spans))
        items = [cache._layer_items(request_ids[a:b]) for a, b in spans]
        entry = graphs.get(key)
        if entry is not None and (entry["cache"] is not cache or any(x is not y for x, y in zip(entry["items"], items))):
            del graphs[key]
            entry = None
        token_ids = [torch.tensor(tokens[a:b], dtype=torch.int64).pin_memory() for a, b in spans]

        def open_steps(buffers):
            steps = []
            for (a, b), (lengths, _) in zip(spans, buffers):
                step = cache.decode_batch(request_ids[a:b], overlap, lengths_buffer=lengths)
                step.sync_tables()
                step.clear_reads()
                steps.append(step)
            for (_, ids), t in zip(buffers, token_ids):
                ids.copy_(t, non_blocking=True)
            return steps

        if entry is None:
            buffers = [(torch.empty(2, b - a, dtype=torch.int64, device=cache.device),
                        torch.empty(b - a, dtype=torch.int64, device=cache.device)) for a, b in spans]
            steps = open_steps(buffers)
            graph = torch.cuda.CUDAGraph()
            side = torch.cuda.Stream(device=cache.device)
            side.wait_stream(store.compute)
            if overlap:
                side.wait_stream(store.transfer)
            with store.capturing(side), torch.cuda.graph(graph, stream=side):
                groups = [_Group(self, None, request_ids[a:b], cache, overlap, step=step, ids=ids)
                          for (a, b), step, (_, ids) in zip(spans, steps, buffers)]
                logits = self._run_groups(groups, top_k)
            for step in steps:
                step.forget_capture_events()
            # the capture stream lives as long as the graph: buffers cached per stream during the capture
            # (the attention workspace) belong to the graph's memory
            entry = {"cache": cache, "items": items, "buffers": buffers, "graph": graph, "logits": logits,
                     "stream": side}
            graphs[key] = entry
            while len(graphs) > 8:  # the most recent compositions keep their graphs
                del graphs[next(iter(graphs))]
        else:
            steps = open_steps(entry["buffers"])
            for step in steps:
                step.account_replayed()
        entry["graph"].replay()
        for step in steps:
            step.end()
        return entry["logits"].clone()


class _Group:
    """One batch group of decode_batch: its residual stream, RoPE tables,
    cache step and the gather handle in flight."""

    def __init__(self, model, tokens, request_ids, cache, overlap, step=None, ids=None):
        cfg = model.config
        self.model, self.cfg = model, cfg
        self.step = cache.decode_batch(request_ids, overlap) if step is None else step
        D = cfg.head_dim
        positions = self.step.dev_lengths[0]  # already on the device
        inv_freq = cfg.rope_theta ** (-torch.arange(0, D, 2, device=model.device).float() / D)
        angle = positions.float()[:, None] * inv_freq[None, :]
        self.cos = angle.cos().to(model.dtype).contiguous()
        self.sin = angle.sin().to(model.dtype).contiguous()
        if ids is None:
            ids = torch.tensor(tokens, dtype=torch.int64).pin_memory().to(model.device, non_blocking=True)
        self.x = model.model.embed_tokens(ids).contiguous()
        self.delta = None
        self.handle = None

    def pre(self, index, layer, fused, top_k):
        """Norm, projections, RoPE, append, selection; the gather is left in flight."""
        from . import row_kernels as rk

        cfg, B = self.cfg, len(self.x)
        D, Hq, Hkv = cfg.head_dim, cfg.num_attention_heads, cfg.num_key_value_heads
        qkv_w, qkv_b, _ = fused
        self.gu_w = fused[2]
        h = rk.add_rmsnorm(self.x, self.delta, layer.input_layernorm.weight, _eps(layer.input_layernorm, cfg))
        if _small_m(h, qkv_w, qkv_b) and D % 16 == 0:  # projection and RoPE in one launch
            qkv = rk.linear_rope(h, qkv_w, qkv_b, Hq + Hkv, D, self.cos, self.sin)
        else:
            qkv = _linear(h, qkv_w, qkv_b)
            rk.rope_(qkv, Hq + Hkv, D, self.cos, self.sin)
        q = qkv[:, : Hq * D].view(B, Hq, D)
        k = qkv[:, Hq * D: (Hq + Hkv) * D].view(B, Hkv, D)
        v = qkv[:, (Hq + Hkv) * D:].view(B, Hkv, D)
        self.step.append(index, k, v)
        self.handle = self.step.select(index, q, top_k)

    def post(self, layer):
        """Attention once the gather is in, output projection, MLP."""
        from . import row_kernels as rk

        cfg, B = self.cfg, len(self.x)
        attention = self.step.finish(self.handle)
        o_proj = layer.self_attn.o_proj
        o = _linear(attention.reshape(B, -1), o_proj.weight, o_proj.bias)
        norm2 = layer.post_attention_layernorm
        h = rk.add_rmsnorm(self.x, o, norm2.weight, _eps(norm2, cfg))
        down = layer.mlp.down_proj
        if _small_m(h, self.gu_w, None) and self.gu_w.shape[0] % 16 == 0:  # gate/up and SiLU in one launch
            act = rk.linear_silu_mul(h, self.gu_w)
        else:
            act = rk.silu_mul(_linear(h, self.gu_w, None))
        self.delta = _linear(act, down.weight, down.bias)

def _linear(x, weight, bias):
    """x @ weight.T + bias for a decode batch: the MFMA weight-stream kernel
    (nhs_linear_small_m) for bf16/fp16 batches of up to 16 rows whose shapes
    it takes, else torch."""
    from . import row_kernels as rk

    if _small_m(x, weight, bias):
        return rk.linear_small_m(x, weight, bias)
    return F.linear(x, weight, bias)


def _small_m(x, weight, bias):
    """Whether the decode projection x @ weight.T (+ bias) fits the
    weight-stream kernels (nhs_linear_small_m and its fused forms)."""
    m, k = x.shape
    n = weight.shape[0]
    return (x.is_cuda and x.dtype in (torch.bfloat16, torch.float16) and weight.dtype == x.dtype and m <= 16
            and n % 16 == 0 and k % 2048 == 0 and x.stride(1) == 1 and weight.is_contiguous()
            and (bias is None or bias.is_contiguous()))


def _eps(norm, cfg):
    return getattr(norm, "eps", getattr(norm, "variance_epsilon", cfg.rms_norm_eps))


def _fuse(modules, name):
    """Concatenate the modules' `name` parameters along dim 0 and make each
    module's parameter a view of the result (None if any is missing)."""
    params = [getattr(m, name) for m in modules]
    if any(p is None for p in params):
        return None
    whole = torch.cat([p.detach() for p in params], 0)
    row = 0
    for m, p in zip(modules, params):
        n = p.shape[0]
        setattr(m, name, nn.Parameter(whole[row: row + n], requires_grad=p.requires_grad))
        row += n
    return whole
