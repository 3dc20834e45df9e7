"""Token-row traces: capture from a dense teacher, replay through the cache.

Reference: nano_hisparse/trace.py:14-291. A trace is a dict (schema 2: one
shared token list per event; schema 1: one list per query head) holding a
prefill K/V and a sequence of decode events {q, k, v, positions}. Replay
appends each event to a one-layer HybridKVCache, resolves and gathers the
selected rows through the HIP resolver and gather kernels, attends over them
with the HIP attention kernel, checks the output against a dense masked
softmax, and reports per-step locality (row/page Jaccard, page density,
reuse gaps, hot slots as logical tokens) and the cache's row counters.
Replay synchronizes for its diagnostics; it is not a timing path.
"""

from __future__ import annotations

import json
from hashlib import sha256
from math import ceil
from statistics import mean

import torch

from .config import CacheConfig
from .hybrid import HotConfig, HybridKVCache
from .selection import Selection, selection_oracle

PATTERNS = ("reuse", "alternating", "streaming", "packed")


def token_topk(query, keys, count):
    """Top-`count` token rows by the query-head mean of q . k (fp32);
    reference trace.py:14-20. query [Hq, D], keys [T, Hkv, D]; returned in
    descending score order."""
    if count < 1:
        raise ValueError("token count must be positive")
    q_heads, kv_heads = query.shape[0], keys.shape[1]
    per_group = q_heads // kv_heads
    q = query.float().reshape(kv_heads, per_group, -1)  # [Hkv, g, D]
    k = keys.float().permute(1, 2, 0)  # [Hkv, D, T]
    scores = torch.bmm(q, k.contiguous()).reshape(q_heads, -1)  # [Hq, T]
    return scores.mean(0).topk(min(count, keys.shape[0])).indices.tolist()


def _rows_of(pattern, step):
    """Token rows read at `step` by each synthetic access pattern (four rows
    per step over a 64-token prefill of 16 pages of 4)."""
    if pattern == "packed":
        return [0, 1, 2, 3]
    if pattern == "streaming":
        return [step, 16 + step, 32 + step, 48 + step]
    shift = step % 2 if pattern == "alternating" else 0
    return [shift, 4 + shift, 8 + shift, 12 + shift]


def synthetic_trace(pattern, steps=8, seed=42):
    """A controlled access pattern over one KV head of width 8 and two query
    heads; tensors come from a seeded CPU generator in a fixed draw order
    (prefill K, prefill V, then q, k, v per event), so a trace is the same
    on every machine (reference trace.py:23-53)."""
    if pattern not in PATTERNS:
        raise ValueError("unknown access pattern")
    if not 2 <= steps <= 8:
        raise ValueError("synthetic traces support 2..8 steps")
    gen = torch.Generator().manual_seed(seed)

    def draw(*shape):
        return torch.randn(*shape, generator=gen)

    prefill = {"k": draw(64, 1, 8), "v": draw(64, 1, 8)}
    events = []
    for step in range(steps):
        q, k, v = draw(2, 8), draw(1, 1, 8), draw(1, 1, 8)
        events.append({"q": q, "k": k, "v": v, "positions": _rows_of(pattern, step)})
    return {
        "schema_version": 2,
        "source": {"kind": "synthetic", "pattern": pattern, "seed": seed},
        "page_size": 4,
        "prefill": prefill,
        "events": events,
    }


def _check_event(event, k):
    q, new_k, new_v = event["q"], event["k"], event["v"]
    row_shape = (1, *k.shape[1:])
    ok = (
        new_k.shape == row_shape
        and new_v.shape == row_shape
        and new_k.dtype == new_v.dtype == q.dtype == k.dtype
        and q.ndim == 2
        and q.shape[0] >= 1
        and q.shape[1] == k.shape[2]
        and q.shape[0] % k.shape[1] == 0
    )
    if not ok:
        raise ValueError("incompatible event Q/K/V")


def validate_trace(trace):
    """Checks a trace and returns the largest union of selected rows over
    its events (reference trace.py:56-94)."""
    if trace.get("schema_version") not in (1, 2) or not isinstance(trace.get("source"), dict):
        raise ValueError("trace requires schema_version=1 or 2 and source metadata")
    if not trace.get("events"):
        raise ValueError("trace needs at least one event")
    k, v = trace["prefill"]["k"], trace["prefill"]["v"]
    if k.ndim != 3 or k.shape != v.shape or min(k.shape) < 1 or k.dtype != v.dtype:
        raise ValueError("invalid prefill KV")
    if k.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise ValueError("unsupported KV dtype")
    length, widest = k.shape[0], 0
    for event in trace["events"]:
        _check_event(event, k)
        length += 1
        positions = event["positions"]
        if trace["schema_version"] == 2 and (
            not isinstance(positions, (list, tuple)) or not all(isinstance(t, int) for t in positions)
        ):
            raise ValueError("schema_version=2 requires one shared token ID list per query")
        selection = Selection.from_tokens(positions, length, trace["page_size"], event["q"].shape[0])
        widest = max(widest, len(set().union(*selection.positions)))
    return widest


def save_trace(trace, path):
    validate_trace(trace)
    path.parent.mkdir(parents=True, exist_ok=True)
    torch.save(trace, path)


def load_trace(path):
    """Loads a trace with torch's weights-only unpickler (tensors, lists,
    dicts and scalars; nothing in the file is executed)."""
    trace = torch.load(path, map_location="cpu", weights_only=True)
    validate_trace(trace)
    return trace


def _jaccard(current, previous):
    if previous is None:
        return None
    return len(current & previous) / len(current | previous)


def _mean(values):
    """Exact mean (statistics.mean), None for no values."""
    values = list(values)
    return mean(values) if values else None


def _default_device():
    return "cuda:0" if torch.cuda.is_available() else "cpu"


@torch.inference_mode()
def replay_trace(trace, hot_rows=None, device=None):
    """Replays a trace through a fresh one-layer cache on `device` (default:
    the first GPU when there is one). The prefill history is evicted to host
    memory before the first event (only the two protected tail pages stay
    resident, the hot buffer starts empty), so every selected row is a hot
    hit or a miss. hot_rows defaults to the largest row union of the trace.
    Reference trace.py:105-216."""
    device = device or _default_device()
    union_bound = validate_trace(trace)
    P = trace["page_size"]
    k = trace["prefill"]["k"].to(device)
    v = trace["prefill"]["v"].to(device)
    total = k.shape[0] + len(trace["events"])
    hot = HotConfig(union_bound, union_bound if hot_rows is None else hot_rows)
    config = CacheConfig(
        gpu_pages=hot.admission_blocks(P),
        host_pages=ceil(total / P),
        page_size=P,
        kv_heads=k.shape[1],
        head_dim=k.shape[2],
        dtype=k.dtype,
        device=device,
    )
    cache = HybridKVCache(config, hot)
    row_bytes = 2 * config.kv_heads * config.head_dim * k.element_size()
    tolerance = 3e-5 if k.dtype == torch.float32 else 0.008
    records, last_seen, gaps = [], {}, []
    previous_rows = previous_pages = None
    try:
        cache.reserve("trace", total, 1)
        cache.write("trace", 0, k, v)
        cache.storage.synchronize()
        cache.reclaim_history("trace", 0, evict=True)
        cache.reset_stats()
        for step, event in enumerate(trace["events"]):
            q = event["q"].to(device)
            new_k, new_v = event["k"].to(device), event["v"].to(device)
            cache.write("trace", 0, new_k, new_v)
            k, v = torch.cat((k, new_k)), torch.cat((v, new_v))
            length = k.shape[0]
            selection = Selection.from_tokens(event["positions"], length, P, q.shape[0])
            rows = set().union(*selection.positions)
            pages = {t // P for t in rows}
            counters_before = cache.row_stats.clone()
            actual = cache.attention(q, "trace", 0, selection)
            expected, _ = selection_oracle(q, k, v, selection)
            torch.testing.assert_close(actual, expected, atol=tolerance, rtol=tolerance)
            resident, hits, misses = (cache.row_stats - counters_before).cpu().tolist()
            if resident + hits + misses != len(rows):
                raise AssertionError("row counters do not cover the selected rows")
            for token in sorted(rows):
                if token in last_seen:
                    gaps.append(step - last_seen[token])
                last_seen[token] = step
            # hot tags hold host rows: map them back to logical token positions
            page_of_host = {page.host_slot: page.key[2] for page in cache.storage.pages.values()}
            tags = cache.tables["trace", 0].tags.cpu().tolist()
            slots = [None if t < 0 else page_of_host[t // P] * P + t % P for t in tags]
            span = sum(min(P, length - p * P) for p in pages)
            records.append({
                "step": step,
                "length": length,
                "positions": selection.positions[0] if trace["schema_version"] == 2 else selection.positions,
                "union_rows": sorted(rows),
                "selected_pages": sorted(pages),
                "row_jaccard": _jaccard(rows, previous_rows),
                "page_jaccard": _jaccard(pages, previous_pages),
                "page_density": len(rows) / span,
                "resident_hits": resident,
                "hot_hits": hits,
                "misses": misses,
                "h2d_bytes": misses * row_bytes,
                "hot_slots": slots,
                "max_abs_error": (actual.float() - expected.float()).abs().max().item(),
            })
            previous_rows, previous_pages = rows, pages
            cache.assert_invariants()
        totals = cache.snapshot()["row_stats"]
        nonresident = totals["hot_hits"] + totals["misses"]
        later = records[1:]
        summary = {
            **totals,
            "hot_hit_rate": totals["hot_hits"] / nonresident if nonresident else None,
            "unique_rows": len(last_seen),
            "mean_reuse_gap_steps": _mean(gaps),
            "mean_row_jaccard": _mean(r["row_jaccard"] for r in later),
            "mean_page_jaccard": _mean(r["page_jaccard"] for r in later),
            "mean_page_density": _mean(r["page_density"] for r in records),
            "max_abs_error": max(r["max_abs_error"] for r in records),
        }
        return {
            "schema_version": trace["schema_version"],
            "source": trace["source"],
            "device": str(cache.device),
            "dtype": str(k.dtype),
            "page_size": P,
            "row_bytes": row_bytes,
            "max_union_rows": union_bound,
            "hot_rows": hot.hot_rows,
            "gpu_blocks": config.gpu_pages,
            "initial_residency": "history evicted; two tail pages retained; hot empty",
            "summary": summary,
            "events": records,
        }
    finally:
        if "trace" in cache.storage.requests:
            cache.release_request("trace")
        cache.close()


def report_json(report, indent=2):
    """The replay report as JSON text (tuples become lists)."""
    return json.dumps(report, indent=indent, ensure_ascii=False)


@torch.inference_mode()
def capture_trace(model, tokens, steps=8, token_budget=8, layer=0, page_size=16, source=None):
    """Greedy dense decode of `steps` tokens after `tokens`, recording layer
    `layer`'s prefill K/V and each step's q, new k/v and the token_topk of q
    over the full key history. The recorded selection never drives
    generation: attention stays dense. Reference trace.py:219-291."""
    cfg = model.config
    if not tokens or steps < 1 or token_budget < 1 or not 0 <= layer < cfg.num_hidden_layers:
        raise ValueError("invalid capture prompt, steps, token budget or layer")
    trace = {
        "schema_version": 2,
        "page_size": page_size,
        "prefill": {},
        "events": [],
        "source": {
            **(source or {}),
            "kind": "dense_teacher_token_oracle",
            "layer": layer,
            "token_budget_per_query": token_budget,
            "selection": "shared_mean_qk",
            "prompt_tokens": len(tokens),
            "prompt_sha256": sha256(str(tokens).encode()).hexdigest(),
            "torch": str(torch.__version__),
            "capture_device": str(model.device),
            "capture_dtype": str(model.dtype),
        },
    }
    recorded = {}

    class Recorder(HybridKVCache):
        def write(self, request_id, layer_id, k, v):
            super().write(request_id, layer_id, k, v)
            if layer_id == layer:
                recorded["kv"] = {"k": k.detach().cpu().clone(), "v": v.detach().cpu().clone()}
                if not trace["prefill"]:
                    trace["prefill"] = recorded["kv"]

        def attention(self, query, request_id, layer_id, selection, backend="auto"):
            if layer_id == layer:
                keys, _ = self.storage.host_kv(request_id, layer_id)
                q = query.detach().cpu().clone()
                event = {**recorded["kv"], "q": q, "positions": token_topk(q, keys, token_budget)}
                trace["events"].append(event)
            return super().attention(query, request_id, layer_id, selection, backend)

    total = len(tokens) + steps
    pages = ceil(total / page_size)
    hot = HotConfig(total, total, resident_window_pages=pages + 1, transition_watermark=0)
    cache = Recorder(
        CacheConfig(
            gpu_pages=hot.admission_blocks(page_size, cfg.num_hidden_layers),
            host_pages=pages * cfg.num_hidden_layers,
            page_size=page_size,
            kv_heads=cfg.num_key_value_heads,
            head_dim=cfg.head_dim,
            device=str(model.device),
            dtype=model.dtype,
        ),
        hot,
    )
    try:
        cache.reserve("capture", total, cfg.num_hidden_layers)
        logits = model.prefill(tokens, cache, "capture")
        for _ in range(steps):
            logits = model.decode(int(logits.argmax()), "capture", cache, top_k=None)
        validate_trace(trace)
        return trace
    finally:
        if "capture" in cache.storage.requests:
            cache.release_request("capture")
        cache.close()
