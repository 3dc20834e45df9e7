"""Trace capture and replay (reference tests/test_trace.py:18-144).

The locality known-answer cases pin the resolver and gather end to end:
hit/miss counts, Jaccard indices, page density, reuse gaps and the hot
slots of the alternating pattern are the reference's own expected values
(tests/golden/reference_kats.json).
On CPU the kernels are the oracle; marked gpu they are libnhs_hip.so.
"""

import copy
import json
import os

import pytest
import torch

from nano_hisparse.model import Model, ModelConfig
from nano_hisparse.trace import (
    capture_trace,
    load_trace,
    replay_trace,
    report_json,
    save_trace,
    synthetic_trace,
    token_topk,
    validate_trace,
)

with open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")) as _f:
    LOCALITY = json.load(_f)["trace_locality"]


@pytest.mark.parametrize("kat", LOCALITY, ids=[f"{k['pattern']}-{k['capacity']}" for k in LOCALITY])
def test_row_locality_counts(device, kat):
    pattern, capacity, hits, misses = kat["pattern"], kat["capacity"], kat["hits"], kat["misses"]
    row_j, page_j, density = kat["row_jaccard"], kat["page_jaccard"], kat["density"]
    report = replay_trace(synthetic_trace(pattern), capacity, device)
    summary = report["summary"]
    assert summary["resident_hits"] == 0
    assert (summary["hot_hits"], summary["misses"]) == (hits, misses)
    assert summary["h2d_bytes"] == misses * 2 * 1 * 8 * 4
    assert summary["mean_row_jaccard"] == pytest.approx(row_j)
    assert summary["mean_page_jaccard"] == pytest.approx(page_j)
    assert summary["mean_page_density"] == density
    assert summary["mean_reuse_gap_steps"] == kat["reuse_gap"]
    for event in report["events"]:
        assert len(event["positions"]) == 4
        assert event["positions"] == tuple(event["union_rows"])
        assert event["hot_hits"] + event["misses"] == 4
        assert set(event["union_rows"]) <= set(event["hot_slots"])
    if pattern == "alternating" and capacity == 8:
        assert set(report["events"][1]["hot_slots"]) == {0, 1, 4, 5, 8, 9, 12, 13}
    assert report["device"].startswith(device.split(":")[0])


def test_token_ranking_selects_rows_without_expanding_pages():
    keys = torch.zeros(16, 1, 2)
    keys[[0, 4, 8, 12], 0, 0] = torch.tensor([4.0, 3, 2, 1])
    keys[[1, 5, 9, 13], 0, 1] = torch.tensor([3.5, 2.5, 1.5, 0.5])
    assert token_topk(torch.eye(2), keys, 4) == [0, 1, 4, 5]


def test_token_ranking_uses_each_query_heads_own_kv_head():
    # 4 query heads over 2 KV heads: heads 0,1 read KV head 0, heads 2,3 KV head 1
    keys = torch.zeros(6, 2, 2)
    keys[0, 0, 0] = 8.0  # only query heads 0/1 see it
    keys[1, 1, 1] = 6.0  # only query heads 2/3 see it
    keys[2, 1, 0] = 100.0  # KV head 1, dimension 0: no query reads it
    q = torch.tensor([[1.0, 0], [1.0, 0], [0, 1.0], [0, 1.0]])
    assert token_topk(q, keys, 2) == [0, 1]
    with pytest.raises(ValueError):
        token_topk(q, keys, 0)


def test_trace_roundtrip_and_invalid_input(cpu_kernels, tmp_path):
    trace = synthetic_trace("alternating")
    path = tmp_path / "trace.pt"
    save_trace(trace, path)
    loaded = load_trace(path)
    assert replay_trace(loaded, 8, "cpu") == replay_trace(trace, 8, "cpu")
    invalid = copy.deepcopy(trace)
    invalid["events"][0]["positions"][0] = 65
    with pytest.raises(ValueError, match="noncausal"):
        validate_trace(invalid)
    invalid = copy.deepcopy(trace)
    invalid["events"][0]["k"] = torch.zeros(2, 1, 8)
    with pytest.raises(ValueError, match="incompatible"):
        validate_trace(invalid)
    with pytest.raises(ValueError):
        replay_trace(trace, 3, "cpu")
    invalid = copy.deepcopy(trace)
    invalid["events"][0]["positions"] = [[0, 4], [8, 12]]
    with pytest.raises(ValueError, match="one shared"):
        validate_trace(invalid)
    with pytest.raises(ValueError, match="unknown"):
        synthetic_trace("random")
    with pytest.raises(ValueError, match="2..8"):
        synthetic_trace("reuse", steps=9)


def test_synthetic_trace_is_seeded_and_portable():
    a, b = synthetic_trace("streaming", steps=3, seed=7), synthetic_trace("streaming", steps=3, seed=7)
    assert all(torch.equal(x["q"], y["q"]) for x, y in zip(a["events"], b["events"]))
    assert torch.equal(a["prefill"]["k"], b["prefill"]["k"])
    # draw order: prefill K, prefill V, then q, k, v of each event
    gen = torch.Generator().manual_seed(7)
    assert torch.equal(torch.randn(64, 1, 8, generator=gen), a["prefill"]["k"])
    torch.randn(64, 1, 8, generator=gen)
    assert torch.equal(torch.randn(2, 8, generator=gen), a["events"][0]["q"])
    assert [e["positions"] for e in a["events"]] == [[0, 16, 32, 48], [1, 17, 33, 49], [2, 18, 34, 50]]


def test_legacy_per_head_trace_preserves_masks_and_capacity(device):
    trace = synthetic_trace("reuse")
    trace["schema_version"] = 1
    for event in trace["events"]:
        event["positions"] = [[0, 4, 8], [4, 12]]
    report = replay_trace(trace, device=device)
    assert report["schema_version"] == 1
    assert report["max_union_rows"] == 4
    assert report["events"][0]["positions"] == ((0, 4, 8), (4, 12))
    assert report["summary"]["misses"] == 4
    assert '"schema_version": 1' in report_json(report)


def test_capture_records_real_queries_and_preserves_dense_trajectory(device, tmp_path):
    torch.manual_seed(3)
    model = Model(
        ModelConfig(
            hidden_size=32,
            intermediate_size=64,
            num_hidden_layers=2,
            num_attention_heads=4,
            num_key_value_heads=2,
            vocab_size=64,
        )
    ).eval().to(device)
    tokens = list(range(1, 34))
    trace = capture_trace(model, tokens, steps=3, token_budget=2, layer=1, page_size=4)
    # a dense forward over the growing history, recording layer 1's q/k/v:
    # a sparse teacher would change the later queries
    observed = []
    project = model._project

    def record(layer, x, start):
        q, k, v = project(layer, x, start)
        if layer is model.model.layers[1]:
            observed.append((q[-1].cpu(), k.cpu(), v.cpu()))
        return q, k, v

    model._project = record
    history = list(tokens)
    logits = model.prefill(history)
    observed.clear()
    for _ in range(3):
        history.append(int(logits.argmax()))
        logits = model.prefill(history)
    tol = dict(atol=2e-6, rtol=2e-5) if device == "cpu" else dict(atol=2e-4, rtol=2e-3)
    for event, (q, k, v) in zip(trace["events"], observed, strict=True):
        torch.testing.assert_close(event["q"], q, **tol)
        torch.testing.assert_close(event["k"], k[-1:], **tol)
        torch.testing.assert_close(event["v"], v[-1:], **tol)
        assert event["positions"] == token_topk(q, k, 2)
    save_trace(trace, tmp_path / "model.pt")
    report = replay_trace(load_trace(tmp_path / "model.pt"), device=device)
    assert report["summary"]["misses"] > 0
    assert report["max_union_rows"] == 2
    assert report["source"]["token_budget_per_query"] == 2
    assert trace["schema_version"] == 2
    assert report["source"]["kind"] == "dense_teacher_token_oracle"
