"""Selection, LogicalTopK, quest_selection and resolve_rows through the
package API, on CPU tensors (oracle provider) and on cuda:0 (libnhs_hip.so).

Known answers from the reference's tests/test_selection.py:8-50.
"""

import pytest
import torch

from nano_hisparse.row_index import LogicalTopK, resolve_rows
from nano_hisparse.selection import Selection, quest_selection


def test_per_head_masks_and_invalid_positions():
    sel = Selection.from_tokens([[3, 1, 1, -1], [0]], 4, 2, 2)
    topk = LogicalTopK.from_selection(sel, "cpu")
    assert topk.positions.tolist() == [0, 1, 3]
    assert topk.head_columns.tolist() == [[1, 2], [0, -1]]
    for bad in ([4], [-2], [-1], [1.2], []):
        with pytest.raises((ValueError, TypeError)):
            Selection.from_tokens(bad, 4, 2, 2)


def test_from_pages_expands_causal_tokens():
    sel = Selection.from_pages([2, 0], 11, 4, 3)
    assert sel.positions == ((0, 1, 2, 3, 8, 9, 10),) * 3
    assert sel.pages == [0, 2]
    with pytest.raises(ValueError, match="logical page"):
        Selection.from_pages([3], 11, 4, 1)


def test_quest_keeps_a_page_whose_mean_cancels(device):
    low = torch.tensor([[[-10.0, 0.0]], [[1.0, 0.0]], [[0.0, 0.0]]], device=device)
    high = torch.tensor([[[10.0, 0.0]], [[1.0, 0.0]], [[0.0, 0.0]]], device=device)
    sel = quest_selection(torch.tensor([[1.0, 0.0]], device=device), low, high, 5, 2, 2, keep_sink=False)
    assert sel.pages == [0, 2]


def test_quest_budget_is_shared_across_heads(device):
    # head 0 prefers page 0 (9), head 1 page 1 (10): the head mean picks page 1
    # (5 > 4.5); per-head top-k followed by a union would pick both
    bounds = torch.tensor([[[9.0, 0.0]], [[0.0, 10.0]], [[-1.0, -1.0]]], device=device)
    sel = quest_selection(torch.eye(2, device=device), bounds, bounds, 5, 2, 2, keep_sink=False)
    assert sel.positions == ((2, 3, 4),) * 2
    topk = LogicalTopK.from_selection(sel, device)
    assert topk.positions.tolist() == [2, 3, 4]
    assert topk.head_columns is None


def test_quest_with_sink_keeps_first_and_last(device):
    torch.manual_seed(3)
    q = torch.randn(4, 8, device=device)
    keys = torch.randn(40, 2, 8, device=device)
    lo = keys.view(10, 4, 2, 8).amin(1)
    hi = keys.view(10, 4, 2, 8).amax(1)
    sel = quest_selection(q, lo, hi, 40, 4, 3, keep_sink=True)
    assert 0 in sel.pages and 9 in sel.pages and len(sel.pages) == 3
    everything = quest_selection(q, lo, hi, 40, 4, 10)
    assert everything.pages == list(range(10))


def test_resolver_known_answer(device):
    def t(values):
        return torch.tensor(values, dtype=torch.int64, device=device)

    source, resident, hot = t([5, 2, 9, 4]), t([-1, 7, -1, 3]), t([6, 1])
    tags = t([-1, -1, -1, -1, -1, 22, -1, -1])
    lru = t([0, 1, 2, 3, 4, 6, 7, 5])
    plan = resolve_rows(LogicalTopK(t([9, 2, 6, 9, 14, -1])), source, resident, hot, tags, lru, 16, 4)
    assert plan.physical_rows.tolist() == [24, 5, 30, -1, 14, -1]
    assert plan.counts.tolist() == [2, 1, 1]
    assert plan.miss_host_rows.tolist() == [37, -1, -1, -1, -1, -1]
    assert plan.miss_device_rows.tolist() == [24, -1, -1, -1, -1, -1]
    assert tags[0].item() == 37 and tags[5].item() == 22
    assert lru.tolist() == [1, 2, 3, 4, 6, 7, 0, 5]


def test_resolver_expands_per_head_columns(device):
    sel = Selection.from_tokens([[0, 5], [5, 6], [6]], 8, 4, 3)
    topk = LogicalTopK.from_selection(sel, device)
    i32 = dict(dtype=torch.int32, device=device)
    source = torch.tensor([0, 1], **i32)
    resident = torch.tensor([2, 3], **i32)
    hot = torch.tensor([0], **i32)
    tags = torch.full((4,), -1, **i32)
    lru = torch.arange(4, dtype=torch.int64, device=device)
    plan = resolve_rows(topk, source, resident, hot, tags, lru, 8, 4)
    assert plan.physical_rows.tolist() == [[8, 13], [13, 14], [14, -1]]
