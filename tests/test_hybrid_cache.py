"""HybridKVCache end to end: resident hits, hot-row hits and misses, leases,
admission and row attention, on CPU (oracle provider) and cuda:0.

Scenarios and expected counters follow the reference's
tests/test_hybrid.py:13-296.
"""

from dataclasses import replace

import pytest
import torch

from nano_hisparse.attention import row_attention
from nano_hisparse.config import CacheConfig, CapacityError
from nano_hisparse.hybrid import HotConfig, HybridKVCache
from nano_hisparse.row_index import LogicalTopK, resolve_rows
from nano_hisparse.selection import Selection, dense_attention, selection_oracle


def make(device, **changes):
    cfg = CacheConfig(gpu_pages=3, host_pages=64, page_size=4, kv_heads=1, head_dim=8, device=device)
    return HybridKVCache(replace(cfg, **changes), HotConfig(4, 4))


def append(cache, name="a", count=32, layer=0):
    shape = (count, cache.config.kv_heads, cache.config.head_dim)
    k = torch.randn(shape, device=cache.device, dtype=cache.config.dtype)
    v = torch.randn(shape, device=cache.device, dtype=cache.config.dtype)
    cache.write(name, layer, k, v)
    return k, v


def positions(cache, values):
    return LogicalTopK(torch.tensor(values, dtype=torch.int32, device=cache.device))


def test_misses_gather_rows_and_resident_pages_skip_the_hot_rows(device):
    cache = make(device)
    cache.reserve("a", 40, 1)
    k, v = append(cache)
    q = torch.randn(2, 8, device=device)
    chosen = [0, 7, 17, 31]
    for _ in range(2):  # second pass: the three earlier misses are hot hits
        out = row_attention(q, cache, "a", 0, positions(cache, chosen))
        torch.testing.assert_close(out, dense_attention(q, k[chosen], v[chosen]), atol=2e-6, rtol=2e-5)
    assert cache.snapshot()["row_stats"] == {"resident_hits": 2, "hot_hits": 3, "misses": 3, "h2d_bytes": 192}
    assert cache.pool.data_ptr() == cache.allocator.storage.data_ptr()
    cache.assert_invariants()


def test_fully_resident_history_takes_no_hot_blocks(device):
    cache = make(device, gpu_pages=8)
    cache.reserve("a", 32, 1)
    k, v = append(cache, count=20)
    q = torch.randn(2, 8, device=device)
    chosen = [1, 7, 17, 19]
    out = row_attention(q, cache, "a", 0, positions(cache, chosen))
    torch.testing.assert_close(out, dense_attention(q, k[chosen], v[chosen]))
    assert not cache.tables["a", 0].blocks
    assert cache.snapshot()["row_stats"]["misses"] == 0


def test_selected_hot_rows_are_protected_and_lru_evicts_the_rest(device):
    cache = make(device)
    cache.reserve("a", 40, 1)
    k, v = append(cache)
    q = torch.randn(2, 8, device=device)
    for chosen in ([0, 4, 8, 12], [16, 4, 8, 12], [4, 4, -1, 12]):
        out = row_attention(q, cache, "a", 0, positions(cache, chosen))
        distinct = sorted({t for t in chosen if t >= 0})  # duplicates count once
        torch.testing.assert_close(out, dense_attention(q, k[distinct], v[distinct]), atol=2e-6, rtol=2e-5)
    assert cache.snapshot()["row_stats"]["misses"] == 5
    first_host_row = cache.storage.pages["a", 0, 0].host_slot * 4
    assert first_host_row not in cache.tables["a", 0].tags.tolist()
    cache.assert_invariants()


@pytest.mark.parametrize("shared", [True, False])
def test_shared_and_per_head_masks_over_fragmented_hot_blocks(device, shared):
    cfg = CacheConfig(gpu_pages=8, host_pages=64, page_size=3, kv_heads=2, head_dim=8, device=device)
    cache = HybridKVCache(cfg, HotConfig(6, 6, transition_watermark=0))
    cache.reserve("a", 40, 1)
    cache.reserve("b", 40, 1)
    for _ in range(3):  # interleaved so the reclaimed blocks of "a" are fragmented
        append(cache, "a", 3)
        append(cache, "b", 3)
    append(cache, "b", 3)
    cache.storage.synchronize()
    cache.transition_to_host("a", 0)
    assert cache.tables["a", 0].blocks == [7, 0]
    append(cache, "a", 18)
    k, v = (t.to(device) for t in cache.storage.host_kv("a", 0))
    q = torch.randn(4, 8, device=device)
    tokens = [0, 2, 7, 11, 19] if shared else [[0, 7], [2], [7, 11], [19, 0]]
    sel = Selection.from_tokens(tokens, 27, 3, 4)
    out = cache.attention(q, "a", 0, selection=sel)
    expected, _ = selection_oracle(q, k, v, sel)
    torch.testing.assert_close(out, expected, atol=2e-6, rtol=2e-5)
    cache.assert_invariants()


def test_admission_and_topk_overflow_change_nothing(device):
    cache = make(device, gpu_pages=3)
    cache.reserve("a", 40, 1)
    index_before = cache.index_bytes
    with pytest.raises(CapacityError, match="credits"):
        cache.reserve("b", 40, 1)
    assert "b" not in cache.storage.requests and cache.index_bytes == index_before
    append(cache)
    tags_before = cache.tables["a", 0].tags.clone()
    with pytest.raises(ValueError, match="max_union_rows"):
        cache.resolve("a", 0, positions(cache, [0, 1, 2, 3, 4]))
    torch.testing.assert_close(tags_before, cache.tables["a", 0].tags)
    with pytest.raises(ValueError):
        HotConfig(8, 4)
    cache.assert_invariants()


def test_index_tables_count_against_the_index_budget(device):
    need = make(device).index_reservation_bytes(40, 1)
    small = make(device, index_budget_bytes=need - 1)
    with pytest.raises(CapacityError, match="index budget"):
        small.reserve("a", 40, 1)
    assert not small.storage.requests and not small.tables
    exact = make(device, index_budget_bytes=need)
    exact.reserve("a", 40, 1)
    assert exact.index_bytes == need
    exact.release_request("a")
    assert exact.index_bytes == 0


def test_row_lease_blocks_appends_and_release_until_returned(device):
    cache = make(device, gpu_pages=3)
    cache.reserve("a", 40, 1)
    append(cache)
    lease = cache.resolve("a", 0, positions(cache, [0, 4, 8, 31]))
    lease.wait()
    with pytest.raises(RuntimeError, match="already leased"):
        cache.resolve("a", 0, positions(cache, [1]))
    with pytest.raises(RuntimeError, match="active row"):
        cache.release_request("a")
    with pytest.raises(RuntimeError, match="append"):
        append(cache, count=1)
    lease.release()
    append(cache, count=1)  # token 32 opens page 8; pages 7 and 8 are the tails
    pages = cache.storage.pages
    assert pages["a", 0, 8].slot is not None and pages["a", 0, 7].slot is not None
    assert pages["a", 0, 6].slot is None
    cache.assert_invariants()
    cache.release_request("a")
    with pytest.raises(RuntimeError, match="released"):
        lease.wait()


def test_random_requests_layers_appends_and_replacement(device):
    torch.manual_seed(17)
    cache = make(device, gpu_pages=12, host_pages=256)
    history = {}
    for name in ("a", "b"):
        cache.reserve(name, 64, 2)
        for layer in range(2):
            history[name, layer] = append(cache, name, 19, layer)
    for step in range(32):
        name, layer = ("a", "b")[step % 2], (step // 2) % 2
        k, v = history[name, layer]
        nk, nv = append(cache, name, 1, layer)
        k, v = torch.cat((k, nk)), torch.cat((v, nv))
        history[name, layer] = (k, v)
        chosen = [*torch.randperm(len(k) - 1)[:3].tolist(), len(k) - 1]
        q = torch.randn(2, 8, device=device)
        out = row_attention(q, cache, name, layer, positions(cache, chosen))
        torch.testing.assert_close(out, dense_attention(q, k[chosen], v[chosen]), atol=3e-6, rtol=3e-5)
        cache.assert_invariants()
    for name in ("a", "b"):
        cache.release_request(name)
    cache.assert_invariants()


def test_padding_and_out_of_range_positions_read_nothing(device):
    cache = make(device)
    cache.reserve("a", 40, 1)
    append(cache)
    q = torch.randn(2, 8, device=device)
    out = row_attention(q, cache, "a", 0, positions(cache, [-1, -2, 100, 32]))
    torch.testing.assert_close(out, torch.zeros_like(out))
    assert cache.snapshot()["row_stats"]["misses"] == 0


def test_failed_resolve_returns_every_reference(device, monkeypatch):
    cache = make(device)
    cache.reserve("a", 40, 1)
    append(cache)
    refs = [s.ref_cnt for s in cache.allocator.slots]

    def broken(*args):
        raise RuntimeError("resolver failed on purpose")

    with monkeypatch.context() as patch:
        patch.setattr("nano_hisparse.hybrid.resolve_rows", broken)
        with pytest.raises(RuntimeError, match="on purpose"):
            cache.resolve("a", 0, positions(cache, [0, 4, 8, 31]))
    assert [s.ref_cnt for s in cache.allocator.slots] == refs
    assert not cache.tables["a", 0].busy and not cache.storage.pinned
    with cache.resolve("a", 0, positions(cache, [0, 4, 8, 31])):
        cache.assert_invariants()
    cache.release_request("a")
    assert all(s.ref_cnt == 0 for s in cache.allocator.slots)
    cache.assert_invariants()


# ---- GPU only -------------------------------------------------------------------------------


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_low_precision_rows_gather_and_attend(gpu, dtype):
    torch.manual_seed(5)
    cache = make("cuda:0", dtype=dtype, page_size=7, head_dim=24, kv_heads=2)
    cache.reserve("a", 100, 1)
    k, v = append(cache, count=80)
    q = torch.randn(6, 24, device="cuda", dtype=dtype)
    chosen = [0, 13, 39, 79]
    out = row_attention(q, cache, "a", 0, positions(cache, chosen))
    torch.testing.assert_close(out, dense_attention(q, k[chosen], v[chosen]), atol=0.004, rtol=0.02)


@pytest.mark.gpu
def test_every_reference_backend_name_runs_the_hip_kernel_on_a_gpu_cache(gpu):
    """The reference accepts backend auto|torch|triton on CUDA tensors
    (attention.py:8-35, cli.py:48, engine.py:30); on a GPU cache each name,
    and "hip", runs the one HIP kernel, so the outputs are bit-identical and
    match the dense reference; an unknown name still raises."""
    torch.manual_seed(11)
    cache = make("cuda:0", dtype=torch.bfloat16, page_size=8, head_dim=64, kv_heads=2)
    cache.reserve("a", 120, 1)
    k, v = append(cache, count=100)
    q = torch.randn(8, 64, device="cuda", dtype=torch.bfloat16)
    chosen = [0, 9, 63, 99]  # HotConfig(4, 4): at most 4 rows
    outs = {}
    for backend in ("auto", "torch", "triton", "hip"):
        outs[backend] = row_attention(q, cache, "a", 0, positions(cache, chosen), backend=backend)
    for backend, out in outs.items():
        assert torch.equal(out, outs["auto"]), backend
    torch.testing.assert_close(outs["torch"], dense_attention(q, k[chosen], v[chosen]), atol=0.004, rtol=0.02)
    with pytest.raises(ValueError, match="invalid attention backend"):
        row_attention(q, cache, "a", 0, positions(cache, chosen), backend="cuda")
    cache.assert_invariants()


@pytest.mark.gpu
def test_resolver_replays_in_a_captured_graph_without_host_reads(gpu):
    cache = make("cuda:0")
    cache.reserve("a", 40, 1)
    append(cache)
    tables = cache.tables["a", 0]
    logical = positions(cache, [0, 4, 8, 31])

    def run():
        return resolve_rows(logical, tables.source, tables.resident, tables.hot, tables.tags, tables.lru, 32, 4)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            run()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan = run()
    logical.positions.copy_(torch.tensor([1, 5, 9, 31], device="cuda", dtype=torch.int32))
    graph.replay()
    assert plan.counts.tolist() == [1, 0, 3]
    eager = run()  # a replay leaves the tables as an eager call would
    torch.cuda.synchronize()
    assert eager.counts.tolist() == [1, 3, 0]


@pytest.mark.gpu
def test_deferred_reuse_keeps_host_rows_and_hot_readers_alive(gpu):
    cache = make("cuda:0", gpu_pages=3)
    cache.reserve("same", 40, 1)
    k, _ = append(cache, "same")
    with cache.resolve("same", 0, positions(cache, [0, 4, 8, 31])) as lease:
        torch.cuda._sleep(2_000_000)
        row = lease.plan.physical_rows[0]
        seen = cache.pool[row // 4, 0, row % 4].clone()
    old_hosts = {p.host_slot for p in cache.storage.pages.values()}
    cache.release_request("same", wait=False)
    cache.reserve("same", 40, 1)
    append(cache, "same")
    if cache.storage.retired:
        assert old_hosts.isdisjoint({p.host_slot for p in cache.storage.pages.values()})
    torch.testing.assert_close(seen, k[0])
    cache.release_request("same")
    cache.assert_invariants()


def test_a_selection_of_8192_rows_resolves_and_attends(device):
    """Quest top-128 pages of 64 rows (8192 positions, max_union_rows 8192,
    hot_rows 16384, both within the reference's HotConfig limits,
    hybrid.py:31-41) decodes through HybridKVCache.attention: rows beyond the
    in-LDS resolver's 4096 go through the large-selection resolver."""
    from nano_hisparse.selection import quest_selection

    P, pages = 64, 300
    cfg = CacheConfig(gpu_pages=270, host_pages=pages + 8, page_size=P, kv_heads=2, head_dim=64, device=device)
    cache = HybridKVCache(cfg, HotConfig(128 * P))
    cache.reserve("a", pages * P, 1)
    k, v = append(cache, count=pages * P - 17)
    request = cache.storage.requests["a"]
    length = request.lengths[0]
    for step in range(2):  # the second step hits the rows the first one gathered
        q = torch.randn(4, 64, device=device)
        sel = quest_selection(q, request.minimum[0], request.maximum[0], length, P, 128)
        assert len(sel.pages) == 128 and pages - 1 in sel.pages
        chosen = list(sel.positions[0])
        assert len(chosen) == 128 * P - 17
        out = cache.attention(q, "a", 0, sel)
        torch.testing.assert_close(out, dense_attention(q, k[chosen], v[chosen]), atol=1e-4, rtol=1e-4)
    stats = cache.snapshot()["row_stats"]
    assert stats["resident_hits"] + stats["hot_hits"] + stats["misses"] == 2 * len(chosen)
    cache.assert_invariants()
