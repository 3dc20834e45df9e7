"""The fused selection + resolution launch (nhs_select_resolve_rows / _items)
against the selector launch followed by the resolver launch on the same
scores and tables: chosen pages, positions, physical rows, miss plans,
counts and the tags / LRU post-state must be bit-identical, step after step
as the hot rows evolve. Both are pinned to the oracle elsewhere (the
selector and resolver tests, and the Llama-3-8B-width batched decode test,
which runs this launch); this file pins the fusion itself.
"""

import numpy as np
import pytest
import torch

from nano_hisparse import row_kernels as rk
from test_gpu_kernels import make_resolver_state


def log_case(**kw):
    print("case:", kw, flush=True)


def test_fused_select_fits_the_documented_limits():
    assert rk.fused_select_fits(512, 32, 64)
    assert rk.fused_select_fits(1024, 64, 64)  # 16 pages per lane, 4096 positions
    assert rk.fused_select_fits(1024, 1024, 4)  # one wave: any budget up to its pages
    assert rk.fused_select_fits(1025, 32, 64)  # four waves
    assert rk.fused_select_fits(4096, 256, 16)
    assert not rk.fused_select_fits(4097, 32, 64)
    assert not rk.fused_select_fits(2048, 257, 8)  # four waves choose at most 256
    assert not rk.fused_select_fits(40, 1025, 1)
    assert not rk.fused_select_fits(512, 65, 64)


CASES = [
    # mode, B, Hq, Hkv, D, P, n_pages, top, H, keep_sink, nan_pages, steps
    ("quest", 16, 32, 8, 128, 64, 512, 32, 2048, True, 0, 3),  # Llama-3-8B heads at 32K context
    ("quest", 4, 32, 8, 128, 64, 1024, 64, 4096, True, 0, 2),  # 16 pages per lane, 4096 positions
    ("quest", 3, 8, 2, 64, 16, 700, 100, 1600, False, 5, 3),  # NaN pages, no sink
    ("quest", 2, 8, 2, 64, 16, 200, 8, 300, True, 20, 2),  # more NaN pages than the budget: last page may lose
    ("quest", 2, 4, 2, 64, 16, 40, 100, 1600, True, 0, 2),  # budget above the page count: -1 padding
    ("quest", 3, 4, 2, 32, 7, 300, 1, 64, True, 2, 3),  # one page, odd page size
    ("mean", 4, 8, 2, 64, 32, 400, 20, 700, True, 3, 3),  # page-mean selector
    ("mean", 2, 4, 1, 32, 16, 900, 1, 128, True, 0, 2),
    # more than 256 chosen: wave 0 ranks alone, 8 or 16 pages per lane
    ("quest", 2, 8, 2, 64, 4, 900, 300, 1400, True, 3, 2),
    ("mean", 2, 4, 1, 32, 2, 500, 400, 900, True, 0, 2),
    # beyond 1024 pages: four waves rank, 4 or 16 candidates per lane
    ("quest", 4, 32, 8, 128, 64, 2048, 64, 4096, True, 0, 2),  # Llama-3-8B heads at 128K context
    ("quest", 8, 28, 4, 128, 32, 2048, 32, 2048, True, 3, 2),  # Qwen2-7B heads at 64K context, NaN pages
    ("quest", 3, 8, 2, 64, 4, 1500, 150, 700, False, 0, 3),  # 16 candidates per lane, no sink
    ("mean", 2, 4, 1, 32, 16, 3000, 200, 4096, True, 4, 2),  # 16 pages per lane
    ("quest", 2, 8, 2, 64, 16, 4096, 9, 300, True, 12, 2),  # more NaN pages than the budget
]


def _scores_inputs(g, mode, B, Hq, Hkv, D, n_pages, nan_pages, dtype):
    if mode == "quest":
        a = torch.randn(B, n_pages, Hkv, D, generator=g)
        c = torch.randn(B, n_pages, Hkv, D, generator=g)
        mu = 0.5 * torch.randn(B, n_pages, 1, 1, generator=g)
        lo, hi = torch.minimum(a, c) + mu, torch.maximum(a, c) + mu
        for b in range(B):
            for p in torch.randperm(n_pages - 2, generator=g)[:nan_pages].tolist():
                hi[b, p + 1, 0, 0] = float("nan")
        return lo.to(dtype), hi.to(dtype)
    summ = torch.randn(B, n_pages, Hkv, D, generator=g) + 0.5 * torch.randn(B, n_pages, 1, 1, generator=g)
    for b in range(B):
        for p in torch.randperm(n_pages - 2, generator=g)[:nan_pages].tolist():
            summ[b, p + 1, 0, 0] = float("nan")
    return (summ,)


@pytest.mark.gpu
@pytest.mark.parametrize("mode,B,Hq,Hkv,D,P,n_pages,top,H,keep_sink,nan_pages,steps", CASES)
def test_fused_select_resolve_equals_select_then_resolve(gpu, mode, B, Hq, Hkv, D, P, n_pages, top, H, keep_sink,
                                                         nan_pages, steps):
    log_case(test="select-resolve", mode=mode, B=B, n_pages=n_pages, top=top, P=P, H=H, nan_pages=nan_pages)
    assert rk.fused_select_fits(n_pages, top, P)
    rng = np.random.default_rng(n_pages * 7 + top)
    g = torch.Generator().manual_seed(n_pages + top)
    dtype = torch.bfloat16 if mode == "quest" else torch.float32
    bounds = [t.to(gpu) for t in _scores_inputs(g, mode, B, Hq, Hkv, D, n_pages, nan_pages, dtype)]
    source, resident, hot, tags, lru = make_resolver_state(rng, B, H, P, n_pages, 2 * n_pages,
                                                           n_pages + -(-H // P) + 8, 0.4, 0.6)
    g_src, g_res, g_hot = (torch.from_numpy(x).to(gpu) for x in (source, resident, hot))
    # three copies of the mutable hot state: two-launch path, fused strided, fused per-item
    state = [(torch.from_numpy(tags).to(gpu), torch.from_numpy(lru).to(gpu)) for _ in range(3)]
    lengths = torch.from_numpy(rng.integers(max(1, (n_pages - 3) * P), n_pages * P + 1, size=B)).to(gpu)
    lengths[0] = min(int(lengths[0]), 5 * P + 3)  # a short request: fewer pages than max_pages
    items = rk.layer_items([[dict(source=g_src[b], resident=g_res[b], hot=g_hot[b], tags=state[2][0][b],
                                  lru=state[2][1][b], minimum=g_src[b], maximum=g_src[b], summaries=g_src[b],
                                  n_pages=n_pages) for b in range(B)]], gpu)[0]
    totals = [torch.zeros(3, dtype=torch.int64, device=gpu) for _ in range(3)]
    for step in range(steps):
        q = torch.randn(B, Hq, D, generator=g).to(gpu, dtype if mode == "quest" else torch.bfloat16)
        if mode == "quest":
            pages, positions, _ = rk.quest_batched(q, *bounds, lengths, P, top, keep_sink)
            _, none, scores = rk.quest_batched(q, *bounds, lengths, P, top, keep_sink, select=False)
        else:
            pages, positions, _ = rk.mean_batched(q, *bounds, lengths, P, top)
            _, none, scores = rk.mean_batched(q, *bounds, lengths, P, top, select=False)
        assert none is None
        (tags_a, lru_a), (tags_b, lru_b), (tags_c, lru_c) = state
        want = rk.resolve_batched(positions, g_src, g_res, g_hot, tags_a, lru_a, lengths, P, counts_total=totals[0])
        got = rk.select_resolve_batched(scores, g_src, g_res, g_hot, tags_b, lru_b, lengths, P, top, keep_sink, mode,
                                        counts_total=totals[1])
        got_items = rk.select_resolve_items(scores, items, H, lengths, P, top, keep_sink, mode,
                                            counts_total=totals[2])
        torch.cuda.synchronize()
        for name, x, y in zip(("pages", "positions", "physical", "miss_host", "miss_device", "counts"),
                              (pages, positions) + tuple(want), got):
            assert torch.equal(x, y), (step, name)
        for x, y in zip(got, got_items):
            assert torch.equal(x, y), step
        for t in (tags_b, tags_c):
            assert torch.equal(t, tags_a), step
        for t in (lru_b, lru_c):
            assert torch.equal(t, lru_a), step
    assert torch.equal(totals[0], totals[1]) and torch.equal(totals[0], totals[2])


@pytest.mark.gpu
def test_fused_select_resolve_rejects_shapes_beyond_its_selection(gpu):
    log_case(test="select-resolve-limits")
    B, H, P = 1, 8192, 8
    scores = torch.zeros(B, 4097, dtype=torch.float32, device=gpu)
    tabs = [torch.zeros(B, 4097, dtype=torch.int32, device=gpu) for _ in range(2)]
    hot = torch.zeros(B, H // P, dtype=torch.int32, device=gpu)
    tags = torch.full((B, H), -1, dtype=torch.int32, device=gpu)
    lru = torch.arange(H, device=gpu)[None].clone()
    with pytest.raises(RuntimeError, match="4096"):  # too many pages
        rk.select_resolve_batched(scores, *tabs, hot, tags, lru, 4097 * P, P, 32)
    with pytest.raises(RuntimeError, match="256"):  # four waves choose at most 256
        rk.select_resolve_batched(scores[:, :2048], tabs[0][:, :2048], tabs[1][:, :2048], hot, tags, lru, 2048 * P,
                                  P, 257)
    with pytest.raises(RuntimeError, match="4096"):  # more positions than the LDS holds
        rk.select_resolve_batched(scores[:, :512], tabs[0][:, :512], tabs[1][:, :512], hot, tags, lru, 512 * P, P,
                                  513)
    # beyond the resolver's 32768 positions: NHS_ERR_UNSUPPORTED (the caller
    # may fall back to two launches); a budget below 1 is NHS_ERR_INVALID
    with pytest.raises(RuntimeError, match=r"status -2: .*32768"):
        rk.select_resolve_batched(scores[:, :1024], tabs[0][:, :1024], tabs[1][:, :1024], hot, tags, lru,
                                  1024 * 64, 64, 520)
    with pytest.raises(RuntimeError, match=r"status -1: .*top_pages"):
        rk.select_resolve_batched(scores[:, :512], tabs[0][:, :512], tabs[1][:, :512], hot, tags, lru, 512 * P, P, 0)
    # a budget of more rows than the hot buffer holds: the reference's
    # max_union_rows <= hot_rows (HotConfig) is violated, NHS_ERR_INVALID
    with pytest.raises(RuntimeError, match=r"status -1: .*hot_rows"):
        rk.select_resolve_batched(scores[:, :512], tabs[0][:, :512], tabs[1][:, :512], hot[:, :4], tags[:, :32],
                                  lru[:, :32].clone(), 512 * P, P, 5)


@pytest.mark.gpu
def test_fused_four_wave_selection_replays_in_a_captured_graph(gpu):
    """The four-wave fused launch (2048 pages, as the resolver-stress bench
    replays it) captured once into a HIP graph and replayed step after step,
    with eager work and a synchronization between the replays: every
    replay's outputs and the evolving tags / LRU equal eager launches on a
    copy of the same state."""
    log_case(test="select-resolve-graph")
    B, Hq, Hkv, D, P, n_pages, top, H = 3, 8, 2, 64, 16, 2048, 40, 1024
    assert rk.fused_select_fits(n_pages, top, P) and n_pages > rk.FUSED_WAVE_PAGES
    rng = np.random.default_rng(11)
    g = torch.Generator().manual_seed(11)
    lo, hi = (t.to(gpu) for t in _scores_inputs(g, "quest", B, Hq, Hkv, D, n_pages, 2, torch.bfloat16))
    source, resident, hot, tags, lru = make_resolver_state(rng, B, H, P, n_pages, 2 * n_pages,
                                                           n_pages + -(-H // P) + 8, 0.4, 0.6)
    g_src, g_res, g_hot = (torch.from_numpy(x).to(gpu) for x in (source, resident, hot))
    # three copies of the hot state: warm-up, graph, eager
    (tags_w, lru_w), (tags_g, lru_g), (tags_e, lru_e) = [
        (torch.from_numpy(tags).to(gpu), torch.from_numpy(lru).to(gpu)) for _ in range(3)]
    lengths = torch.from_numpy(rng.integers((n_pages - 3) * P, n_pages * P + 1, size=B)).to(gpu)
    scores = []
    for _ in range(4):
        q = torch.randn(B, Hq, D, generator=g).to(gpu, torch.bfloat16)
        scores.append(rk.quest_batched(q, lo, hi, lengths, P, top, select=False)[2])
    static = scores[0].clone()
    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        rk.select_resolve_batched(static, g_src, g_res, g_hot, tags_w, lru_w, lengths, P, top)
    torch.cuda.current_stream(gpu).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        outs = rk.select_resolve_batched(static, g_src, g_res, g_hot, tags_g, lru_g, lengths, P, top)
    for step in range(4):
        static.copy_(scores[step])
        graph.replay()
        want = rk.select_resolve_batched(scores[step], g_src, g_res, g_hot, tags_e, lru_e, lengths, P, top)
        torch.cuda.synchronize()
        for name, x, y in zip(("pages", "positions", "physical", "miss_host", "miss_device", "counts"), outs, want):
            assert torch.equal(x, y), (step, name)
        assert torch.equal(tags_g, tags_e) and torch.equal(lru_g, lru_e), step
