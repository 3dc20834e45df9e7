"""Batched decode (one launch per stage and layer for all running requests).

- The per-item entry points (nhs_append_items, nhs_quest_select_items,
  nhs_resolve_items) against their strided twins on the same tables: bounds,
  summaries, pool and host bytes, selections, rows, plans, tags and LRU
  bit-exact.
- BatchDecode against the per-request cache path (write + Quest selection +
  attention) on the same queries and K/V over many steps: identical
  selections and host histories, attention within tolerance, invariants.
- Engine(batch_decode=True) against the sequential engine: same tokens.
"""

import pytest
import torch

from nano_hisparse import row_kernels as rk
from nano_hisparse.config import CacheConfig
from nano_hisparse.engine import Engine
from nano_hisparse.hybrid import HotConfig, HybridKVCache
from nano_hisparse.model import Model, ModelConfig
from nano_hisparse.selection import quest_selection


def log_case(**kw):
    print("case:", kw, flush=True)


def make_cache(device, dtype=torch.float32, gpu_pages=48, P=8, Hkv=2, D=16, union=32, hot_rows=48):
    cfg = CacheConfig(gpu_pages=gpu_pages, host_pages=512, page_size=P, kv_heads=Hkv, head_dim=D, dtype=dtype,
                      device=device)
    return HybridKVCache(cfg, HotConfig(union, hot_rows, resident_window_pages=6))


def test_batched_decode_needs_a_gpu_cache(cpu_kernels):
    cache = make_cache("cpu")
    cache.reserve("a", 64, 1)
    cache.write("a", 0, torch.randn(9, 2, 16), torch.randn(9, 2, 16))
    with pytest.raises(RuntimeError, match="GPU cache"):
        cache.decode_batch(["a"])


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_item_entry_points_match_the_strided_ones(gpu, dtype):
    log_case(test="item-kernels", dtype=str(dtype))
    g = torch.Generator(device=gpu).manual_seed(5)
    B, Hq, Hkv, D, P, H = 3, 8, 2, 64, 16, 64
    n_pages = [9, 14, 6]
    blocks = 64
    pool = torch.randn(blocks, 2, P, Hkv, D, generator=g, device=gpu).to(dtype)
    host = torch.zeros(64, 2, P, Hkv, D, dtype=dtype, pin_memory=True)
    alias = rk.MappedHost(host)
    lengths = [n * P - 3 for n in n_pages]  # the appended token lands mid-page
    tabs = []
    for b, n in enumerate(n_pages):
        source = torch.arange(n, dtype=torch.int32, device=gpu) + 20 * b
        resident = torch.randperm(blocks, generator=g, device=gpu)[:n].to(torch.int32)
        hot = torch.randperm(blocks, generator=g, device=gpu)[: H // P].to(torch.int32)
        tags = torch.full((H,), -1, dtype=torch.int32, device=gpu)
        lru = torch.randperm(H, generator=g, device=gpu)
        mn = torch.randn(n, Hkv, D, generator=g, device=gpu).to(dtype)
        mx = mn + torch.rand(n, Hkv, D, generator=g, device=gpu).to(dtype)
        summ = torch.randn(n, Hkv, D, generator=g, device=gpu)
        tabs.append(dict(source=source, resident=resident, hot=hot, tags=tags, lru=lru, minimum=mn, maximum=mx,
                         summaries=summ, n_pages=n))
    # resident blocks must be distinct across items for the append comparison
    used = torch.randperm(blocks, generator=g, device=gpu)[: sum(n_pages)].to(torch.int32)
    off = 0
    for t, n in zip(tabs, n_pages):
        t["resident"] = used[off: off + n].clone()
        off += n
    ref = [{k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in t.items()} for t in tabs]
    items = rk.layer_items([tabs], gpu)[0]
    dev_len = torch.tensor(lengths, dtype=torch.int64, device=gpu)
    k = torch.randn(B, Hkv, D, generator=g, device=gpu).to(dtype)
    v = torch.randn(B, Hkv, D, generator=g, device=gpu).to(dtype)
    ref_pool, ref_host = pool.clone(), host.clone().pin_memory()
    ref_alias = rk.MappedHost(ref_host)
    rk.append_items(k, v, pool, alias, items, dev_len)
    for b, t in enumerate(ref):
        page, within = divmod(lengths[b], P)
        rk.append_page(k[b: b + 1], v[b: b + 1], ref_pool, int(t["resident"][page]), within, ref_alias,
                       int(t["source"][page]), t["summaries"][page], t["minimum"][page], t["maximum"][page])
    torch.cuda.synchronize()
    assert torch.equal(pool.view(torch.uint8), ref_pool.view(torch.uint8))
    assert torch.equal(host.view(torch.uint8), ref_host.view(torch.uint8))
    for t, r in zip(tabs, ref):
        for name in ("minimum", "maximum", "summaries"):
            assert torch.equal(t[name].view(torch.uint8), r[name].view(torch.uint8)), name
    # Quest over per-item bounds vs the strided kernel, request by request
    after = dev_len + 1
    q = torch.randn(B, Hq, D, generator=g, device=gpu).to(dtype)
    top = 4
    pages, positions, _ = rk.quest_items(q, items, dtype, Hkv, after, P, max(n_pages), top)
    for b, t in enumerate(tabs):
        e_pages, e_pos, _ = rk.quest_batched(q[b: b + 1], t["minimum"][None], t["maximum"][None],
                                             int(after[b]), P, top)
        assert torch.equal(pages[b], e_pages[0]) and torch.equal(positions[b], e_pos[0])
    # resolver over per-item tables vs the strided kernel, twice (tags and LRU
    # evolve); every other page is host-only so both steps have misses
    for t in tabs:
        t["resident"][0:-1:2] = -1
    for _ in range(2):
        before = [(t["tags"].clone(), t["lru"].clone()) for t in tabs]
        phys, mh, md, cnt = rk.resolve_items(positions, items, H, after, P)
        for b, t in enumerate(tabs):
            tags, lru = before[b]
            e = rk.resolve_batched(positions[b: b + 1], t["source"][None], t["resident"][None], t["hot"][None],
                                   tags[None], lru[None], int(after[b]), P)
            for got, want in zip((phys[b], mh[b], md[b], cnt[b]), (x[0] for x in e)):
                assert torch.equal(got, want)
            assert torch.equal(t["tags"], tags) and torch.equal(t["lru"], lru)


@pytest.mark.gpu
@pytest.mark.parametrize("K", [96, 4608])  # resolve_rows_kernel, and resolve_large_kernel beyond 4096 positions
def test_resolve_items_with_an_item_of_no_pages(gpu, K):
    """An item with no pages (n_pages 0, length 0) beside normal items in one
    nhs_resolve_items launch: its table pointers are never read, every entry
    of its plan is unset (-1), its counts are zero and its tags and LRU order
    are unchanged; the other items resolve as the strided kernel does."""
    log_case(test="resolve-empty-item", K=K)
    g = torch.Generator(device=gpu).manual_seed(11)
    P, H = 16, max(512, 2 * K)  # hot rows cover the selection (max_union_rows <= hot_rows)
    n_pages = [K // P + 4, 0, K // P + 9]
    blocks = 4 * max(n_pages) + 64
    tabs = []
    for b, n in enumerate(n_pages):
        m = max(n, 1)  # a one-element table for the empty item: a valid pointer it must not read
        source = torch.arange(m, dtype=torch.int32, device=gpu) + 1000 * b
        resident = torch.randperm(blocks, generator=g, device=gpu)[:m].to(torch.int32)
        resident[::2] = -1
        hot = torch.randperm(blocks, generator=g, device=gpu)[: H // P].to(torch.int32)
        tags = torch.full((H,), -1, dtype=torch.int32, device=gpu)
        lru = torch.randperm(H, generator=g, device=gpu)
        tabs.append(dict(source=source, resident=resident, hot=hot, tags=tags, lru=lru, minimum=source,
                         maximum=source, summaries=source, n_pages=n))
    items = rk.layer_items([tabs], gpu)[0]
    lengths = torch.tensor([n * P for n in n_pages], dtype=torch.int64, device=gpu)
    positions = torch.stack([torch.randperm(max(n, 1) * P, generator=g, device=gpu)[:K] if n else
                             torch.randint(0, 1 << 20, (K,), generator=g, device=gpu) for n in n_pages]).to(torch.int32)
    positions = positions.sort(1).values.contiguous()
    before = [(t["tags"].clone(), t["lru"].clone()) for t in tabs]
    with pytest.raises(RuntimeError, match="hot_rows"):  # more positions than hot rows: rejected, nothing runs
        rk.resolve_items(positions, items, K - 1, lengths, P)
    phys, mh, md, cnt = rk.resolve_items(positions, items, H, lengths, P)
    torch.cuda.synchronize()
    assert (phys[1] == -1).all() and (mh[1] == -1).all() and (md[1] == -1).all()
    assert not cnt[1].any()
    assert torch.equal(tabs[1]["tags"], before[1][0]) and torch.equal(tabs[1]["lru"], before[1][1])
    for b in (0, 2):
        t = tabs[b]
        tags, lru = before[b]
        e = rk.resolve_batched(positions[b: b + 1], t["source"][None], t["resident"][None], t["hot"][None],
                               tags[None], lru[None], int(lengths[b]), P)
        for got, want in zip((phys[b], mh[b], md[b], cnt[b]), (x[0] for x in e)):
            assert torch.equal(got, want)
        assert torch.equal(t["tags"], tags) and torch.equal(t["lru"], lru)
        assert int(cnt[b, 2]) > 0


def _prefill(caches, names, lengths, layers, g, device, dtype):
    cfg = caches[0].config
    for name, n in zip(names, lengths):
        for c in caches:
            c.reserve(name, n + 64, layers)
        for layer in range(layers):
            k = torch.randn(n, cfg.kv_heads, cfg.head_dim, generator=g, device=device).to(dtype)
            v = torch.randn(n, cfg.kv_heads, cfg.head_dim, generator=g, device=device).to(dtype)
            for c in caches:
                c.write(name, layer, k, v)


@pytest.mark.gpu
@pytest.mark.parametrize("overlap", [False, True])
@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_batch_decode_matches_the_per_request_cache_path(gpu, dtype, tol, overlap):
    log_case(test="batch-decode-vs-sequential", dtype=str(dtype), overlap=overlap)
    g = torch.Generator(device=gpu).manual_seed(11)
    seq, bat = make_cache(gpu, dtype), make_cache(gpu, dtype)
    names, lengths, layers, top = ["a", "b", "c"], [37, 70, 9], 2, 4
    Hq = 4
    _prefill((seq, bat), names, lengths, layers, g, gpu, dtype)
    P = seq.config.page_size
    for step in range(40):  # crosses page boundaries, transitions and hot-row reuse
        step_b = bat.decode_batch(names, overlap)
        for layer in range(layers):
            k = torch.randn(3, 2, 16, generator=g, device=gpu).to(dtype)
            v = torch.randn(3, 2, 16, generator=g, device=gpu).to(dtype)
            q = torch.randn(3, Hq, 16, generator=g, device=gpu).to(dtype)
            step_b.append(layer, k, v)
            out_b = step_b.attend(layer, q, top)
            for i, name in enumerate(names):
                seq.write(name, layer, k[i: i + 1], v[i: i + 1])
                request = seq.storage.requests[name]
                sel = quest_selection(q[i], request.minimum[layer], request.maximum[layer],
                                      request.lengths[layer], P, top)
                out_s = seq.attention(q[i], name, layer, sel)
                err = (out_b[i].float() - out_s.float()).abs().max().item()
                assert err <= tol, (step, layer, name, err)
        step_b.end()
        for c in (seq, bat):
            c.assert_invariants()
    for name in names:
        for layer in range(layers):
            ks, vs = seq.storage.host_kv(name, layer)
            kb, vb = bat.storage.host_kv(name, layer)
            assert torch.equal(ks.view(torch.uint8), kb.view(torch.uint8))
            assert torch.equal(vs.view(torch.uint8), vb.view(torch.uint8))
            rs, rb = seq.storage.requests[name], bat.storage.requests[name]
            for field in ("minimum", "maximum", "summaries"):
                a, b = getattr(rs, field)[layer], getattr(rb, field)[layer]
                assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), field
    assert bat.snapshot()["row_stats"]["misses"] > 0
    for c in (seq, bat):
        for name in names:
            c.release_request(name)
        c.assert_invariants()
        assert not any(c.owners)


@pytest.mark.gpu
@pytest.mark.parametrize("micro_batches", [1, 2])
def test_engine_batch_decode_generates_the_sequential_tokens(gpu, micro_batches):
    log_case(test="engine-batch-decode", micro_batches=micro_batches)
    torch.manual_seed(31)
    cfg = ModelConfig(hidden_size=64, intermediate_size=128, num_hidden_layers=2, num_attention_heads=4,
                      num_key_value_heads=2, vocab_size=96)
    model = Model(cfg).eval().to(gpu)
    prompts = {"a": list(range(1, 40)), "b": list(range(5, 70)), "c": list(range(2, 19))}
    results = []
    for batch_decode in (False, True):
        cache = HybridKVCache(
            CacheConfig(gpu_pages=40, host_pages=256, page_size=4, kv_heads=2, head_dim=16, device=gpu),
            HotConfig(16, 24, resident_window_pages=4),
        )
        engine = Engine(model, cache, top_k=4, batch_decode=batch_decode, micro_batches=micro_batches)
        for name, prompt in prompts.items():
            engine.add_request(name, prompt, 12)
        results.append(engine.run())
        assert not cache.storage.requests and not any(cache.owners)
        cache.assert_invariants()
    assert results[0] == results[1]


@pytest.mark.gpu
@pytest.mark.parametrize("micro_batches", [1, 2])
def test_graph_replayed_decode_equals_the_eager_decode(gpu, micro_batches):
    """Engine(graph=True) replays each batch composition's step from a HIP
    graph captured at its first step. Run in lockstep with an eager batched
    engine on the same model and prompts (separate caches of one config),
    over admissions (each new composition is captured) and a finished
    request, with the engines' own host work and synchronisations between
    the replays: every step's logits are equal bit for bit, and so are the
    tokens. Projections of this model all take nhs_linear_small_m. With two
    micro-batches the graph holds both groups' schedule, each gather a branch
    on the transfer stream beside the other group's compute."""
    log_case(test="decode-graph", micro_batches=micro_batches)
    cfg = ModelConfig(vocab_size=32000, hidden_size=2048, intermediate_size=4096, num_hidden_layers=2,
                      num_attention_heads=16, num_key_value_heads=4)
    torch.manual_seed(7)
    default = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(gpu):
            model = Model(cfg).eval()
    finally:
        torch.set_default_dtype(default)
    P, top = 16, 4
    hot = HotConfig(top * P, top * P)
    g = torch.Generator().manual_seed(3)
    prompts = [torch.randint(0, cfg.vocab_size, (n,), generator=g).tolist() for n in (200, 150, 260)]
    budgets = (12, 5, 12)  # the second request finishes mid-run: a new composition

    def engine(graph):
        kv = CacheConfig(gpu_pages=3 * hot.admission_blocks(P, 2) + 16, host_pages=3 * 2 * 24, page_size=P,
                         kv_heads=4, head_dim=128, dtype=torch.bfloat16, device=str(gpu))
        e = Engine(model, HybridKVCache(kv, hot), top_k=top, batch_decode=True, graph=graph,
                   micro_batches=micro_batches)
        for i, (prompt, n) in enumerate(zip(prompts, budgets)):
            e.add_request(f"r{i}", prompt, n)
        return e

    seen = []
    decode_batch = model.decode_batch

    def recording(*a, **k):
        out = decode_batch(*a, **k)
        seen.append((k.get("graph", False), out.clone()))
        return out

    model.decode_batch = recording
    try:
        eager, replayed = engine(False), engine(True)
        steps = 0
        while eager.waiting or eager.running:
            a, b = eager.step(), replayed.step()
            torch.cuda.synchronize()
            assert a == b, steps
            steps += 1
    finally:
        del model.decode_batch
    assert steps >= 10
    pairs = list(zip(seen[0::2], seen[1::2]))
    assert pairs and all(not ge and gr for (ge, _), (gr, _) in pairs)
    for i, ((_, le), (_, lr)) in enumerate(pairs):
        assert torch.equal(le.view(torch.int32), lr.view(torch.int32)), i
    graphs = model.__dict__["_decode_graphs"]
    assert 1 <= len(graphs) < len(pairs)  # most steps replayed an existing graph
    # A step on another cache drops the graphs captured against the old one,
    # which then keep neither that cache (its pool) nor their memory alive;
    # clear_decode_graphs() drops the rest.
    import gc
    import weakref

    old_cache = weakref.ref(replayed.cache)
    del replayed
    fresh = engine(True)
    for _ in range(2):
        fresh.step()
    torch.cuda.synchronize()
    graphs = model.__dict__["_decode_graphs"]
    assert graphs and all(e["cache"] is fresh.cache for e in graphs.values())
    gc.collect()
    assert old_cache() is None
    model.clear_decode_graphs()
    assert "_decode_graphs" not in model.__dict__
    fresh.step()  # captures again
    assert len(model.__dict__["_decode_graphs"]) == 1
