"""Full-size decode workloads on the GPU against the C oracle.

- CPU plumbing config: a random-init 2-layer decoder (hidden 256, 4/2 heads
  of 64, MLP 688, vocab 32000, fp32, seed 42), 3 prompts of 512 seeded
  random tokens, pages of 16, Quest top-8 pages (sink and last page inside
  the 8), 64 greedy tokens each, round robin. The configured hot buffer of
  64 rows is below the 128-row selection and fails HotConfig, so hot rows =
  128 (the reference's minimum legal value); a pool of exactly one hot
  region + 2 tails per layer would admit one request at a time, so the pool
  is 3x that. The GPU engine must generate the CPU (oracle) engine's tokens
  and row counters, and both must equal the reference package's own run of
  this config (tests/golden/reference_plumbing_tokens.json, written by
  tests/golden/make_reference_tokens.py from the reference on the CPU): all
  192 tokens and the resident / hot / miss row counters.

- Default benchmark step: 16 requests of 32K tokens, Llama-3-8B heads,
  top-32 pages, the selected pages 16 resident / 8 hot / 8 in host memory:
  one step bit-exact (positions, rows, tags, LRU, pool bytes), attention
  within 2e-2.
- Resolver stress: 64 requests with Qwen2-7B heads (28 query / 4 KV heads x
  128, bf16), contexts uniform in [4096, 65536], pages of 32, a 1024-row
  budget (32 pages), 2048 hot rows per request all occupied, 16 decode steps
  with fresh queries: selected pages, row addresses, miss plans, tags and
  LRU order bit-exact at every step.
- Miss-heavy long context: 4 requests of 131072 tokens (2048 pages of 64),
  Llama-3-8B heads, a 4096-row budget (64 pages) of which only the two tail
  pages are resident and 4 are in the hot buffer, so ~90% of the rows are
  gathered from pinned host memory; K/V are N(0, 1) plus a per-page offset
  N(0, 0.5) so Quest scores are spread out. Selection, rows and gathered
  bytes bit-exact; attention within 2e-2.
"""

import gc
import json
import os

import numpy as np
import pytest
import torch

import oracle
from nano_hisparse import row_kernels as rk


def _release_memory():
    """Frees what earlier tests left cached: device blocks and the pinned host
    blocks of their host stores (the full-size tests pin up to 16 GiB each)."""
    gc.collect()
    torch.cuda.empty_cache()
    torch._C._host_emptyCache()


def log_case(**kw):
    print("case:", kw, flush=True)


def run_plumbing_config(device):
    from nano_hisparse.config import CacheConfig
    from nano_hisparse.engine import Engine
    from nano_hisparse.hybrid import HotConfig, HybridKVCache
    from nano_hisparse.model import Model, ModelConfig

    torch.manual_seed(42)
    cfg = ModelConfig(vocab_size=32000, hidden_size=256, intermediate_size=688, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2)
    model = Model(cfg).eval().to(device)  # initialised on the CPU: same weights everywhere
    P, top, T, new = 16, 8, 512, 64
    hot = HotConfig(top * P, top * P)
    g = torch.Generator().manual_seed(42)
    prompts = [torch.randint(0, cfg.vocab_size, (T,), generator=g).tolist() for _ in range(3)]
    kv = CacheConfig(gpu_pages=3 * hot.admission_blocks(P, cfg.num_hidden_layers),
                     host_pages=3 * cfg.num_hidden_layers * -(-(T + new) // P), page_size=P, kv_heads=2,
                     head_dim=64, device=str(device))
    cache = HybridKVCache(kv, hot)
    engine = Engine(model, cache, top_k=top)
    for i, prompt in enumerate(prompts):
        engine.add_request(f"p{i}", prompt, new)
    out = engine.run()
    cache.assert_invariants()
    return out, cache.snapshot()["row_stats"]


def reference_plumbing_run():
    """Tokens and row counters of the reference package's own run of the
    plumbing config (a fixture; the reference is not imported here)."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_plumbing_tokens.json")
    with open(path) as f:
        record = json.load(f)
    return record["tokens"], record["row_stats"]


def test_plumbing_config_runs_on_the_oracle(cpu_kernels):
    out, stats = run_plumbing_config("cpu")
    assert sorted(out) == ["p0", "p1", "p2"] and all(len(v) == 64 for v in out.values())
    assert stats["misses"] > 0 and stats["hot_hits"] > 0
    tokens, ref_stats = reference_plumbing_run()
    assert {k: list(v) for k, v in out.items()} == tokens
    assert dict(stats) == ref_stats


@pytest.mark.gpu
def test_plumbing_config_matches_the_oracle_engine(gpu):
    log_case(test="plumbing-config")
    import cpu_provider

    cpu_provider.install()
    try:
        want, want_stats = run_plumbing_config("cpu")
    finally:
        cpu_provider.uninstall()
    got, got_stats = run_plumbing_config(gpu)
    assert got == want
    assert got_stats == want_stats
    tokens, ref_stats = reference_plumbing_run()
    assert {k: list(v) for k, v in got.items()} == tokens
    assert dict(got_stats) == ref_stats


@pytest.mark.gpu
def test_resolver_stress_64_requests_16_steps(gpu):
    log_case(test="resolver-stress", B=64, steps=16)
    B, Hq, Hkv, D, P, K, H = 64, 28, 4, 128, 32, 1024, 2048
    top = K // P
    g = torch.Generator(device=gpu).manual_seed(42)
    rng = np.random.default_rng(42)
    lengths = rng.integers(4096, 65536 + 1, size=B)
    n_pages = int(-(-lengths.max() // P))
    counts = -(-lengths // P)
    # per-page key bounds of random N(0,1) keys (bf16, exact min/max of 32 rows)
    minimum = torch.empty(B, n_pages, Hkv, D, dtype=torch.bfloat16, device=gpu)
    maximum = torch.empty_like(minimum)
    for b in range(B):
        keys = torch.randn(n_pages, P, Hkv, D, generator=g, device=gpu).to(torch.bfloat16)
        minimum[b], maximum[b] = keys.amin(1), keys.amax(1)
    # host pages, resident pages (30% of each history) and a fully occupied hot buffer
    hot_blocks = H // P
    source = np.full((B, n_pages), -1, np.int32)
    resident = np.full((B, n_pages), -1, np.int32)
    hot = np.zeros((B, hot_blocks), np.int32)
    tags = np.full((B, H), -1, np.int32)
    lru = np.zeros((B, H), np.int64)
    next_host, next_block = 0, 0
    for b in range(B):
        c = int(counts[b])
        source[b, :c] = np.arange(next_host, next_host + c)
        next_host += c
        hot[b] = np.arange(next_block, next_block + hot_blocks)
        next_block += hot_blocks
        res = rng.permutation(c)[: (3 * c) // 10]
        resident[b, res] = np.arange(next_block, next_block + res.size)
        next_block += res.size
        nonres = np.flatnonzero(resident[b, :c] < 0)
        cand = (source[b, nonres][:, None].astype(np.int64) * P + np.arange(P)).ravel()
        tags[b] = rng.choice(cand, size=H, replace=False)  # 100% occupancy
        lru[b] = rng.permutation(H)
    g_len = torch.from_numpy(lengths).to(gpu)
    g_src, g_res, g_hot = (torch.from_numpy(x).to(gpu) for x in (source, resident, hot))
    g_tags, g_lru = torch.from_numpy(tags).to(gpu), torch.from_numpy(lru).to(gpu)
    o_tags, o_lru = tags.astype(np.int64), lru.copy()
    c_min, c_max = minimum.cpu(), maximum.cpu()
    replaced = 0
    for step in range(16):
        q = torch.randn(B, Hq, D, generator=g, device=gpu).to(torch.bfloat16)
        pages, positions, _ = rk.quest_batched(q, minimum, maximum, g_len, P, top)
        if step < 2:  # the CPU Quest oracle over all 64 requests takes seconds
            _, e_pages, e_pos = oracle.quest_select(q.cpu(), c_min, c_max, lengths, P, top)
            assert torch.equal(pages.cpu(), e_pages), f"step {step}: pages"
            assert torch.equal(positions.cpu(), e_pos), f"step {step}: positions"
        phys, mh, md, cnt = rk.resolve_batched(positions, g_src, g_res, g_hot, g_tags, g_lru, g_len, P)
        pos_np = positions.cpu().numpy()
        phys, mh, md, cnt = (t.cpu().numpy() for t in (phys, mh, md, cnt))
        for b in range(B):
            e_phys, e_mh, e_md, e_cnt = oracle.resolve_rows(
                pos_np[b], source[b], resident[b], hot[b], o_tags[b], o_lru[b], lengths[b], P
            )
            np.testing.assert_array_equal(phys[b], e_phys, err_msg=f"step {step} request {b}: rows")
            np.testing.assert_array_equal(mh[b], e_mh)
            np.testing.assert_array_equal(md[b], e_md)
            np.testing.assert_array_equal(cnt[b], e_cnt)
            replaced += int(e_cnt[2])
        np.testing.assert_array_equal(g_tags.cpu().numpy(), o_tags, err_msg=f"step {step}: tags")
        np.testing.assert_array_equal(g_lru.cpu().numpy(), o_lru, err_msg=f"step {step}: lru")
    assert replaced > 0  # every step evicts from a full hot buffer


@pytest.mark.gpu
def test_default_step_full_size_matches_the_oracle(gpu):
    """The benchmark's default step at full size (16 requests, 32K context,
    Llama-3-8B heads, bf16, top-32 pages = 2048 rows, of the selected pages
    16 resident / 8 hot / 8 in host memory, 4096 hot rows), built by
    bench.py's workload classes, one step of SparseDecodeBatch against the C
    oracle request by request: positions, physical rows, tags, LRU order and
    the whole pool after the gather bit-exact; attention within 2e-2 of the
    float64 oracle."""
    log_case(test="default-step", B=16, context=32768)
    import bench

    store = bench.HostStore(16, 32768, 1234, gpu)
    w = bench.Layer(store, 1234)
    B, P, top = w.batch, w.page, w.top_pages
    cpool = w.pool.cpu()
    q, mn, mx, lengths = w.q.cpu(), w.minimum.cpu(), w.maximum.cpu(), w.lengths.cpu()
    result = bench.run_step(w)
    torch.cuda.synchronize()
    _, _, e_pos = oracle.quest_select(q, mn, mx, lengths, P, top)
    assert torch.equal(result.positions.cpu(), e_pos)
    source, resident, hot = w.source.cpu().numpy(), w.resident.cpu().numpy(), w.hot.cpu().numpy()
    tags, lru = w.tags0.cpu().numpy().astype(np.int64), w.lru0.cpu().numpy().copy()
    e_phys = np.empty((B, w.K), np.int64)
    counts = np.zeros(3, np.int64)
    for b in range(B):
        ph, mh, md, cnt = oracle.resolve_rows(e_pos[b].numpy(), source[b], resident[b], hot[b], tags[b], lru[b],
                                               int(lengths[b]), P)
        oracle.gather_rows(w.host, cpool, mh, md, P)
        e_phys[b] = ph
        counts += cnt
    assert counts.tolist() == [16 * 16 * P, 16 * 8 * P, 16 * 8 * P]  # resident / hot / missed rows, as built
    np.testing.assert_array_equal(result.physical.cpu().numpy(), e_phys)
    np.testing.assert_array_equal(w.tables.tags.cpu().numpy(), tags)
    np.testing.assert_array_equal(w.tables.lru.cpu().numpy(), lru)
    assert torch.equal(w.pool.cpu().view(torch.uint8), cpool.view(torch.uint8))
    e_out = oracle.attend_rows(q, cpool, torch.from_numpy(e_phys), P)
    assert (w.out.float().cpu() - e_out).abs().max().item() <= 2e-2
    del w, store, result, cpool
    _release_memory()


@pytest.mark.gpu
def test_miss_heavy_long_context(gpu):
    log_case(test="miss-heavy", B=4, context=131072)
    from nano_hisparse.batch_step import BatchTables, SparseDecodeBatch

    B, Hq, Hkv, D, P, ctx, top, H = 4, 32, 8, 128, 64, 131072, 64, 8192
    n_pages, K = ctx // P, top * P
    dtype = torch.bfloat16
    g = torch.Generator(device=gpu).manual_seed(43)
    host = torch.empty(B * n_pages, 2, P, Hkv, D, dtype=dtype, pin_memory=True)
    mn = torch.empty(B * n_pages, Hkv, D, dtype=dtype, device=gpu)
    mx = torch.empty_like(mn)
    chunk = 512
    for s in range(0, B * n_pages, chunk):
        kv = torch.randn(chunk, 2, P, Hkv, D, generator=g, device=gpu)
        kv += 0.5 * torch.randn(chunk, 1, 1, 1, 1, generator=g, device=gpu)  # per-page offset
        kv = kv.to(dtype)
        host[s : s + chunk].copy_(kv)
        mn[s : s + chunk] = kv[:, 0].amin(1)
        mx[s : s + chunk] = kv[:, 0].amax(1)
    minimum, maximum = mn.view(B, n_pages, Hkv, D), mx.view(B, n_pages, Hkv, D)
    q = torch.randn(B, Hq, D, generator=g, device=gpu).to(dtype)
    lengths = torch.full((B,), ctx, dtype=torch.int64, device=gpu)
    pages, _, _ = rk.quest_batched(q, minimum, maximum, lengths, P, top)
    pages = pages.cpu()
    # residency over the selected pages: the two tail pages resident, 4 pages
    # in the hot buffer, the other 58 only in host memory
    hot_blocks = H // P
    blocks_per = hot_blocks + 2
    pool = torch.zeros(B * blocks_per, 2, P, Hkv, D, dtype=dtype, device=gpu)
    source = torch.arange(B * n_pages, dtype=torch.int32).view(B, n_pages)
    resident = torch.full((B, n_pages), -1, dtype=torch.int32)
    hot = torch.empty(B, hot_blocks, dtype=torch.int32)
    tags = torch.full((B, H), -1, dtype=torch.int32)
    rng = np.random.default_rng(7)
    for b in range(B):
        sel = pages[b].tolist()
        base = b * blocks_per
        hot[b] = torch.arange(base, base + hot_blocks, dtype=torch.int32)
        for i, p in enumerate((n_pages - 2, n_pages - 1)):
            resident[b, p] = base + hot_blocks + i
            pool[base + hot_blocks + i] = host[b * n_pages + p].to(gpu)
        others = [p for p in sel if p < n_pages - 2]
        hot_pages = rng.choice(others, size=4, replace=False)
        slots = rng.permutation(H)[: 4 * P]
        rows = torch.tensor([(b * n_pages + int(p)) * P + o for p in hot_pages for o in range(P)], dtype=torch.int32)
        tags[b, torch.from_numpy(slots)] = rows
        for s_, r in zip(slots.tolist(), rows.tolist()):
            hb, ho = divmod(r, P)
            pool[int(hot[b, s_ // P]), :, s_ % P] = host[hb, :, ho].to(gpu)
    lru = torch.stack([torch.from_numpy(rng.permutation(H)) for _ in range(B)])
    tables = BatchTables(source, resident, hot, tags, lru, minimum.cpu(), maximum.cpu(), lengths.cpu())
    dev = BatchTables(source.to(gpu), resident.to(gpu), hot.to(gpu), tags.to(gpu), lru.to(gpu), minimum, maximum,
                      lengths)
    cpool = pool.cpu()
    step = SparseDecodeBatch(pool, host, dev, P, top)
    out, result = step.step(q)
    torch.cuda.synchronize()
    # the oracle, request by request
    _, e_pages, e_pos = oracle.quest_select(q.cpu(), tables.minimum, tables.maximum, tables.lengths, P, top)
    assert torch.equal(result.positions.cpu(), e_pos)
    o_tags, o_lru = tags.numpy().astype(np.int64), lru.numpy().copy()
    e_phys = np.empty((B, K), np.int64)
    misses = 0
    for b in range(B):
        ph, mh_, md_, cnt = oracle.resolve_rows(
            e_pos[b].numpy(), source[b].numpy(), resident[b].numpy(), hot[b].numpy(), o_tags[b], o_lru[b], ctx, P
        )
        oracle.gather_rows(host, cpool, mh_, md_, P)
        e_phys[b] = ph
        misses += int(cnt[2])
    assert misses >= int(0.85 * B * K)  # ~90% of the selected rows come from host memory
    np.testing.assert_array_equal(result.physical.cpu().numpy(), e_phys)
    np.testing.assert_array_equal(dev.tags.cpu().numpy(), o_tags)
    np.testing.assert_array_equal(dev.lru.cpu().numpy(), o_lru)
    assert torch.equal(pool.cpu().view(torch.uint8), cpool.view(torch.uint8))
    e_out = oracle.attend_rows(q.cpu(), cpool, torch.from_numpy(e_phys), P)
    assert (out.float().cpu() - e_out).abs().max().item() <= 2e-2


def _llama8b_width_model(device, layers):
    """A random-init decoder of Llama-3-8B width (hidden 4096, 32/8 heads x
    128, MLP 14336, vocab 128256, bf16, seed 42) with `layers` layers."""
    from nano_hisparse.model import Model, ModelConfig

    cfg = ModelConfig(vocab_size=128256, hidden_size=4096, intermediate_size=14336, num_hidden_layers=layers,
                      num_attention_heads=32, num_key_value_heads=8, rope_theta=10000.0)
    torch.manual_seed(42)
    default_dtype = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(device):
            return Model(cfg).eval()
    finally:
        torch.set_default_dtype(default_dtype)


def _llama8b_width_engine(device, layers, prompt, new_tokens, B=8, model=None, resident=0.3, admit=True):
    """B requests of `prompt` seeded random tokens through the batched
    engine on a Llama-3-8B-width decoder (_llama8b_width_model): pages of
    64, 2048 hot rows, Quest top-32 pages and a pool of the admission
    credits plus `resident` of the history. With `admit`, steps the engine
    until every request is admitted (admitted requests decode meanwhile)."""
    from math import ceil

    from nano_hisparse.config import CacheConfig
    from nano_hisparse.engine import Engine
    from nano_hisparse.hybrid import HotConfig, HybridKVCache

    if model is None:
        model = _llama8b_width_model(device, layers)
    P, H, top = 64, 2048, 32
    pages = ceil((prompt + new_tokens) / P)
    hot = HotConfig(H, H)
    kv = CacheConfig(gpu_pages=B * hot.admission_blocks(P, layers) + int(resident * B * layers * pages),
                     host_pages=B * layers * pages, page_size=P, kv_heads=8, head_dim=128, dtype=torch.bfloat16,
                     device=str(device), index_budget_bytes=1 << 31)
    cache = HybridKVCache(kv, hot)
    engine = Engine(model, cache, top_k=top, batch_decode=True)
    g = torch.Generator().manual_seed(42)
    for b in range(B):
        engine.add_request(f"r{b}", torch.randint(0, model.config.vocab_size, (prompt,), generator=g).tolist(),
                           new_tokens)
    while admit and engine.waiting:
        engine.step()
    return engine, cache


@pytest.mark.gpu
def test_llama8b_width_batched_decode_matches_the_oracle_per_layer(gpu, monkeypatch):
    """Config 4's width at 2 layers: 8 requests x 8229-token prompts (129
    pages, so Quest scores them and picks 32; a history four times the
    32-block hot region, so with a pool of the admission credits plus 30% of
    the history most pages live on the host and selected rows are gathered),
    2048 hot rows, top-32 pages. For every layer of
    every batched decode step (Model.decode_batch -> BatchDecode), the
    selected pages and positions, resolved rows, miss plans, counts, tags
    and LRU order, and the whole pool after the gather equal the oracle's on
    the same inputs, and attention is within 2e-2 of the oracle's."""
    from nano_hisparse import batched

    log_case(test="llama8b-width", layers=2, requests=8, prompt=8229)
    steps = 4
    # admission decodes the admitted requests meanwhile: nobody may finish before the checked steps end
    engine, cache = _llama8b_width_engine(gpu, layers=2, prompt=8229, new_tokens=8 + steps + 2)
    store = cache.storage
    P = cache.config.page_size
    expected_out = {}
    checked = []
    orig_select, orig_finish = batched.BatchDecode.select, batched.BatchDecode.finish

    def select(self, layer, query, top_pages, keep_sink=True):
        torch.cuda.synchronize()
        reqs = [store.requests[r] for r in self.ids]
        lengths = torch.tensor([r.lengths[layer] for r in reqs])
        mn = torch.stack([r.minimum[layer][: self.max_pages] for r in reqs]).cpu()
        mx = torch.stack([r.maximum[layer][: self.max_pages] for r in reqs]).cpu()
        tables = [cache.tables[r, layer] for r in self.ids]
        src = [t.source.cpu().numpy() for t in tables]
        res = [t.resident.cpu().numpy() for t in tables]
        hot = [t.hot.cpu().numpy() for t in tables]
        tags = [t.tags.cpu().numpy().astype(np.int64) for t in tables]
        lru = [t.lru.cpu().numpy().copy() for t in tables]
        q, pool = query.cpu(), cache.pool.cpu()
        seen = {}

        def quest_items(*a, **k):
            seen["quest"] = rk_quest(*a, **k)
            return seen["quest"]

        def resolve_items(*a, **k):
            seen["resolve"] = rk_resolve(*a, **k)
            return seen["resolve"]

        def select_resolve_items(*a, **k):
            seen["fused"] = rk_fused(*a, **k)
            return seen["fused"]

        hooks = {"quest_items": quest_items, "resolve_items": resolve_items,
                 "select_resolve_items": select_resolve_items}
        for name, f in hooks.items():
            monkeypatch.setattr(rk, name, f)
        try:
            handle = orig_select(self, layer, query, top_pages, keep_sink)
        finally:
            for name, f in originals.items():
                monkeypatch.setattr(rk, name, f)
        torch.cuda.synchronize()
        _, e_pages, e_pos = oracle.quest_select(q, mn, mx, lengths, P, top_pages, keep_sink)
        # this shape takes the fused selection + resolve launch
        assert "fused" in seen and "resolve" not in seen
        pages, positions = seen["fused"][:2]
        assert torch.equal(pages.cpu(), e_pages) and torch.equal(positions.cpu(), e_pos), layer
        physical, mh, md, counts = (t.cpu().numpy() for t in seen["fused"][2:])
        for b, t in enumerate(tables):
            want = oracle.resolve_rows(e_pos[b].numpy(), src[b], res[b], hot[b], tags[b], lru[b],
                                       int(lengths[b]), P)
            for got, exp in zip((physical[b], mh[b], md[b], counts[b]), want):
                np.testing.assert_array_equal(got, exp)
            np.testing.assert_array_equal(t.tags.cpu().numpy(), tags[b])
            np.testing.assert_array_equal(t.lru.cpu().numpy(), lru[b])
        oracle.gather_rows(store.host, pool, mh.reshape(-1), md.reshape(-1), P)
        assert torch.equal(cache.pool.cpu().view(torch.uint8), pool.view(torch.uint8)), layer
        expected_out[id(self), layer] = oracle.attend_rows(q, pool, torch.from_numpy(physical), P)
        checked.append((layer, int(counts[:, 2].sum())))
        return handle

    def finish(self, handle):
        out = orig_finish(self, handle)
        torch.cuda.synchronize()
        want = expected_out.pop((id(self), handle[0]))
        assert (out.cpu().float() - want).abs().max().item() <= 2e-2
        return out

    rk_quest, rk_resolve, rk_fused = rk.quest_items, rk.resolve_items, rk.select_resolve_items
    originals = {"quest_items": rk_quest, "resolve_items": rk_resolve, "select_resolve_items": rk_fused}
    monkeypatch.setattr(batched.BatchDecode, "select", select)
    monkeypatch.setattr(batched.BatchDecode, "finish", finish)
    for _ in range(steps):
        assert len(engine.step()) == 8
    assert len(checked) == 2 * steps and not expected_out
    assert sum(m for _, m in checked) > 0  # rows were gathered from the host store
    cache.assert_invariants()


def _compact_rows(pool, physical, P):
    """The pool rows that `physical` [B, K] (-1 masked) names, copied to the
    host as a compact pool of their own, and the same rows renumbered into
    it: attention over them equals attention over the whole pool."""
    B, K = physical.shape
    valid = physical >= 0
    rows = physical[valid]
    blocks = -(-max(1, rows.numel()) // P)
    flat = torch.zeros(blocks * P, 2, pool.shape[3], pool.shape[4], dtype=pool.dtype)
    if rows.numel():
        flat[: rows.numel()] = pool[rows // P, :, rows % P].cpu()
    compact = flat.view(blocks, P, 2, pool.shape[3], pool.shape[4]).transpose(1, 2).contiguous()
    renum = torch.full((B, K), -1, dtype=torch.int64)
    renum[valid.cpu()] = torch.arange(rows.numel())
    return compact, renum


@pytest.mark.gpu
@pytest.mark.timeout(900)
def test_llama8b_full_size_decode_matches_the_oracle_per_layer(gpu, monkeypatch):
    """Config 4 at full size: 32 layers, 8 requests x 16384-token prompts,
    2048 hot rows, Quest top-32 pages, a pool of the admission credits plus
    30% of the history. For every layer of two batched decode steps, the
    selected pages and positions, resolved rows, miss plans, counts, tags
    and LRU order equal the oracle's on the same inputs; every gathered pool
    row equals its host row byte for byte; and attention is within 2e-2 of
    the oracle's over the selected rows (copied to the host on their own:
    only the rows a layer's plan touches leave the device, not the pool)."""
    from nano_hisparse import batched

    log_case(test="llama8b-full", layers=32, requests=8, prompt=16384)
    _release_memory()
    steps, layers = 2, 32
    engine, cache = _llama8b_width_engine(gpu, layers=layers, prompt=16384, new_tokens=8 + steps + 2)
    store = cache.storage
    P = cache.config.page_size
    expected_out = {}
    checked = []
    orig_select, orig_finish = batched.BatchDecode.select, batched.BatchDecode.finish
    rk_fused = rk.select_resolve_items

    def select(self, layer, query, top_pages, keep_sink=True):
        torch.cuda.synchronize()
        reqs = [store.requests[r] for r in self.ids]
        lengths = torch.tensor([r.lengths[layer] for r in reqs])
        mn = torch.stack([r.minimum[layer][: self.max_pages] for r in reqs]).cpu()
        mx = torch.stack([r.maximum[layer][: self.max_pages] for r in reqs]).cpu()
        tables = [cache.tables[r, layer] for r in self.ids]
        src = [t.source.cpu().numpy() for t in tables]
        res = [t.resident.cpu().numpy() for t in tables]
        hot = [t.hot.cpu().numpy() for t in tables]
        tags = [t.tags.cpu().numpy().astype(np.int64) for t in tables]
        lru = [t.lru.cpu().numpy().copy() for t in tables]
        q = query.cpu()
        seen = {}

        def select_resolve_items(*a, **k):
            seen["fused"] = rk_fused(*a, **k)
            return seen["fused"]

        monkeypatch.setattr(rk, "select_resolve_items", select_resolve_items)
        try:
            handle = orig_select(self, layer, query, top_pages, keep_sink)
        finally:
            monkeypatch.setattr(rk, "select_resolve_items", rk_fused)
        torch.cuda.synchronize()  # the gather has landed
        _, e_pages, e_pos = oracle.quest_select(q, mn, mx, lengths, P, top_pages, keep_sink)
        assert "fused" in seen, layer
        pages, positions = seen["fused"][:2]
        assert torch.equal(pages.cpu(), e_pages) and torch.equal(positions.cpu(), e_pos), layer
        physical_dev = seen["fused"][2]
        physical, mh, md, counts = (t.cpu().numpy() for t in seen["fused"][2:])
        for b, t in enumerate(tables):
            want = oracle.resolve_rows(e_pos[b].numpy(), src[b], res[b], hot[b], tags[b], lru[b],
                                       int(lengths[b]), P)
            for got, exp in zip((physical[b], mh[b], md[b], counts[b]), want):
                np.testing.assert_array_equal(got, exp)
            np.testing.assert_array_equal(t.tags.cpu().numpy(), tags[b])
            np.testing.assert_array_equal(t.lru.cpu().numpy(), lru[b])
        # gathered rows: pool row md holds host row mh, both planes, byte for byte
        miss = mh.reshape(-1) >= 0
        h_rows, d_rows = torch.from_numpy(mh.reshape(-1)[miss]), torch.from_numpy(md.reshape(-1)[miss])
        got = cache.pool[d_rows.to(gpu) // P, :, d_rows.to(gpu) % P].cpu()
        want = store.host[h_rows // P, :, h_rows % P]
        assert torch.equal(got.view(torch.uint8), want.view(torch.uint8)), layer
        compact, renum = _compact_rows(cache.pool, physical_dev, P)
        expected_out[id(self), layer] = oracle.attend_rows(q, compact, renum, P)
        checked.append((layer, int(miss.sum())))
        return handle

    def finish(self, handle):
        out = orig_finish(self, handle)
        torch.cuda.synchronize()
        want = expected_out.pop((id(self), handle[0]))
        assert (out.cpu().float() - want).abs().max().item() <= 2e-2, handle[0]
        return out

    monkeypatch.setattr(batched.BatchDecode, "select", select)
    monkeypatch.setattr(batched.BatchDecode, "finish", finish)
    for step in range(steps):
        assert len(engine.step()) == 8
        print(f"step {step}: {layers} layers checked", flush=True)
    assert len(checked) == layers * steps and not expected_out
    assert sum(m for _, m in checked) > 0  # rows were gathered from the host store
    cache.assert_invariants()


@pytest.mark.gpu
@pytest.mark.timeout(900)
def test_llama8b_full_size_tokens_do_not_depend_on_the_pool_size(gpu):
    """Config 4 at full size (32 layers, 8 x 16384-token prompts, 2048 hot
    rows, Quest top-32) generates the same greedy tokens with a pool of the
    admission credits plus 30% of the history (most selected rows gathered
    from the host) as with a pool that keeps the whole history resident: the
    reference's partial-residency property (tests/test_engine.py:27-64) at
    config 4's size, over 24 tokens per request."""
    log_case(test="llama8b-pool-sizes", layers=32, requests=8, prompt=16384)
    _release_memory()
    model = _llama8b_width_model(gpu, 32)
    outputs, misses = [], []
    for resident in (0.3, 1.0):
        engine, cache = _llama8b_width_engine(gpu, layers=32, prompt=16384, new_tokens=24, model=model,
                                              resident=resident, admit=False)
        outputs.append(engine.run())
        misses.append(cache.snapshot()["row_stats"]["misses"])
        cache.assert_invariants()
        print(f"pool {resident}: misses {misses[-1]}", flush=True)
        del engine, cache
        _release_memory()  # the cache's pinned host store is released before the next one is allocated
    assert misses[0] > 0
    assert outputs[0] == outputs[1]
    assert all(len(t) == 24 for t in outputs[0].values())
