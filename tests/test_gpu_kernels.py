"""Parity of the HIP kernels (through the C ABI) with the CPU oracle.

Integer and byte outputs (selected pages, positions, resolved rows, miss
plans, tags, LRU order, gathered bytes) must be bit-exact; Quest scores are
bit-exact because the oracle restates the kernels' fixed fp32 summation
order; attention must be within max-abs 2e-2 (bf16/fp16) or 1e-4 (fp32) of
the oracle's float64 masked softmax.
"""

import math

import numpy as np
import pytest
import torch

import oracle
from nano_hisparse import row_kernels as rk

pytestmark = pytest.mark.gpu

ATOL = {torch.bfloat16: 2e-2, torch.float16: 2e-2, torch.float32: 1e-4}


def log_case(**kw):
    print("case:", kw, flush=True)


# ---- gather ----------------------------------------------------------------------


@pytest.mark.parametrize(
    "dtype,page,kv_heads,head_dim",
    [(torch.bfloat16, 64, 8, 128), (torch.float32, 4, 1, 8), (torch.float16, 7, 2, 24), (torch.float32, 3, 1, 1)],
)
def test_gather_rows_bit_exact(gpu, dtype, page, kv_heads, head_dim):
    log_case(test="gather", dtype=dtype, page=page, kv_heads=kv_heads, head_dim=head_dim)
    g = torch.Generator().manual_seed(1)
    host_pages, pool_blocks = 48, 20
    host = torch.randn(host_pages, 2, page, kv_heads, head_dim, generator=g).to(dtype).pin_memory()
    pool_cpu = torch.randn(pool_blocks, 2, page, kv_heads, head_dim, generator=g).to(dtype)
    n = 3 * page + 5
    rows = torch.randperm(pool_blocks * page, generator=g)[:n]
    srcs = torch.randint(0, host_pages * page, (n,), generator=g)
    mh, md = srcs.clone(), rows.clone()
    mh[n // 2 :] = -1  # compact prefix, then padding
    md[n // 2 :] = -1
    mh[3] = -1  # a hole inside the prefix is skipped too
    expected = pool_cpu.clone()
    oracle.gather_rows(host, expected, mh, md, page)
    pool = pool_cpu.to(gpu)
    alias = rk.MappedHost(host)
    rk.gather_plan(alias, pool, mh.to(gpu), md.to(gpu), page)
    torch.cuda.synchronize()
    assert torch.equal(pool.cpu().view(torch.uint8), expected.view(torch.uint8))


@pytest.mark.parametrize("dtype,page,kv_heads,head_dim", [(torch.bfloat16, 64, 8, 128), (torch.float16, 16, 2, 64),
                                                      (torch.float32, 8, 4, 32)])
def test_padded_pool_reads_and_writes_as_the_contiguous_pool(gpu, dtype, page, kv_heads, head_dim):
    """The cache's pool leaves rk.POOL_PAD_SLOTS head slots of padding after
    every block (rk.padded_pool). Gather, append and attention on it write and read the
    same rows as on a contiguous pool: the gathered and appended bytes, the
    bounds and the attention outputs are bit-identical, and the padding is
    never written."""
    log_case(test="padded-pool", dtype=dtype, page=page, kv_heads=kv_heads, head_dim=head_dim)
    g = torch.Generator().manual_seed(5)
    blocks, host_pages = 24, 40
    padded = rk.padded_pool(blocks, page, kv_heads, head_dim, dtype, gpu)
    block, pad = 2 * page * kv_heads * head_dim, rk.POOL_PAD_SLOTS * head_dim
    assert padded.stride(0) == block + pad and rk.pool_block_stride(padded) == (block + pad) * padded.element_size()
    flat = torch.as_strided(padded, (blocks * (block + pad),), (1,))
    flat.fill_(7.0)  # the padding must keep this
    start = torch.randn(blocks, 2, page, kv_heads, head_dim, generator=g).to(dtype)
    padded.copy_(start.to(gpu))
    plain = start.to(gpu)
    host = torch.randn(host_pages, 2, page, kv_heads, head_dim, generator=g).to(dtype).pin_memory()
    alias = rk.MappedHost(host)
    n = 3 * page + 5
    md = torch.randperm(blocks * page, generator=g)[:n]
    mh = torch.randint(0, host_pages * page, (n,), generator=g)
    mh[n // 2:], md[n // 2:] = -1, -1
    for pool in (padded, plain):
        rk.gather_plan(alias, pool, mh.to(gpu), md.to(gpu), page)
    # append three tokens into block 5 of each, with bounds
    k = torch.randn(3, kv_heads, head_dim, generator=g).to(dtype).to(gpu)
    v = torch.randn(3, kv_heads, head_dim, generator=g).to(dtype).to(gpu)
    bounds = []
    for pool in (padded, plain):
        summary = torch.zeros(kv_heads, head_dim, dtype=torch.float32, device=gpu)
        lo = torch.full((kv_heads, head_dim), float("inf"), device=gpu).to(dtype)
        hi = torch.full((kv_heads, head_dim), float("-inf"), device=gpu).to(dtype)
        rk.append_page(k, v, pool, 5, 2, None, 0, summary, lo, hi)
        bounds.append((summary, lo, hi))
    torch.cuda.synchronize()
    assert torch.equal(padded.cpu().view(torch.uint8), plain.cpu().view(torch.uint8))
    for x, y in zip(*bounds):
        assert torch.equal(x.view(torch.uint8), y.view(torch.uint8))
    gaps = flat.view(blocks, block + pad)[:, block:]
    assert bool((gaps == 7.0).all())
    if (head_dim * padded.element_size()) % 16 == 0:
        q = torch.randn(2, 2 * kv_heads, head_dim, generator=g).to(dtype).to(gpu)
        rows = torch.randint(0, blocks * page, (2, 3 * page), generator=g)
        rows[0, ::5] = -1
        a = rk.attend_batched(q, padded, rows.to(gpu), page)
        b = rk.attend_batched(q, plain, rows.to(gpu), page)
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))


def test_pool_block_stride_is_checked_by_the_c_abi(gpu):
    """Every entry point that takes the pool's block stride rejects one below
    a block (the attention also one that is not a multiple of 16 bytes),
    before it launches anything; 0 means contiguous blocks."""
    import ctypes

    from nano_hisparse import _hip

    lib = _hip.load()
    P, Hkv, D = 4, 2, 8  # bf16: a block is 2 * 4 * 2 * 8 * 2 = 256 bytes
    pool = torch.zeros(4, 2, P, Hkv, D, dtype=torch.bfloat16, device=gpu)
    host = torch.zeros(4, 2, P, Hkv, D, dtype=torch.bfloat16).pin_memory()
    alias = rk.MappedHost(host)
    plan = torch.full((4,), -1, dtype=torch.int64, device=gpu)
    q = torch.zeros(1, 2 * Hkv, D, dtype=torch.bfloat16, device=gpu)
    rows = torch.zeros(1, 8, dtype=torch.int64, device=gpu)
    out = torch.empty_like(q)
    ws = torch.zeros(lib.nhs_attend_workspace_bytes(1, 2 * Hkv, D, 8), dtype=torch.uint8, device=gpu)
    kv = torch.zeros(1, Hkv, D, dtype=torch.bfloat16, device=gpu)
    lo = torch.full((Hkv, D), float("inf"), dtype=torch.bfloat16, device=gpu)
    hi = torch.full((Hkv, D), float("-inf"), dtype=torch.bfloat16, device=gpu)
    summary = torch.zeros(Hkv, D, dtype=torch.float32, device=gpu)
    s = ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    bf16 = 2

    def gather(stride):
        return lib.nhs_gather_rows(ctypes.c_void_p(alias.data_ptr()), p(pool), p(plan), p(plan), 4, P,
                                   Hkv * D * 2, stride, s)

    def attend(stride):
        return lib.nhs_attend_rows(p(q), bf16, 0, D, p(pool), bf16, stride, p(rows), 0, 0, 1, 1, 8, 2 * Hkv, Hkv, D,
                                   P, p(out), 0, D, p(ws), ws.numel(), s)

    def append(stride):
        return lib.nhs_append_page(p(kv), p(kv), Hkv * D, bf16, Hkv * D, P, p(pool), stride, 1, 0, 1, None, 0,
                                   p(summary), p(lo), p(hi), s)

    for call in (gather, attend, append):
        assert call(255) != 0, call.__name__
        assert b"pool_block_stride" in lib.nhs_last_error(), call.__name__
        assert call(0) == 0 and call(256) == 0 and call(512) == 0, call.__name__
    assert attend(264) != 0 and b"multiple of 16" in lib.nhs_last_error()
    torch.cuda.synchronize()


# ---- attention ------------------------------------------------------------------


def _attention_case(gpu, dtype, q_dtype, B, Hq, Hkv, D, P, N, per_head, seed):
    g = torch.Generator().manual_seed(seed)
    blocks = max(4, (N * 2) // P + 2)
    pool = torch.randn(blocks, 2, P, Hkv, D, generator=g).to(dtype)
    q = torch.randn(B, Hq, D, generator=g).to(q_dtype)
    shape = (B, Hq, N) if per_head else (B, N)
    rows = torch.randint(0, blocks * P, shape, generator=g)
    rows[torch.rand(shape, generator=g) < 0.2] = -1
    return pool, q, rows


@pytest.mark.parametrize(
    "dtype,q_dtype,B,Hq,Hkv,D,P,N,per_head",
    [
        (torch.bfloat16, torch.bfloat16, 3, 32, 8, 128, 64, 700, False),  # Llama-3-8B heads, GQA 4
        (torch.bfloat16, torch.bfloat16, 2, 28, 4, 128, 32, 300, False),  # Qwen2-7B heads, GQA 7
        (torch.float32, torch.float32, 2, 4, 2, 64, 16, 129, False),  # toy fp32 decoder, GQA 2
        (torch.float32, torch.float32, 1, 2, 1, 8, 4, 6, False),
        (torch.float16, torch.float16, 1, 6, 2, 24, 7, 9, False),  # head_dim*2 bytes = 48
        (torch.float16, torch.float16, 2, 4, 2, 24, 3, 11, True),  # per-head (legacy) rows
        (torch.bfloat16, torch.float32, 2, 16, 2, 128, 64, 257, False),  # fp32 query, bf16 KV, GQA 8
        (torch.bfloat16, torch.bfloat16, 1, 48, 4, 64, 16, 100, False),  # GQA 12 (two workgroups per KV head)
        (torch.float32, torch.float32, 1, 3, 3, 256, 8, 40, False),  # 1 KiB rows
        # 256+ (request, KV head) items: one workgroup per item, all 7 heads of a group in it
        (torch.bfloat16, torch.bfloat16, 64, 28, 4, 128, 32, 256, False),
        (torch.bfloat16, torch.float32, 128, 14, 2, 64, 16, 100, False),  # fp32 query: unpacked scores
        (torch.float32, torch.float32, 128, 14, 2, 64, 16, 60, False),
    ],
)
def test_attend_rows_matches_oracle(gpu, dtype, q_dtype, B, Hq, Hkv, D, P, N, per_head):
    log_case(test="attend", dtype=dtype, B=B, Hq=Hq, Hkv=Hkv, D=D, P=P, N=N, per_head=per_head)
    pool, q, rows = _attention_case(gpu, dtype, q_dtype, B, Hq, Hkv, D, P, N, per_head, seed=B * 100 + Hq)
    expected = oracle.attend_rows(q, pool, rows, P)
    out = rk.attend_batched(q.to(gpu), pool.to(gpu), rows.to(gpu), P)
    torch.cuda.synchronize()
    assert out.dtype == q_dtype
    err = (out.cpu().float() - expected).abs().max().item()
    assert err <= ATOL[dtype if dtype != torch.float32 else q_dtype], err


@pytest.mark.parametrize(
    "dtype,B,Hq,Hkv,P,N,all_masked",
    [
        (torch.bfloat16, 1, 8, 8, 64, 33000, False),  # 1 head per KV head; 16 splits of 3 passes each
        (torch.float16, 2, 16, 8, 16, 1500, True),  # 2 heads; request 0 has no valid row
        (torch.bfloat16, 3, 24, 8, 32, 600, False),  # 3 heads
        (torch.float16, 4, 32, 8, 64, 2048, False),  # Llama-3-8B heads in fp16
        (torch.bfloat16, 2, 20, 4, 16, 900, True),  # 5 heads
        (torch.bfloat16, 2, 24, 4, 8, 100, False),  # 6 heads, one tile per wave at most
        (torch.bfloat16, 1, 7, 1, 32, 5, False),  # 7 heads, five rows
        (torch.bfloat16, 5, 64, 8, 64, 1200, False),  # 8 heads
        # (request, KV head) counts that are not a multiple of 8: the splits of
        # one item land on different XCDs, so the merge crosses their L2s
        (torch.bfloat16, 3, 12, 3, 64, 1500, False),  # 9 items x 12 splits
        (torch.float16, 5, 35, 5, 32, 2000, True),  # 7 heads, 25 items x 8 splits
    ],
)
def test_attend_mfma_shapes_match_oracle(gpu, dtype, B, Hq, Hkv, P, N, all_masked):
    """head_dim 128 with 16-bit KV and query and one row list per request
    runs attend_mfma_kernel (QK^T on MFMA): every group size 1-8 it serves,
    fp16 and bf16, row splits merged across workgroups (up to 16), several
    LDS passes per split, a few rows only, 20% masked rows and requests with
    none valid; within the bf16/fp16 tolerance of the float64 oracle, and a
    second call gives the same bits."""
    log_case(test="attend-mfma", dtype=dtype, B=B, Hq=Hq, Hkv=Hkv, P=P, N=N)
    pool, q, rows = _attention_case(gpu, dtype, dtype, B, Hq, Hkv, 128, P, N, False, seed=N + Hq)
    if all_masked:
        rows[0] = -1
    expected = oracle.attend_rows(q, pool, rows, P)
    g_q, g_pool, g_rows = q.to(gpu), pool.to(gpu), rows.to(gpu)
    out = rk.attend_batched(g_q, g_pool, g_rows, P)
    again = rk.attend_batched(g_q, g_pool, g_rows, P)
    torch.cuda.synchronize()
    assert torch.equal(out, again)
    err = (out.cpu().float() - expected).abs().max().item()
    assert err <= ATOL[dtype], err
    if all_masked:
        assert not out[0].any()


@pytest.mark.parametrize("N", [16, 64, 256, 2048])
@pytest.mark.parametrize("score_std,v_std", [(4.0, 4.0), (4.0, 8.0), (3.0, 8.0)])
def test_attend_rows_precision_with_peaky_scores_and_large_values(gpu, N, score_std, v_std):
    """Scores of std 3-4 (few rows carry the weight) and V of std 4-8, bf16
    query and KV (the packed path): within 2e-2 of the float64 oracle beyond
    the rounding of the output to bf16 (half an ulp of the expected value;
    the reference rounds its output to the query's dtype too,
    attention.py:35). The weights stay fp32 in P.V as in the reference
    (row_kernels.py:109-110)."""
    log_case(test="attend-precision", N=N, score_std=score_std, v_std=v_std)
    B, Hq, Hkv, D, P = 4, 32, 8, 128, 64
    g = torch.Generator().manual_seed(N + int(10 * score_std + v_std))
    blocks = max(4, -(-N // P) + 4)
    s = score_std ** 0.5  # q and k of std s: q.k / sqrt(D) has std s^2
    pool = torch.randn(blocks, 2, P, Hkv, D, generator=g)
    pool[:, 0] *= s
    pool[:, 1] *= v_std
    pool = pool.bfloat16()
    q = (s * torch.randn(B, Hq, D, generator=g)).bfloat16()
    rows = torch.stack([torch.randperm(blocks * P, generator=g)[:N] for _ in range(B)])
    expected = oracle.attend_rows(q, pool, rows, P)
    out = rk.attend_batched(q.to(gpu), pool.to(gpu), rows.to(gpu), P).cpu().float()
    mag = torch.maximum(expected.abs(), out.abs()).clamp_min(2.0 ** -126)
    half_ulp = (mag.log2().floor() - 8).exp2()  # bf16 keeps 8 significant bits
    beyond = ((out - expected).abs() - half_ulp).clamp_min(0).max().item()
    print(f"max error beyond output rounding {beyond:.3e}; max-abs {(out - expected).abs().max().item():.3e}")
    assert beyond <= 2e-2


def test_attend_rows_repeated_calls_share_one_workspace(gpu):
    """The splits of a head group are merged by the last workgroup to arrive
    (arrival counters in the workspace, left at zero by every call). Many
    back-to-back calls of alternating shapes on one workspace must each
    produce the same bits as the first call of that shape."""
    log_case(test="attend-repeat")
    cases = [
        _attention_case(gpu, torch.bfloat16, torch.bfloat16, 16, 32, 8, 128, 64, 2048, False, seed=11),
        _attention_case(gpu, torch.bfloat16, torch.bfloat16, 3, 28, 4, 128, 32, 1024, False, seed=12),
    ]
    cases = [(q.to(gpu), pool.to(gpu), rows.to(gpu), P) for (pool, q, rows), P in zip(cases, (64, 32))]
    first = [rk.attend_batched(q, pool, rows, P).clone() for q, pool, rows, P in cases]
    for i in range(60):
        q, pool, rows, P = cases[i % 2]
        out = rk.attend_batched(q, pool, rows, P)
        assert torch.equal(out, first[i % 2]), i
    q, pool, rows, P = cases[1]
    expected = oracle.attend_rows(q.cpu(), pool.cpu(), rows.cpu(), P)
    assert (first[1].cpu().float() - expected).abs().max().item() <= 2e-2


def test_attend_rows_masking_edge_cases(gpu):
    log_case(test="attend-edges")
    P, Hkv, D = 16, 2, 64
    g = torch.Generator().manual_seed(7)
    pool = torch.randn(8, 2, P, Hkv, D, generator=g)
    q = torch.randn(3, 4, D, generator=g)
    rows = torch.full((3, 50), -1, dtype=torch.int64)
    rows[1, 37] = 21  # a single valid row: output is exactly that V row
    rows[2, :] = 5  # the same row repeated: still that V row
    out = rk.attend_batched(q.to(gpu), pool.to(gpu), rows.to(gpu), P).cpu()
    assert torch.equal(out[0], torch.zeros(4, D))  # no valid row -> zeros
    v21 = pool[21 // P, 1, 21 % P]
    v5 = pool[5 // P, 1, 5 % P]
    for h in range(4):
        torch.testing.assert_close(out[1, h], v21[h // 2], atol=1e-6, rtol=1e-6)
        torch.testing.assert_close(out[2, h], v5[h // 2], atol=1e-5, rtol=1e-5)


# ---- resolver -----------------------------------------------------------------------


def make_resolver_state(rng, B, H, P, n_pages, host_pages, pool_blocks, resident_frac, tag_frac):
    """Random but consistent tables: distinct host slots per page, distinct
    resident blocks, hot blocks disjoint from resident blocks, unique tags."""
    source = np.full((B, n_pages), -1, np.int32)
    resident = np.full((B, n_pages), -1, np.int32)
    hot_blocks = -(-H // P)
    hot = np.zeros((B, hot_blocks), np.int32)
    tags = np.full((B, H), -1, np.int32)
    lru = np.zeros((B, H), np.int64)
    for b in range(B):
        source[b] = rng.permutation(host_pages)[:n_pages]
        blocks = rng.permutation(pool_blocks)
        hot[b] = blocks[:hot_blocks]
        res_pages = rng.random(n_pages) < resident_frac
        res_ids = blocks[hot_blocks : hot_blocks + res_pages.sum()]
        resident[b, res_pages] = res_ids
        n_tags = int(H * tag_frac)
        cand = (source[b][:, None].astype(np.int64) * P + np.arange(P)).ravel()
        cand = cand[np.repeat(resident[b] < 0, P)]
        chosen = rng.choice(cand, size=min(n_tags, cand.size), replace=False)
        slots = rng.permutation(H)[: chosen.size]
        tags[b, slots] = chosen
        lru[b] = rng.permutation(H)
    return source, resident, hot, tags, lru


def random_positions(rng, B, K, length, P, mode):
    pos = np.full((B, K), -1, np.int64)
    for b in range(B):
        if mode == "pages":  # whole pages, sorted, tail clipped, -1 padded
            count = -(-int(length[b]) // P)
            k_pages = K // P
            pages = np.sort(rng.choice(count, size=min(k_pages, count), replace=False))
            toks = (pages[:, None] * P + np.arange(P)).ravel()
            toks = toks[toks < length[b]]
            pos[b, : toks.size] = toks
        else:  # arbitrary order, duplicates, out-of-range and negative values
            pos[b] = rng.integers(-3, int(length[b]) + 5, size=K)
            dup = rng.integers(0, K, size=K // 8)
            pos[b, dup] = pos[b, rng.integers(0, K, size=dup.size)]
    return pos


@pytest.mark.parametrize(
    "B,K,H,P,n_pages,mode,steps",
    [
        (4, 2048, 4096, 64, 512, "pages", 3),  # Llama-3-8B shape at 32K context, 2048-row budget
        (8, 1024, 2048, 32, 2048, "pages", 3),  # Qwen2-7B stress shape, H = 2U
        (3, 1024, 1024, 32, 256, "pages", 4),  # H = U: every miss replaces a row
        (2, 777, 1500, 7, 300, "random", 4),  # unsorted, duplicates, invalid entries, odd sizes
        (2, 4096, 8192, 64, 2048, "pages", 2),  # 128K context, 4096-row budget
        (1, 4096, 32768, 16, 4096, "random", 2),  # largest in-LDS sort
        (3, 4097, 8192, 32, 1000, "pages", 2),  # first size of the large-K kernel
        (2, 8192, 16384, 64, 1024, "pages", 3),  # top-128 pages of 64 rows
        (2, 8192, 8192, 64, 512, "random", 3),  # unsorted large K: radix sort, duplicates, H = K
        (2, 5000, 6000, 7, 2000, "random", 3),  # odd sizes
        (1, 32768, 32768, 64, 2048, "pages", 2),  # maximum, sorted (selector output)
        (1, 32768, 32768, 16, 4096, "random", 2),  # maximum, unsorted
    ],
)
def test_resolver_matches_oracle_over_steps(gpu, B, K, H, P, n_pages, mode, steps):
    log_case(test="resolve", B=B, K=K, H=H, P=P, n_pages=n_pages, mode=mode)
    rng = np.random.default_rng(B * 1000 + K)
    host_pages = n_pages * 2
    pool_blocks = n_pages + -(-H // P) + 8
    source, resident, hot, tags, lru = make_resolver_state(rng, B, H, P, n_pages, host_pages, pool_blocks, 0.4, 0.6)
    lengths = rng.integers(n_pages * P // 2, n_pages * P + 1, size=B)
    g_src, g_res, g_hot = (torch.from_numpy(x).to(gpu) for x in (source, resident, hot))
    g_tags, g_lru = torch.from_numpy(tags).to(gpu), torch.from_numpy(lru).to(gpu)
    o_tags, o_lru = tags.astype(np.int64), lru.copy()
    total = torch.zeros(3, dtype=torch.int64, device=gpu)
    expected_total = np.zeros(3, np.int64)
    for step in range(steps):
        pos = random_positions(rng, B, K, lengths, P, mode)
        dtype = torch.int32 if step % 2 else torch.int64
        phys, mh, md, counts = rk.resolve_batched(
            torch.from_numpy(pos).to(gpu, dtype), g_src, g_res, g_hot, g_tags, g_lru,
            torch.from_numpy(lengths).to(gpu), P, counts_total=total,
        )
        phys, mh, md, counts = (t.cpu().numpy() for t in (phys, mh, md, counts))
        for b in range(B):
            e_phys, e_mh, e_md, e_counts = oracle.resolve_rows(
                pos[b], source[b], resident[b], hot[b], o_tags[b], o_lru[b], lengths[b], P
            )
            np.testing.assert_array_equal(phys[b], e_phys)
            np.testing.assert_array_equal(mh[b], e_mh)
            np.testing.assert_array_equal(md[b], e_md)
            np.testing.assert_array_equal(counts[b], e_counts)
            expected_total += e_counts
        np.testing.assert_array_equal(g_tags.cpu().numpy(), o_tags)
        np.testing.assert_array_equal(g_lru.cpu().numpy(), o_lru)
    np.testing.assert_array_equal(total.cpu().numpy(), expected_total)
    for b in range(B):  # invariants: lru is a permutation, non-negative tags are unique
        assert sorted(o_lru[b].tolist()) == list(range(H))
        t = o_tags[b][o_tags[b] >= 0]
        assert t.size == np.unique(t).size


# ---- selectors -----------------------------------------------------------------------


def _bounds(g, B, n_pages, Hkv, D, dtype, offsets=False):
    a = torch.randn(B, n_pages, Hkv, D, generator=g)
    c = torch.randn(B, n_pages, Hkv, D, generator=g)
    if offsets:
        mu = 0.5 * torch.randn(B, n_pages, 1, 1, generator=g)
        a, c = a + mu, c + mu
    return torch.minimum(a, c).to(dtype), torch.maximum(a, c).to(dtype)


@pytest.mark.parametrize(
    "dtype,q_dtype,B,Hq,Hkv,D,P,n_pages,top,keep_sink",
    [
        (torch.bfloat16, torch.bfloat16, 16, 32, 8, 128, 64, 512, 32, True),  # 32K context, 32 pages
        (torch.bfloat16, torch.bfloat16, 4, 32, 8, 128, 64, 2048, 64, True),  # 128K context, 64 pages
        (torch.bfloat16, torch.bfloat16, 8, 28, 4, 128, 32, 2048, 32, True),  # 32 lanes per page: half-wave fold
        (torch.bfloat16, torch.float32, 2, 28, 4, 128, 32, 700, 20, True),  # half-wave fold of an fp32 query
        (torch.float32, torch.float32, 2, 12, 4, 64, 16, 300, 20, True),  # fp32 bounds, half-wave fold, group 3
        (torch.float16, torch.float32, 2, 10, 2, 256, 16, 300, 20, True),  # fp16 bounds, half-wave fold, group 5
        (torch.float32, torch.float32, 3, 4, 2, 64, 16, 40, 8, True),
        (torch.float32, torch.float32, 2, 4, 2, 64, 16, 40, 8, False),
        (torch.float16, torch.float32, 2, 6, 2, 24, 7, 30, 5, True),
        (torch.float32, torch.float32, 2, 2, 1, 2, 2, 3, 2, False),  # head_dim 2 (element lanes)
        (torch.bfloat16, torch.bfloat16, 2, 8, 2, 64, 16, 9000, 300, True),
        (torch.bfloat16, torch.bfloat16, 3, 8, 2, 64, 16, 1000, 40, True),  # four-wave select, 4 keys per lane
        (torch.bfloat16, torch.bfloat16, 2, 8, 2, 64, 4, 900, 300, True),  # 300 chosen: one-wave select, 16 per lane
        (torch.bfloat16, torch.bfloat16, 2, 8, 2, 64, 4, 400, 260, False),  # 260 chosen: one-wave select, 8 per lane
        (torch.bfloat16, torch.bfloat16, 3, 8, 2, 64, 16, 3000, 200, True),  # four-wave select, 16 keys per lane
        (torch.float32, torch.float32, 2, 4, 2, 16, 5, 1500, 150, False),  # four-wave select, 8 keys per lane
        (torch.float32, torch.float32, 2, 4, 2, 16, 5, 513, 64, False),
        (torch.float32, torch.float32, 2, 4, 2, 64, 16, 40, 100, True),  # budget above the page count: -1 padding
        (torch.bfloat16, torch.bfloat16, 2, 96, 8, 128, 64, 300, 16, True),  # 12 query heads per KV head
        (torch.bfloat16, torch.bfloat16, 2, 12, 1, 72, 16, 100, 10, True),  # GQA 12, rows of 144 bytes
        (torch.float32, torch.float32, 2, 8, 2, 100, 16, 60, 8, True),  # rows of 400 bytes: 25 lanes of 16 bytes
        (torch.bfloat16, torch.bfloat16, 2, 4, 2, 100, 16, 60, 8, True),  # rows of 200 bytes: 2 elements per lane
        (torch.bfloat16, torch.float32, 1, 16, 8, 520, 16, 50, 6, True),  # 9 elements per lane, last lane short
        (torch.bfloat16, torch.bfloat16, 2, 64, 16, 128, 64, 200, 12, True),  # 128 lanes per page: general kernel
        (torch.float32, torch.float32, 1, 64, 64, 256, 4, 20, 4, True),  # 2048 lanes per page: KV heads in passes
        (torch.bfloat16, torch.bfloat16, 1, 8, 2, 64, 2, 20000, 100, True),  # beyond 16384 pages
    ],
)
def test_quest_select_bit_exact(gpu, dtype, q_dtype, B, Hq, Hkv, D, P, n_pages, top, keep_sink):
    log_case(test="quest", dtype=dtype, B=B, Hq=Hq, Hkv=Hkv, D=D, P=P, n_pages=n_pages, top=top)
    g = torch.Generator().manual_seed(n_pages + B)
    q = torch.randn(B, Hq, D, generator=g).to(q_dtype)
    mn, mx = _bounds(g, B, n_pages, Hkv, D, dtype, offsets=True)
    lengths = torch.randint(1, n_pages * P + 1, (B,), generator=g)
    lengths[0] = n_pages * P  # full
    if B > 1:
        lengths[1] = min(int(lengths[1]), top * P - 3)  # fewer pages than the budget
    e_scores, e_pages, e_pos = oracle.quest_select(q, mn, mx, lengths, P, top, keep_sink)
    pages, pos, scores = rk.quest_batched(q.to(gpu), mn.to(gpu), mx.to(gpu), lengths.to(gpu), P, top, keep_sink)
    pages, pos, scores = pages.cpu(), pos.cpu(), scores.cpu()
    assert torch.equal(pages, e_pages)
    assert torch.equal(pos, e_pos)
    for b in range(B):
        count = -(-int(lengths[b]) // P)
        if top < count:
            assert torch.equal(scores[b, :count].view(torch.int32), e_scores[b, :count].view(torch.int32))


@pytest.mark.parametrize(
    "dtype,Hq,Hkv,D,nan_pages,top,inf_query",
    [
        (torch.bfloat16, 32, 8, 128, 0, 8, False),  # page kernel, group 4
        (torch.bfloat16, 32, 8, 128, 3, 8, False),  # NaN pages below the budget
        (torch.bfloat16, 28, 4, 128, 8, 8, False),  # group 7: NaN pages fill the budget
        (torch.bfloat16, 28, 4, 128, 3, 8, True),  # group 7 (half-wave fold), an infinite query
        (torch.float32, 12, 4, 64, 3, 6, True),  # fp32, half-wave fold
        (torch.bfloat16, 8, 2, 64, 11, 8, False),  # more NaN pages than slots
        (torch.float32, 8, 2, 64, 3, 6, False),  # fp32 page kernel
        (torch.float16, 6, 2, 128, 3, 6, False),  # fp16, group 3
        (torch.bfloat16, 12, 1, 72, 4, 10, False),  # group 12, general kernel
        (torch.bfloat16, 64, 16, 128, 4, 10, False),  # general kernel, 16-byte loads
        (torch.bfloat16, 32, 8, 128, 4, 4, True),  # an infinite query
        (torch.bfloat16, 32, 8, 128, 4, 8, True),
    ],
)
def test_quest_special_values_match_oracle_and_reference(gpu, dtype, Hq, Hkv, D, nan_pages, top, inf_query):
    """Zero and infinite queries; +-inf, NaN, zero and inverted bounds; NaN
    pages below, at and above the budget. Every score (NaN as 0x7fc00000)
    and every page equals the oracle's, and the pages are a top-k of the
    reference formula's ranking (torch.maximum scores, forced pages at +inf,
    NaN above them: selection.py:82-90), the same set wherever that ranking
    has no tie at the k-th key."""
    from quest_reference import check_page_set, reference_ranked, special_case

    log_case(test="quest-special", dtype=dtype, Hq=Hq, Hkv=Hkv, D=D, nan_pages=nan_pages, top=top, inf=inf_query)
    n_pages, P, B = 40, 16, 6
    cases = [special_case(100 * s + Hq + D, Hq, Hkv, D, n_pages, nan_pages, inf_query, dtype) for s in range(B)]
    q = torch.stack([c[0] for c in cases])
    mn = torch.stack([c[1] for c in cases])
    mx = torch.stack([c[2] for c in cases])
    lengths = torch.full((B,), n_pages * P - 5)
    e_scores, e_pages, e_pos = oracle.quest_select(q, mn, mx, lengths, P, top)
    pages, pos, scores = rk.quest_batched(q.to(gpu), mn.to(gpu), mx.to(gpu), lengths.to(gpu), P, top)
    scores = scores.cpu()
    assert torch.equal(scores.view(torch.int32), e_scores.view(torch.int32))
    assert torch.equal(pages.cpu(), e_pages)
    assert torch.equal(pos.cpu(), e_pos)
    for b, (qb, lob, hib, nan_set) in enumerate(cases):
        assert {p for p in range(n_pages) if torch.isnan(scores[b, p])} == nan_set
        check_page_set(pages[b].cpu(), reference_ranked(qb, lob, hib, int(lengths[b]), P, top), top)


@pytest.mark.gpu
@pytest.mark.parametrize("n_pages,top,P,nan_pages", [(1500, 64, 16, 0), (3000, 200, 16, 3), (4096, 256, 8, 0),
                                                     (2100, 1, 16, 5), (1800, 33, 16, 40), (1025, 17, 4, 2)])
def test_quest_select_ties_beyond_one_wave(gpu, n_pages, top, P, nan_pages):
    """Beyond 1024 pages (the four-wave selector up to 4096): each request's
    pages repeat six distinct bound rows, so pages tie in large groups across
    all four waves, and request 2 holds NaN pages (tied above every number,
    more of them than the budget in some cases). Pages, positions and scores
    equal the oracle's: ties go to the lowest pages."""
    log_case(test="quest-ties", n_pages=n_pages, top=top, P=P, nan_pages=nan_pages)
    B, Hq, Hkv, D = 3, 8, 2, 64
    g = torch.Generator().manual_seed(n_pages * 3 + top)
    q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16)
    lo6, hi6 = _bounds(g, B, 6, Hkv, D, torch.bfloat16, offsets=True)
    idx = torch.randint(0, 6, (B, n_pages), generator=g)
    mn = torch.stack([lo6[b, idx[b]] for b in range(B)])
    mx = torch.stack([hi6[b, idx[b]] for b in range(B)])
    for p in (torch.randperm(n_pages - 2, generator=g)[:nan_pages] + 1).tolist():
        mx[2, p, 0, 5] = float("nan")
    lengths = torch.tensor([n_pages * P, (n_pages - 300) * P - 1, n_pages * P - 3])
    e_scores, e_pages, e_pos = oracle.quest_select(q, mn, mx, lengths, P, top, True)
    pages, pos, scores = rk.quest_batched(q.to(gpu), mn.to(gpu), mx.to(gpu), lengths.to(gpu), P, top, True)
    assert torch.equal(pages.cpu(), e_pages)
    assert torch.equal(pos.cpu(), e_pos)
    for b in range(B):
        count = -(-int(lengths[b]) // P)
        assert torch.equal(scores.cpu()[b, :count].view(torch.int32), e_scores[b, :count].view(torch.int32))


@pytest.mark.parametrize("B,Hq,Hkv,D,P,n_pages,top", [(4, 32, 8, 128, 64, 512, 32), (3, 4, 2, 8, 4, 20, 1),
                                                      (2, 4, 2, 8, 4, 20, 2), (2, 6, 3, 24, 5, 33, 7),
                                                      (2, 4, 2, 16, 8, 700, 50),
                                                      (2, 4, 2, 16, 8, 2500, 100),  # four-wave select
                                                      (2, 4, 2, 16, 8, 1100, 256),
                                                      (2, 24, 2, 100, 16, 60, 8),  # GQA 12, 25 lanes of 16 bytes
                                                      (2, 8, 2, 300, 16, 40, 6),  # 5 elements per lane
                                                      (1, 8, 2, 16, 2, 20000, 64)])  # beyond 16384 pages
def test_mean_select_bit_exact(gpu, B, Hq, Hkv, D, P, n_pages, top):
    log_case(test="mean", B=B, Hq=Hq, D=D, n_pages=n_pages, top=top)
    g = torch.Generator().manual_seed(5 + n_pages)
    q = torch.randn(B, Hq, D, generator=g)
    summ = torch.randn(B, n_pages, Hkv, D, generator=g)
    lengths = torch.randint(1, n_pages * P + 1, (B,), generator=g)
    e_scores, e_pages, e_pos = oracle.mean_select(q, summ, lengths, P, top)
    pages, pos, scores = rk.mean_batched(q.to(gpu), summ.to(gpu), lengths.to(gpu), P, top)
    assert torch.equal(pages.cpu(), e_pages)
    assert torch.equal(pos.cpu(), e_pos)


@pytest.mark.gpu
@pytest.mark.parametrize("top", [1, 2, 3, 6, 29])
def test_mean_select_nan_summaries_match_oracle_and_reference(gpu, top):
    """NaN page summaries (below, at and above the budget) and NaN summaries
    on the required first and last pages: pages, positions and every score
    (NaN as 0x7fc00000) equal the oracle's, and the pages are the reference
    page-mean choice (selection.py:131-145 with torch ops), tie-aware."""
    from quest_reference import check_mean_pages

    log_case(test="mean-nan", top=top)
    B, Hq, Hkv, D, P, n_pages = 4, 8, 2, 16, 4, 30
    g = torch.Generator().manual_seed(40 + top)
    q = torch.randn(B, Hq, D, generator=g)
    summ = torch.randn(B, n_pages, Hkv, D, generator=g)
    for b, n_nan in enumerate((0, 3, 9, 27)):
        for p in (torch.randperm(n_pages - 2, generator=g)[:n_nan] + 1).tolist():
            summ[b, p, p % Hkv, p % D] = math.nan
    summ[2, 0, 0, 1] = math.nan  # required pages: kept whatever their summary
    summ[2, n_pages - 1, 1, 3] = math.nan
    lengths = torch.tensor([n_pages * P, n_pages * P - 3, n_pages * P - 1, 20 * P + 2])
    e_scores, e_pages, e_pos = oracle.mean_select(q, summ, lengths, P, top)
    pages, pos, scores = rk.mean_batched(q.to(gpu), summ.to(gpu), lengths.to(gpu), P, top)
    pages, pos, scores = pages.cpu(), pos.cpu(), scores.cpu()
    assert torch.equal(pages, e_pages)
    assert torch.equal(pos, e_pos)
    for b in range(B):
        count = -(-int(lengths[b]) // P)
        if top < count:
            assert torch.equal(scores[b, :count].view(torch.int32), e_scores[b, :count].view(torch.int32))
        check_mean_pages(pages[b], q[b], summ[b], int(lengths[b]), P, top)


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["quest", "mean"])
def test_scores_are_kept_when_every_page_is_selected(gpu, mode):
    """top_pages >= max_pages keeps every page; the scores output still holds
    every page's score, bit-identical to the oracle's (computed there with a
    smaller budget: the scores do not depend on it)."""
    log_case(test="scores-all-pages", mode=mode)
    B, Hq, Hkv, D, P, n_pages = 2, 8, 2, 64, 16, 12
    g = torch.Generator().manual_seed(7)
    q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16)
    lengths = torch.tensor([n_pages * P, n_pages * P - 9])
    if mode == "quest":
        mn, mx = _bounds(g, B, n_pages, Hkv, D, torch.bfloat16, offsets=True)
        e_scores, _, _ = oracle.quest_select(q, mn, mx, lengths, P, 1)
        run = lambda top, select: rk.quest_batched(q.to(gpu), mn.to(gpu), mx.to(gpu), lengths.to(gpu), P, top,
                                                   select=select)
    else:
        summ = torch.randn(B, n_pages, Hkv, D, generator=g)
        e_scores, _, _ = oracle.mean_select(q, summ, lengths, P, 1)
        run = lambda top, select: rk.mean_batched(q.to(gpu), summ.to(gpu), lengths.to(gpu), P, top, select=select)
    for top in (n_pages, n_pages + 5):
        for select in (True, False):
            pages, _, scores = run(top, select)
            for b in range(B):
                count = -(-int(lengths[b]) // P)
                assert torch.equal(scores.cpu()[b, :count].view(torch.int32), e_scores[b, :count].view(torch.int32))
                if select:
                    assert pages.cpu()[b].tolist() == list(range(count)) + [-1] * (top - count)


# ---- append ---------------------------------------------------------------------------


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,P,Hkv,D", [(torch.bfloat16, 64, 8, 128), (torch.float16, 16, 2, 24),
                                           (torch.float32, 7, 1, 8)])
def test_append_page_matches_oracle(gpu, dtype, P, Hkv, D):
    log_case(test="append", dtype=str(dtype), P=P, Hkv=Hkv, D=D)
    g = torch.Generator().manual_seed(P * 100 + D)
    blocks, host_pages = 3, 5
    pool = torch.randn(blocks, 2, P, Hkv, D, generator=g).to(dtype)
    host = torch.empty(host_pages, 2, P, Hkv, D, dtype=dtype, pin_memory=True)
    host.copy_(torch.randn(host.shape, generator=g).to(dtype))
    host_before = host.clone()
    dpool = pool.to(gpu)
    alias = rk.MappedHost(host)
    block, host_page = 1, 3
    summary = torch.zeros(Hkv, D, device=gpu)
    lo = torch.full((Hkv, D), float("inf"), device=gpu).to(dtype)
    hi = torch.full((Hkv, D), float("-inf"), device=gpu).to(dtype)
    e_summary = torch.zeros(Hkv, D)
    e_lo = torch.full((Hkv, D), float("inf"))
    e_hi = torch.full((Hkv, D), float("-inf"))
    keys = torch.randn(P, Hkv, D, generator=g).to(dtype)
    vals = torch.randn(P, Hkv, D, generator=g).to(dtype)
    within = 0
    for count in (1, 2, P // 3 or 1, 1, P):  # appends until the page is full
        count = min(count, P - within)
        if count == 0:
            break
        rk.append_page(keys[within : within + count].to(gpu), vals[within : within + count].to(gpu), dpool, block,
                       within, alias, host_page, summary, lo, hi)
        oracle.append_bounds(keys, within, count, e_summary, e_lo, e_hi)
        pool[block, 0, within : within + count] = keys[within : within + count]
        pool[block, 1, within : within + count] = vals[within : within + count]
        within += count
        torch.cuda.synchronize()
        assert torch.equal(dpool.cpu().view(torch.uint8), pool.view(torch.uint8))
        for plane, src in ((0, keys), (1, vals)):
            assert torch.equal(host[host_page, plane, :within].view(torch.uint8), src[:within].view(torch.uint8))
        assert torch.equal(summary.cpu(), e_summary)  # double sum in row order, rounded once
        assert torch.equal(lo.float().cpu(), e_lo) and torch.equal(hi.float().cpu(), e_hi)
    others = [i for i in range(host_pages) if i != host_page]
    assert torch.equal(host[others].view(torch.uint8), host_before[others].view(torch.uint8))
