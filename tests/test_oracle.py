"""The CPU oracle pinned against the reference's known answers, independent
formulations and closed forms (no GPU needed), plus the C ABI export check.

The reference's own known answers (tests/test_selection.py:18-50, paths
relative to the reference repository) are checked from the fixture
tests/golden/reference_kats.json by test_golden.py.
"""

import ctypes

import numpy as np
import math

import pytest
import torch

import oracle


def test_library_exports_every_header_symbol():
    from nano_hisparse import _hip

    lib = ctypes.CDLL(_hip.LIB_PATH)  # loads without a GPU; nothing is called
    symbols = _hip.header_symbols()
    assert len(symbols) >= 10
    missing = [s for s in symbols if not hasattr(lib, s)]
    assert not missing, missing
    assert set(symbols) == set(_hip.SIGNATURES)


# ---- resolver ----------------------------------------------------------------------


def _random_item(rng, n_pages, P, H):
    host_pages = 2 * n_pages + 3
    source = rng.permutation(host_pages)[:n_pages].astype(np.int64)
    source[rng.random(n_pages) < 0.1] = -1  # pages without host backing
    resident = np.where(rng.random(n_pages) < 0.3, rng.permutation(n_pages) + 50, -1).astype(np.int64)
    hot = rng.permutation(40)[: -(-H // P)].astype(np.int64)
    rows = (np.arange(host_pages)[:, None] * P + np.arange(P)).ravel()
    tags = np.full(H, -1, np.int64)
    k = int(rng.integers(0, min(H, rows.size) + 1))
    tags[rng.permutation(H)[:k]] = rng.choice(rows, size=k, replace=False)
    return source, resident, hot, tags, rng.permutation(H).astype(np.int64)


@pytest.mark.parametrize("seed", range(40))
def test_resolver_c_restatement_equals_bruteforce_simulation(seed):
    rng = np.random.default_rng(seed)
    P = int(rng.integers(1, 6))
    n_pages = int(rng.integers(1, 12))
    H = int(rng.integers(1, 24))
    source, resident, hot, tags, lru = _random_item(rng, n_pages, P, H)
    t_list, l_list = tags.tolist(), lru.tolist()
    for _ in range(4):
        length = int(rng.integers(0, n_pages * P + 1))
        n = int(rng.integers(1, H + 1))  # the cache admits at most H distinct rows
        raw = rng.integers(-2, n_pages * P + 3, size=n)
        got = oracle.resolve_rows(raw, source, resident, hot, tags, lru, length, P)
        want = oracle.resolve_rows_bruteforce(raw, source, resident, hot, t_list, l_list, length, P)
        for g, w in zip(got, want):
            assert g.tolist() == list(w)
        assert tags.tolist() == t_list and lru.tolist() == l_list
        assert sorted(lru.tolist()) == list(range(H))
        assert int(got[3].sum()) == len({int(t) for t in raw if 0 <= t < length and source[min(t // P, n_pages - 1)] >= 0})


# ---- Quest ---------------------------------------------------------------------------


@pytest.mark.parametrize("dtype,D", [(torch.float32, 64), (torch.bfloat16, 128), (torch.float16, 24), (torch.float32, 3)])
def test_quest_scores_closed_form_on_small_integers(dtype, D):
    """Small-integer queries and bounds make every product and partial sum
    exact in fp32, so any summation order gives the float64 value."""
    g = torch.Generator().manual_seed(D)
    B, Hq, Hkv, n_pages, P = 2, 8, 2, 30, 4
    q = torch.randint(-8, 9, (B, Hq, D), generator=g).float()
    a = torch.randint(-8, 9, (B, n_pages, Hkv, D), generator=g).float()
    c = torch.randint(-8, 9, (B, n_pages, Hkv, D), generator=g).float()
    mn, mx = torch.minimum(a, c).to(dtype), torch.maximum(a, c).to(dtype)
    scores, pages, _ = oracle.quest_select(q.to(dtype), mn, mx, [n_pages * P] * B, P, 5)
    qe = q.double().repeat_interleave(1, 1)
    kmin = mn.double().repeat_interleave(Hq // Hkv, 2)
    kmax = mx.double().repeat_interleave(Hq // Hkv, 2)
    exact = torch.maximum(qe[:, None] * kmin, qe[:, None] * kmax).sum(-1).mean(-1)
    assert torch.equal(scores.double(), exact)
    for b in range(B):  # top-5 with page 0 and the last page forced, ties to the lower page
        rest = sorted(range(1, n_pages - 1), key=lambda p: (-exact[b, p].item(), p))[:3]
        assert pages[b].tolist() == sorted([0, n_pages - 1, *rest])


def test_quest_pages_agree_with_float64_scores_outside_ties():
    g = torch.Generator().manual_seed(3)
    B, Hq, Hkv, D, n_pages, P, top = 4, 32, 8, 128, 256, 64, 32
    q = torch.randn(B, Hq, D, generator=g).bfloat16()
    a, c = torch.randn(2, B, n_pages, Hkv, D, generator=g)
    mn, mx = torch.minimum(a, c).bfloat16(), torch.maximum(a, c).bfloat16()
    scores, pages, _ = oracle.quest_select(q, mn, mx, [n_pages * P] * B, P, top)
    qe = q.double()
    kmin, kmax = mn.double().repeat_interleave(4, 2), mx.double().repeat_interleave(4, 2)
    exact = torch.maximum(qe[:, None] * kmin, qe[:, None] * kmax).sum(-1).mean(-1)
    assert (scores.double() - exact).abs().max() < 1e-4
    for b in range(B):
        ex = exact[b].clone()
        ex[0] = ex[-1] = float("inf")
        want = set(ex.topk(top).indices.tolist())
        got = set(pages[b].tolist())
        kth = ex.topk(top).values[-1].item()
        for p in got ^ want:  # any disagreement must be a near-tie at the k-th score
            assert abs(ex[p].item() - kth) < 1e-4


@pytest.mark.parametrize("Hq,Hkv,D,nan_pages,top,inf_query,unique_set", [
    (32, 8, 128, 0, 8, False, True),    # no NaN page
    (32, 8, 128, 3, 8, False, True),    # NaN pages below the budget: forced pages kept
    (28, 4, 128, 8, 8, False, True),    # NaN pages fill the budget: forced pages dropped
    (8, 2, 64, 11, 8, False, False),    # more NaN pages than slots (ties among NaN)
    (6, 2, 24, 5, 9, False, True),      # group 3, rows of 48 bytes (16-byte chunks)
    (12, 1, 72, 4, 10, False, True),    # group 12 (one KV head), head_dim 72
    (32, 8, 128, 4, 4, True, True),     # an infinite query: +-inf and NaN pages only
    (32, 8, 128, 4, 8, True, False),    # ... with slots left inside the +inf tie
])
def test_quest_special_values_match_the_reference_formula(Hq, Hkv, D, nan_pages, top, inf_query, unique_set):
    """Zero and infinite queries, +-inf / NaN / zero / inverted bounds: the
    oracle's scores are NaN, +-inf or finite exactly where the reference's
    torch.maximum formula (evaluated with torch ops, selection.py:82-85) is,
    and its pages are a top-k of the reference's ranking (NaN above the
    forced +inf pages, selection.py:86-90); unique wherever that ranking has
    no tie at the k-th key."""
    from quest_reference import check_page_set, check_score_classes, reference_ranked, reference_scores, special_case

    n_pages, P = 40, 16
    unique = 0
    for seed in range(6):
        q, lo, hi, nan_set = special_case(100 * seed + Hq + D, Hq, Hkv, D, n_pages, nan_pages, inf_query)
        length = n_pages * P - 5
        scores, pages, _ = oracle.quest_select(q[None], lo[None], hi[None], [length], P, top)
        ref = reference_scores(q, lo, hi, n_pages)
        assert {p for p in range(n_pages) if math.isnan(ref[p])} == nan_set
        check_score_classes(scores[0, :n_pages], ref)
        assert all(scores[0, p].view(torch.int32).item() == 0x7FC00000 for p in nan_set)
        ranked = reference_ranked(q, lo, hi, length, P, top)
        unique += check_page_set(pages[0], ranked, top)
        if nan_pages >= top:  # NaN outranks the forced pages: they are dropped
            assert set(pages[0].tolist()) <= nan_set
        if nan_pages > top and not inf_query:  # inside the NaN tie: the lowest pages
            assert pages[0].tolist() == sorted(nan_set)[:top]
    if unique_set:  # the reference's page set is unique for these inputs, and equal
        assert unique == 6


def test_quest_forced_pages_rank_below_nan_and_above_inf():
    """Ranking alone: NaN > forced (+inf) > natural +inf > finite, lowest page
    first inside a class: the sink before the last page (all three +inf in
    the reference, where torch.topk's pick among them is unspecified)."""
    Hq, Hkv, D, P, n_pages = 2, 1, 8, 4, 10
    q = torch.ones(Hq, D)
    lo = torch.zeros(n_pages, Hkv, D)
    hi = torch.arange(n_pages, dtype=torch.float32)[:, None, None].expand(n_pages, Hkv, D).clone()
    hi[3, 0, 2] = math.nan
    hi[6, 0, 4] = math.nan
    hi[5, 0, 0] = math.inf  # natural +inf
    for top, want in ((2, [3, 6]), (3, [0, 3, 6]), (4, [0, 3, 6, 9]), (5, [0, 3, 5, 6, 9]), (6, [0, 3, 5, 6, 8, 9])):
        _, pages, _ = oracle.quest_select(q[None], lo[None], hi[None], [n_pages * P], P, top)
        assert pages[0].tolist() == want, (top, pages[0].tolist())


def test_mean_select_forces_first_and_last_page():
    g = torch.Generator().manual_seed(9)
    q = torch.randn(1, 4, 8, generator=g)
    summ = torch.randn(1, 10, 2, 8, generator=g)
    for top in (1, 2, 3, 6):
        scores, pages, _ = oracle.mean_select(q, summ, [40], 4, top)
        gq = q[0].view(2, 2, 8).double().mean(1)
        exact = torch.einsum("hd,phd->p", gq, summ[0].double())
        required = [9] if top == 1 else [0, 9]
        rest = sorted((p for p in range(10) if p not in required), key=lambda p: (-exact[p].item(), p))
        want = sorted(required + rest[: top - len(required)])
        assert pages[0].tolist() == want


def _mean_case(seed, n_pages=30, Hq=8, Hkv=2, D=16, nan_pages=0, nan_required=False, tie_groups=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(Hq, D, generator=g)
    summ = torch.randn(n_pages, Hkv, D, generator=g)
    if tie_groups:  # pages that repeat a few summary rows tie exactly
        idx = torch.randint(0, tie_groups, (n_pages,), generator=g)
        summ = summ[idx].clone()
    for p in (torch.randperm(n_pages - 2, generator=g)[:nan_pages] + 1).tolist():
        summ[p, p % Hkv, p % D] = math.nan
    if nan_required:  # the reference sets the required pages to -inf whatever their summary
        summ[0, 0, 1] = math.nan
        summ[n_pages - 1, Hkv - 1, 3] = math.nan
    return q, summ


@pytest.mark.parametrize("seed,nan_pages,nan_required,tie_groups",
                         [(0, 0, False, 0), (1, 3, False, 0), (2, 9, True, 0), (3, 0, True, 4), (4, 27, False, 0),
                          (5, 5, True, 3)])
def test_mean_select_matches_the_reference_formula_tie_aware(seed, nan_pages, nan_required, tie_groups):
    """oracle.mean_select against the reference's page-mean selector
    (selection.py:131-145) evaluated with torch ops (quest_reference): budgets
    1 and 2 (the required pages alone), 3 .. count - 1, and >= count (every
    page); NaN summaries below, at and above the budget (torch.topk ranks
    NaN above every number), required pages whose own summary is NaN (set to
    -inf, still kept), and exact ties between repeated summary rows. The
    chosen pages beside the required ones must be a top-k of the reference
    scores, with any choice inside a tie at the k-th rank accepted."""
    from quest_reference import check_mean_pages

    n_pages, P = 30, 4
    q, summ = _mean_case(seed, n_pages, nan_pages=nan_pages, nan_required=nan_required, tie_groups=tie_groups)
    for length in (n_pages * P, n_pages * P - 3, 9 * P + 1):
        count = -(-length // P)
        for top in (1, 2, 3, 5, 8, count - 1, count, count + 4):
            _, pages, positions = oracle.mean_select(q[None], summ[None], [length], P, top)
            got = [p for p in pages[0].tolist() if p >= 0]
            assert len(got) == min(top, count), (length, top, got)
            check_mean_pages(got, q, summ, length, P, top)
            want_pos = [t for p in got for t in range(p * P, min((p + 1) * P, length))]
            assert [t for t in positions[0].tolist() if t >= 0] == want_pos
    # a planted mistake in the oracle's output fails the check: a NaN page
    # dropped for the best finite one
    if nan_pages and not tie_groups:
        from quest_reference import mean_reference_ranked

        top = 3 + min(nan_pages, 3)
        _, pages, _ = oracle.mean_select(q[None], summ[None], [n_pages * P], P, top)
        required, ranked = mean_reference_ranked(q, summ, n_pages * P, P, top)
        nan_chosen = [p for p in pages[0].tolist() if p not in required and math.isnan(ranked[p])]
        assert nan_chosen
        finite = [p for p in range(n_pages) if p not in pages[0].tolist() and math.isfinite(ranked[p])]
        bad = sorted(set(pages[0].tolist()) - {nan_chosen[0]} | {max(finite, key=lambda p: ranked[p])})
        with pytest.raises(AssertionError):
            check_mean_pages(bad, q, summ, n_pages * P, P, top)


# ---- attention and gather ---------------------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_attention_c_restatement_matches_float64_numpy(dtype):
    g = torch.Generator().manual_seed(1)
    P, Hkv, D = 8, 2, 32
    pool = torch.randn(6, 2, P, Hkv, D, generator=g).to(dtype)
    q = torch.randn(3, 4, D, generator=g).to(dtype)
    rows = torch.randint(-1, 6 * P, (3, 20), generator=g)
    rows[2] = -1
    a = oracle.attend_rows(q, pool, rows, P)
    b = oracle.attend_rows_float64(q, pool, rows, P)
    assert np.abs(a.numpy() - b).max() < 1e-6
    assert not a[2].any()


def test_attention_single_row_and_uniform_keys_closed_forms():
    P, Hkv, D = 4, 1, 8
    pool = torch.randn(3, 2, P, Hkv, D)
    pool[:, 0] = 1.0  # identical keys: uniform weights -> mean of the values
    q = torch.randn(1, 2, D)
    rows = torch.tensor([[0, 5, 9, -1]])
    out = oracle.attend_rows(q, pool, rows, P)
    mean_v = torch.stack([pool[r // P, 1, r % P, 0] for r in (0, 5, 9)]).mean(0)
    torch.testing.assert_close(out[0, 0], mean_v, atol=1e-6, rtol=1e-6)
    out = oracle.attend_rows(q, pool, torch.tensor([[-1, 6, -1]]), P)
    torch.testing.assert_close(out[0, 1], pool[1, 1, 2, 0], atol=1e-6, rtol=1e-6)


def _reference_attention_torch(q, pool, rows, P):
    """The reference's CPU attention formula (attention.py:26-35) evaluated
    with torch's own float32 kernels: q [Hq, D], rows [Hq, N]."""
    Hq, D = q.shape
    Hkv = pool.shape[3]
    safe = rows.clamp(min=0)
    kv_head = (torch.arange(Hq) // (Hq // Hkv))[:, None]
    k = pool[safe // P, 0, safe % P, kv_head].float()
    v = torch.where((rows >= 0)[..., None], pool[safe // P, 1, safe % P, kv_head].float(), 0.0)
    scores = (k * q.float()[:, None]).sum(-1) * D**-0.5
    weights = scores.masked_fill(rows < 0, -torch.inf).softmax(-1).nan_to_num()
    return (weights[..., None] * v).sum(1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_float32_attention_follows_the_reference_cpu_arithmetic(dtype):
    """oracle_attend_rows_f32 (the CPU baseline's attention) against the
    reference formula run by torch in float32 and against the float64
    numpy softmax: within float32 rounding (1e-5), masked and fully masked
    heads included; dropping the scale or the max shift would fail it."""
    g = torch.Generator().manual_seed(3)
    P, Hkv, D, Hq, N = 8, 2, 64, 8, 300
    pool = (torch.randn(60, 2, P, Hkv, D, generator=g) * 2).to(dtype)
    q = torch.randn(2, Hq, D, generator=g).to(dtype)
    rows = torch.randint(-1, 60 * P, (2, Hq, N), generator=g)
    rows[1, 3] = -1  # a head with every row masked: 0
    out = oracle.attend_rows(q, pool, rows, P, arithmetic="float32")
    exact = oracle.attend_rows_float64(q, pool, rows, P)
    assert np.abs(out.numpy() - exact).max() < 1e-5
    assert not out[1, 3].any()
    for b in range(2):
        ref = _reference_attention_torch(q[b], pool, rows[b], P)
        torch.testing.assert_close(out[b], ref, atol=1e-5, rtol=1e-5)
    # a single valid row returns its V exactly (weight 1)
    one = torch.full((1, Hq, 5), -1, dtype=torch.int64)
    one[0, :, 2] = 17
    out1 = oracle.attend_rows(q[:1], pool, one, P, arithmetic="float32")
    for h in range(Hq):
        assert torch.equal(out1[0, h], pool[17 // P, 1, 17 % P, h // (Hq // Hkv)].float())


def test_gather_closed_form_matches_fancy_indexing():
    g = torch.Generator().manual_seed(2)
    P = 5
    host = torch.randn(9, 2, P, 2, 4, generator=g)
    pool = torch.zeros(4, 2, P, 2, 4)
    mh = torch.tensor([3, 44, 17, -1, -1])
    md = torch.tensor([0, 19, 7, -1, 2])
    oracle.gather_rows(host, pool, mh, md, P)
    expected = torch.zeros_like(pool)
    for h, d in ((3, 0), (44, 19), (17, 7)):
        expected[d // P, :, d % P] = host[h // P, :, h % P]
    assert torch.equal(pool, expected)


# ---- bounds producer -------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_append_bounds_are_exact_min_max_and_rounded_mean(dtype):
    """storage.py:302-309: the page summary is the fp32 mean of the valid
    keys; minimum/maximum fold the new keys into the old bounds exactly."""
    g = torch.Generator().manual_seed(12)
    P, Hkv, D = 16, 2, 8
    keys = torch.randn(P, Hkv, D, generator=g).to(dtype)
    summary = torch.zeros(Hkv, D)
    lo = torch.full((Hkv, D), float("inf"))
    hi = torch.full((Hkv, D), float("-inf"))
    valid = 0
    for count in (5, 1, 7):  # appends of 5, 1 and 7 tokens into one page
        oracle.append_bounds(keys, valid, count, summary, lo, hi)
        valid += count
        seen = keys[:valid].double()
        assert torch.equal(lo, keys[:valid].float().amin(0))
        assert torch.equal(hi, keys[:valid].float().amax(0))
        mean = seen.mean(0)
        assert torch.allclose(summary.double(), mean, rtol=2 ** -23, atol=1e-12)
