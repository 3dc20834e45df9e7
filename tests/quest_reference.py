"""The reference's Quest and page-mean page choices, evaluated with torch
operations, and a tie-aware comparison of page sets against them.

reference_scores() evaluates nano_hisparse/selection.py:82-85 as written
there (torch.maximum of the two products per query head, summed over the
head dimension, averaged over heads), in float64 so that finite scores carry
no fp32 rounding; 0 * inf, NaN and opposite infinities behave as in float32.
reference_ranked() applies selection.py:86-89 (forced pages set to +inf).
torch.topk ranks NaN above every number (aten's CPU comparator tests isnan
before >), so check_page_set() orders NaN > +inf > finite > -inf.

mean_reference_ranked() evaluates the page-mean selector,
nano_hisparse/selection.py:131-143: the early returns (every page when
top_k >= count; the required pages alone when top_k equals their number),
the required pages ([count - 1] for top_k == 1, else [0, count - 1]), the
group-mean query in float32 as written there, its dot products with the
summaries in float64, and the required pages set to -inf before
torch.topk; check_mean_pages() applies check_page_set() to the pages chosen
beside the required ones.

Where the k-th and (k+1)-th reference keys tie (equal class, or finite
scores closer than `tol`), torch's choice inside the tie is not defined by
the formula (std::nth_element / partial_sort are unstable): the check then
only requires every page strictly above the tie and the rest from the tie.
"""

from __future__ import annotations

import math

import torch


def quest_count(length, page_size):
    return -(-int(length) // int(page_size))


def reference_scores(q, lo, hi, count):
    """q [Hq, D]; lo, hi [pages, Hkv, D]: scores [count] in float64."""
    groups = q.shape[0] // lo.shape[1]
    low = lo[:count].double().repeat_interleave(groups, 1).transpose(0, 1)
    high = hi[:count].double().repeat_interleave(groups, 1).transpose(0, 1)
    qd = q.double()[:, None]
    return torch.maximum(qd * low, qd * high).sum(-1).mean(0)


def reference_ranked(q, lo, hi, length, page_size, top_pages, keep_sink=True):
    """The reference's ranked values: scores with the forced pages at +inf."""
    count = quest_count(length, page_size)
    scores = reference_scores(q, lo, hi, count)
    required = [count - 1]
    if keep_sink and top_pages > 1 and count > 1:
        required.append(0)
    scores[required] = math.inf
    return scores


def _key(v, tol):
    if math.isnan(v):
        return (3, 0.0)
    if math.isinf(v):
        return (2, 0.0) if v > 0 else (0, 0.0)
    return (1, v)


def _same(a, b, tol):
    return a[0] == b[0] and abs(a[1] - b[1]) <= tol * (1.0 + abs(a[1]))


def check_page_set(got, ranked, top_pages, tol=1e-5):
    """Asserts that `got` (page ids) is a top-k of `ranked` under the
    reference's order; returns True when that top-k is unique."""
    values = ranked.tolist()
    count = len(values)
    got = sorted(int(p) for p in got if int(p) >= 0)
    if top_pages >= count:
        assert got == list(range(count))
        return True
    keys = [_key(v, tol) for v in values]
    order = sorted(range(count), key=lambda p: keys[p], reverse=True)
    kth = keys[order[top_pages - 1]]
    tie = {p for p in range(count) if _same(keys[p], kth, tol)}
    above = {p for p in range(count) if p not in tie and keys[p] > kth}
    assert len(got) == top_pages, (got, top_pages)
    assert above <= set(got), sorted(above - set(got))
    assert set(got) <= above | tie, sorted(set(got) - above - tie)
    return len(above) + len(tie) == top_pages


def check_score_classes(scores, reference, tol=1e-4):
    """Per page: NaN where the reference is NaN, the same infinity, or a
    finite score within tol (relative) of the float64 reference."""
    for p, (s, r) in enumerate(zip(scores.tolist(), reference.tolist())):
        if math.isnan(r):
            assert math.isnan(s), (p, s, r)
        elif math.isinf(r):
            assert s == r, (p, s, r)
        else:
            assert math.isfinite(s) and abs(s - r) <= tol * (1.0 + abs(r)), (p, s, r)


def special_case(seed, Hq, Hkv, D, n_pages, nan_pages, inf_query=False, dtype=torch.bfloat16):
    """One request's query [Hq, D] and bounds [n_pages, Hkv, D] holding the
    special values the reference's formula gives meaning to.

    Always: +-0 queries, +-inf bounds that no product turns into NaN
    (natural +-inf scores), zero bounds, inverted bounds (lo > hi) and
    `nan_pages` NaN pages made by a NaN bound or by a zero query against an
    infinite bound. With inf_query, one head's query is +inf at one dim, so
    every page scores +inf, -inf (both bounds negative there) or NaN (a zero
    bound there); a third of the NaN pages are made that way."""
    assert D >= 6 and n_pages >= nan_pages + 8
    g = torch.Generator().manual_seed(seed)
    G = Hq // Hkv
    q = torch.randn(Hq, D, generator=g)
    a, c = torch.randn(2, n_pages, Hkv, D, generator=g)
    mu = torch.randn(n_pages, 1, 1, generator=g)
    lo, hi = torch.minimum(a, c) + mu, torch.maximum(a, c) + mu
    q[q == 0] = 0.5
    q[0, 1], q[G - 1, 2] = 0.0, -0.0  # zero queries at dims 1 and 2 of KV head 0's group
    kq = Hkv - 1  # the KV head whose group holds the infinite query (dim 3)
    if inf_query:
        q[kq * G, 3] = math.inf
        neg = torch.rand(n_pages, generator=g) < 0.3
        mag = hi[:, kq, 3].abs() + 0.5
        hi[:, kq, 3] = torch.where(neg, -mag, mag)
        lo[:, kq, 3] = torch.where(neg, -mag - 0.25, mag - 0.25)
    pages = (torch.randperm(n_pages - 2, generator=g)[: nan_pages + 6] + 1).tolist()  # never a forced page
    nan_set, extra = pages[:nan_pages], pages[nan_pages:]
    for i, p in enumerate(nan_set):
        kind = i % 3 if inf_query else i % 2
        if kind == 0:
            hi[p, i % Hkv, 5] = math.nan
        elif kind == 1:
            hi[p, 0, 1] = math.inf  # against the +0 query at dim 1
        else:
            lo[p, kq, 3] = 0.0  # against the +inf query at dim 3
    p_inf, p_ninf, p_inv, p_zero = extra[:4]
    # KV head 0, dim 0: every head of its group has a finite nonzero query
    qs = q[0:G, 0]
    if (qs > 0).all():
        hi[p_inf, 0, 0] = math.inf  # all heads read hi: +inf
        lo[p_ninf, 0, 0] = hi[p_ninf, 0, 0] = -math.inf  # -inf
    elif (qs < 0).all():
        lo[p_inf, 0, 0] = -math.inf  # all heads read lo: +inf
        lo[p_ninf, 0, 0] = hi[p_ninf, 0, 0] = math.inf  # -inf
    else:
        lo[p_inf, 0, 0], hi[p_inf, 0, 0] = -math.inf, math.inf  # +inf either way
        hi[p_ninf, 0, 0] = math.inf  # mixed signs allow no -inf: +inf from the positive heads
    if inf_query:  # the infinite query's term takes the natural infinity's sign (else +inf + -inf = NaN)
        ninf_sign = -1.0 if ((qs > 0).all() or (qs < 0).all()) else 1.0
        for p, sign in ((p_inf, 1.0), (p_ninf, ninf_sign)):
            m = hi[p, kq, 3].abs() + 0.5
            hi[p, kq, 3], lo[p, kq, 3] = sign * m, sign * m - 0.25
    lo[p_inv], hi[p_inv] = hi[p_inv] + 0.5, lo[p_inv].clone()  # lo > hi everywhere
    lo[p_zero], hi[p_zero] = 0.0, -0.0
    if inf_query:  # a zero bound against the infinite query would make p_zero NaN
        lo[p_zero, kq, 3], hi[p_zero, kq, 3] = 1.0, 2.0
    return q.to(dtype), lo.to(dtype), hi.to(dtype), set(nan_set)


def mean_reference_ranked(q, summaries, length, page_size, top_k):
    """q [Hq, D]; summaries [pages, Hkv, D]. Returns (pages, None) for the
    early returns of selection.py:131-137, else (required, ranked): the
    scores [count] in float64 with the required pages at -inf
    (selection.py:138-143)."""
    count = quest_count(length, page_size)
    if top_k >= count:
        return list(range(count)), None
    required = [count - 1] if top_k == 1 else [0, count - 1]
    if top_k == len(required):
        return sorted(required), None
    kv_heads = summaries.shape[1]
    grouped = q.float().reshape(kv_heads, q.shape[0] // kv_heads, -1).mean(1)
    scores = torch.einsum("hd,phd->p", grouped.double(), summaries[:count].double())
    scores[required] = -math.inf
    return required, scores


def check_mean_pages(got, q, summaries, length, page_size, top_k, tol=1e-5):
    """Asserts that `got` is the reference's page-mean choice: the required
    pages plus a top-(top_k - len(required)) of the reference scores,
    tie-aware; returns True when that choice is unique."""
    required, ranked = mean_reference_ranked(q, summaries, length, page_size, top_k)
    got = sorted(int(p) for p in got if int(p) >= 0)
    if ranked is None:
        assert got == required, (got, required)
        return True
    assert set(required) <= set(got), (got, required)
    chosen = [p for p in got if p not in required]
    return check_page_set(chosen, ranked, top_k - len(required), tol)
