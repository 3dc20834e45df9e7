"""Writes the committed golden fixtures of this directory.

reference_kats.json: the known answers of the reference's own tests, as data
(inputs and expected outputs, paths relative to the reference repository):
  - tests/test_selection.py:18-33  Quest selection (a page whose mean cancels;
    one shared budget across heads);
  - tests/test_selection.py:36-50  resolve_rows (late hits protected,
    duplicates, fragmented blocks), plus the LRU post-state derived by hand
    from row_index.py:121-138 (the reference test checks tags only);
  - tests/test_trace.py:18-56      row-locality counts of the synthetic
    replay patterns.

oracle_vectors.npz: seeded small cases of every kernel on the hot path
(Quest and mean selection, resolver over several steps, gather, attention,
append bounds), inputs and the CPU oracle's outputs. The oracle itself is
pinned by the known answers above and by closed forms and second
formulations in tests/test_oracle.py; these vectors freeze its outputs so
that the HIP path is checked against committed data, and any later change of
the oracle shows up as a fixture mismatch. Tensors are stored as raw bits
(16-bit floats as int16) with their dtype name beside them; the file holds
no pickled objects (numpy.load with allow_pickle=False reads it).

Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import oracle  # noqa: E402

KATS_PATH = os.path.join(HERE, "reference_kats.json")
VECTORS_PATH = os.path.join(HERE, "oracle_vectors.npz")

_BITS = {torch.bfloat16: torch.int16, torch.float16: torch.int16, torch.float32: torch.int32,
         torch.int32: torch.int32, torch.int64: torch.int64}
_NAMES = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32", torch.int32: "int32",
          torch.int64: "int64"}
_DTYPES = {v: k for k, v in _NAMES.items()}


# ---- storage --------------------------------------------------------------------------


def put(store, name, t):
    """Store tensor or int64 numpy array `t` as raw bits plus its dtype name."""
    if isinstance(t, np.ndarray):
        t = torch.from_numpy(np.ascontiguousarray(t))
    t = t.detach().cpu().contiguous()
    store[name] = t.view(_BITS[t.dtype]).numpy().copy()
    store[name + ".dtype"] = np.array(_NAMES[t.dtype])


def get(vectors, name):
    """The tensor stored under `name` (CPU, original dtype)."""
    bits = torch.from_numpy(np.array(vectors[name]))
    return bits.view(_DTYPES[str(vectors[name + ".dtype"])])


def put_scalars(store, name, **values):
    store[name] = np.array(json.dumps(values, sort_keys=True))


def get_scalars(vectors, name):
    return json.loads(str(vectors[name]))


# ---- known answers of the reference's tests ---------------------------------------------


def reference_kats():
    return {
        "quest": [
            {  # tests/test_selection.py:18-22
                "query": [[1.0, 0.0]],
                "minimum": [[[-10.0, 0.0]], [[1.0, 0.0]], [[0.0, 0.0]]],
                "maximum": [[[10.0, 0.0]], [[1.0, 0.0]], [[0.0, 0.0]]],
                "length": 5, "page_size": 2, "top_pages": 2, "keep_sink": False,
                "pages": [0, 2], "positions": [0, 1, 4, -1],
            },
            {  # tests/test_selection.py:25-33
                "query": [[1.0, 0.0], [0.0, 1.0]],
                "minimum": [[[9.0, 0.0]], [[0.0, 10.0]], [[-1.0, -1.0]]],
                "maximum": [[[9.0, 0.0]], [[0.0, 10.0]], [[-1.0, -1.0]]],
                "length": 5, "page_size": 2, "top_pages": 2, "keep_sink": False,
                "pages": [1, 2], "positions": [2, 3, 4, -1],
            },
        ],
        "resolve": [
            {  # tests/test_selection.py:36-50
                "source": [5, 2, 9, 4], "resident": [-1, 7, -1, 3], "hot": [6, 1],
                "tags": [-1, -1, -1, -1, -1, 22, -1, -1], "lru": [0, 1, 2, 3, 4, 6, 7, 5],
                "positions": [9, 2, 6, 9, 14, -1], "length": 16, "page_size": 4,
                "physical_rows": [24, 5, 30, -1, 14, -1], "counts": [2, 1, 1],
                "miss_host_rows": [37, -1, -1, -1, -1, -1], "miss_device_rows": [24, -1, -1, -1, -1, -1],
                "tags_after": [37, -1, -1, -1, -1, 22, -1, -1],
                # slot 0 inserted (category 1), slot 5 a protected hit (category 2)
                "lru_after": [1, 2, 3, 4, 6, 7, 0, 5],
            },
        ],
        "trace_locality": [  # tests/test_trace.py:18-56
            {"pattern": p, "capacity": c, "hits": h, "misses": m, "row_jaccard": rj, "page_jaccard": pj,
             "density": d, "reuse_gap": g}
            for p, c, h, m, rj, pj, d, g in [
                ("reuse", 4, 28, 4, 1, 1, 0.25, 1),
                ("alternating", 4, 0, 32, 0, 1, 0.25, 2),
                ("alternating", 8, 24, 8, 0, 1, 0.25, 2),
                ("streaming", 8, 0, 32, 0, 6 / 7, 0.25, None),
                ("packed", 4, 28, 4, 1, 1, 1, 1),
            ]
        ],
    }


# ---- seeded oracle vectors -------------------------------------------------------------------

QUEST_CASES = {  # name: (bounds dtype, query dtype, B, Hq, Hkv, D, P, n_pages, top, keep_sink)
    "quest_bf16": (torch.bfloat16, torch.bfloat16, 2, 8, 2, 64, 16, 40, 8, True),
    "quest_f16_f32q": (torch.float16, torch.float32, 2, 6, 2, 24, 7, 30, 5, False),
    "quest_bf16_g7": (torch.bfloat16, torch.bfloat16, 2, 28, 4, 128, 32, 24, 6, True),
}
MEAN_CASES = {"mean_f32": (2, 4, 2, 64, 16, 40, 8)}  # B, Hq, Hkv, D, P, n_pages, top
RESOLVE_CASES = {  # name: (B, K, H, P, n_pages, mode, steps)
    "resolve_pages": (2, 256, 512, 16, 64, "pages", 3),
    "resolve_random": (2, 100, 150, 7, 40, "random", 3),
}
GATHER_CASES = {"gather_bf16": (torch.bfloat16, 8, 2, 32), "gather_f32": (torch.float32, 3, 1, 8)}  # dtype, P, Hkv, D
ATTEND_CASES = {  # name: (KV dtype, query dtype, B, Hq, Hkv, D, P, N)
    "attend_bf16": (torch.bfloat16, torch.bfloat16, 2, 8, 2, 64, 16, 100),
    "attend_f32": (torch.float32, torch.float32, 2, 4, 2, 32, 8, 37),
}
APPEND_CASES = {"append_bf16": (torch.bfloat16, 16, 2, 32, (1, 3, 12)),  # dtype, P, Hkv, D, counts
                "append_f32": (torch.float32, 7, 1, 8, (2, 5))}


def _quest(store, name, spec, seed):
    dtype, q_dtype, B, Hq, Hkv, D, P, n_pages, top, keep_sink = spec
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, D, generator=g).to(q_dtype)
    a = torch.randn(B, n_pages, Hkv, D, generator=g)
    c = torch.randn(B, n_pages, Hkv, D, generator=g)
    mu = 0.5 * torch.randn(B, n_pages, 1, 1, generator=g)
    mn, mx = torch.minimum(a, c).add(mu).to(dtype), torch.maximum(a, c).add(mu).to(dtype)
    lengths = torch.tensor([n_pages * P, min(top * P - 3, n_pages * P - 1)][:B], dtype=torch.int64)
    scores, pages, pos = oracle.quest_select(q, mn, mx, lengths, P, top, keep_sink)
    for k, v in dict(query=q, minimum=mn, maximum=mx, lengths=lengths, scores=scores, pages=pages,
                     positions=pos).items():
        put(store, f"{name}.{k}", v)
    put_scalars(store, f"{name}.args", page_size=P, top_pages=top, keep_sink=keep_sink)


def _mean(store, name, spec, seed):
    B, Hq, Hkv, D, P, n_pages, top = spec
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, D, generator=g)
    summ = torch.randn(B, n_pages, Hkv, D, generator=g)
    lengths = torch.tensor([n_pages * P - 5, 9 * P][:B], dtype=torch.int64)
    scores, pages, pos = oracle.mean_select(q, summ, lengths, P, top)
    for k, v in dict(query=q, summaries=summ, lengths=lengths, scores=scores, pages=pages, positions=pos).items():
        put(store, f"{name}.{k}", v)
    put_scalars(store, f"{name}.args", page_size=P, top_pages=top)


def _resolver_tables(rng, B, H, P, n_pages):
    """Consistent tables: distinct host slots per page, resident blocks
    distinct and disjoint from the hot blocks, unique tags on host rows of
    non-resident pages, LRU a permutation."""
    host_pages, hot_blocks = 2 * n_pages, -(-H // P)
    pool_blocks = n_pages + hot_blocks + 8
    source = np.full((B, n_pages), -1, np.int64)
    resident = np.full((B, n_pages), -1, np.int64)
    hot = np.zeros((B, hot_blocks), np.int64)
    tags = np.full((B, H), -1, np.int64)
    lru = np.zeros((B, H), np.int64)
    for b in range(B):
        source[b] = rng.permutation(host_pages)[:n_pages]
        source[b, rng.random(n_pages) < 0.05] = -1  # pages without host backing
        blocks = rng.permutation(pool_blocks)
        hot[b] = blocks[:hot_blocks]
        res = rng.random(n_pages) < 0.4
        resident[b, res] = blocks[hot_blocks: hot_blocks + res.sum()]
        cand = (source[b][:, None] * P + np.arange(P)).ravel()
        cand = cand[np.repeat((resident[b] < 0) & (source[b] >= 0), P)]
        chosen = rng.choice(cand, size=min(int(0.6 * H), cand.size), replace=False)
        tags[b, rng.permutation(H)[: chosen.size]] = chosen
        lru[b] = rng.permutation(H)
    return source, resident, hot, tags, lru


def _positions(rng, B, K, lengths, P, mode):
    pos = np.full((B, K), -1, np.int64)
    for b in range(B):
        if mode == "pages":  # whole pages, ascending, tail clipped, -1 padded
            count = -(-int(lengths[b]) // P)
            pages = np.sort(rng.choice(count, size=min(K // P, count), replace=False))
            toks = (pages[:, None] * P + np.arange(P)).ravel()
            toks = toks[toks < lengths[b]]
            pos[b, : toks.size] = toks
        else:  # any order, duplicates, out-of-range and negative entries
            pos[b] = rng.integers(-3, int(lengths[b]) + 5, size=K)
            dup = rng.integers(0, K, size=K // 8)
            pos[b, dup] = pos[b, rng.integers(0, K, size=dup.size)]
    return pos


def _resolve(store, name, spec, seed):
    B, K, H, P, n_pages, mode, steps = spec
    rng = np.random.default_rng(seed)
    source, resident, hot, tags, lru = _resolver_tables(rng, B, H, P, n_pages)
    lengths = rng.integers(n_pages * P // 2, n_pages * P + 1, size=B).astype(np.int64)
    for k, v in dict(source=source, resident=resident, hot=hot, tags=tags, lru=lru, lengths=lengths).items():
        put(store, f"{name}.{k}", v)
    for step in range(steps):
        pos = _positions(rng, B, K, lengths, P, mode)
        outs = [oracle.resolve_rows(pos[b], source[b], resident[b], hot[b], tags[b], lru[b], lengths[b], P)
                for b in range(B)]
        put(store, f"{name}.step{step}.positions", pos)
        for i, k in enumerate(("physical", "miss_host", "miss_device", "counts")):
            put(store, f"{name}.step{step}.{k}", np.stack([o[i] for o in outs]))
        put(store, f"{name}.step{step}.tags_after", tags)
        put(store, f"{name}.step{step}.lru_after", lru)
    put_scalars(store, f"{name}.args", page_size=P, steps=steps)


def _gather(store, name, spec, seed):
    dtype, P, Hkv, D = spec
    g = torch.Generator().manual_seed(seed)
    host_pages, pool_blocks = 24, 10
    host = torch.randn(host_pages, 2, P, Hkv, D, generator=g).to(dtype)
    pool = torch.randn(pool_blocks, 2, P, Hkv, D, generator=g).to(dtype)
    n = 3 * P + 5
    md = torch.randperm(pool_blocks * P, generator=g)[:n]
    mh = torch.randint(0, host_pages * P, (n,), generator=g)
    mh[n // 2:], md[n // 2:] = -1, -1  # compact prefix, then padding
    mh[3], md[3] = -1, -1  # a hole inside the prefix
    after = pool.clone()
    oracle.gather_rows(host, after, mh, md, P)
    for k, v in dict(host=host, pool=pool, miss_host=mh, miss_device=md, pool_after=after).items():
        put(store, f"{name}.{k}", v)
    put_scalars(store, f"{name}.args", page_size=P)


def _attend(store, name, spec, seed):
    dtype, q_dtype, B, Hq, Hkv, D, P, N = spec
    g = torch.Generator().manual_seed(seed)
    blocks = max(4, 2 * N // P + 2)
    pool = torch.randn(blocks, 2, P, Hkv, D, generator=g).to(dtype)
    q = torch.randn(B, Hq, D, generator=g).to(q_dtype)
    rows = torch.randperm(blocks * P, generator=g)[: B * N].view(B, N).clone()
    rows[torch.rand(B, N, generator=g) < 0.2] = -1
    out = oracle.attend_rows(q, pool, rows, P)
    for k, v in dict(query=q, pool=pool, rows=rows, out=out).items():
        put(store, f"{name}.{k}", v)
    put_scalars(store, f"{name}.args", page_size=P)


def _append(store, name, spec, seed):
    dtype, P, Hkv, D, counts = spec
    g = torch.Generator().manual_seed(seed)
    keys = torch.randn(P, Hkv, D, generator=g).to(dtype)
    vals = torch.randn(P, Hkv, D, generator=g).to(dtype)
    summary = torch.zeros(Hkv, D)
    lo = torch.full((Hkv, D), float("inf"))
    hi = torch.full((Hkv, D), float("-inf"))
    within = 0
    put(store, f"{name}.keys", keys)
    put(store, f"{name}.values", vals)
    for i, count in enumerate(counts):
        oracle.append_bounds(keys, within, count, summary, lo, hi)
        within += count
        put(store, f"{name}.append{i}.summary", summary)
        put(store, f"{name}.append{i}.minimum", lo)
        put(store, f"{name}.append{i}.maximum", hi)
    put_scalars(store, f"{name}.args", page_size=P, counts=list(counts))


def build_vectors():
    """Every fixture array, as a dict name -> numpy array."""
    store = {}
    for i, (name, spec) in enumerate(QUEST_CASES.items()):
        _quest(store, name, spec, 100 + i)
    for i, (name, spec) in enumerate(MEAN_CASES.items()):
        _mean(store, name, spec, 200 + i)
    for i, (name, spec) in enumerate(RESOLVE_CASES.items()):
        _resolve(store, name, spec, 300 + i)
    for i, (name, spec) in enumerate(GATHER_CASES.items()):
        _gather(store, name, spec, 400 + i)
    for i, (name, spec) in enumerate(ATTEND_CASES.items()):
        _attend(store, name, spec, 500 + i)
    for i, (name, spec) in enumerate(APPEND_CASES.items()):
        _append(store, name, spec, 600 + i)
    return store


def main():
    with open(KATS_PATH, "w") as f:
        json.dump(reference_kats(), f, indent=1)
        f.write("\n")
    store = build_vectors()
    np.savez_compressed(VECTORS_PATH, **store)
    print(f"wrote {KATS_PATH} and {VECTORS_PATH} ({len(store)} arrays, {os.path.getsize(VECTORS_PATH)} bytes)")


if __name__ == "__main__":
    main()
