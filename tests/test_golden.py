"""Golden fixtures (tests/golden/): the reference's known answers and the
oracle's seeded vectors, checked against the oracle on CPU and against the
HIP kernels through the C ABI on GPU.

- reference_kats.json holds the known answers of the reference's tests
  (tests/test_selection.py:18-50; the trace locality table of
  tests/test_trace.py:18-56 is read by test_trace.py).
- oracle_vectors.npz holds small seeded cases of every hot-path kernel with
  the oracle's outputs; make_golden.py rewrites both files, and the CPU test
  below checks that it reproduces them bit for bit.

Bars: pages, positions, rows, plans, counts, tags, LRU, gathered bytes,
Quest scores and append bounds bit-exact; attention max-abs <= 2e-2 (bf16
KV) or <= 1e-4 (fp32 KV) against the oracle's output.
"""

import importlib.util
import json
import os

import numpy as np
import pytest
import torch

import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
_spec = importlib.util.spec_from_file_location("make_golden", os.path.join(GOLDEN, "make_golden.py"))
make_golden = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(make_golden)
get, get_scalars = make_golden.get, make_golden.get_scalars

ATTN_TOL = {torch.bfloat16: 2e-2, torch.float16: 2e-2, torch.float32: 1e-4}


@pytest.fixture(scope="module")
def vectors():
    with np.load(make_golden.VECTORS_PATH, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.fixture(scope="module")
def kats():
    with open(make_golden.KATS_PATH) as f:
        return json.load(f)


def log_case(**kw):
    print("case:", kw, flush=True)


# ---- CPU: the fixtures, the script and the oracle agree ---------------------------------------


def test_script_reproduces_the_committed_vectors(vectors):
    fresh = make_golden.build_vectors()
    assert sorted(fresh) == sorted(vectors)
    for name, arr in fresh.items():
        assert arr.dtype == vectors[name].dtype and np.array_equal(arr, vectors[name]), name


def test_script_reproduces_the_committed_known_answers(kats):
    assert json.loads(json.dumps(make_golden.reference_kats())) == kats


def test_oracle_reproduces_the_reference_quest_known_answers(kats):
    for kat in kats["quest"]:
        q = torch.tensor(kat["query"])[None]
        mn, mx = torch.tensor(kat["minimum"])[None], torch.tensor(kat["maximum"])[None]
        _, pages, pos = oracle.quest_select(q, mn, mx, [kat["length"]], kat["page_size"], kat["top_pages"],
                                            kat["keep_sink"])
        assert pages[0].tolist() == kat["pages"] and pos[0].tolist() == kat["positions"]


def test_oracle_reproduces_the_reference_resolver_known_answer(kats):
    for kat in kats["resolve"]:
        tags, lru = np.array(kat["tags"], np.int64), np.array(kat["lru"], np.int64)
        phys, mh, md, counts = oracle.resolve_rows(kat["positions"], kat["source"], kat["resident"], kat["hot"],
                                                   tags, lru, kat["length"], kat["page_size"])
        assert phys.tolist() == kat["physical_rows"] and counts.tolist() == kat["counts"]
        assert mh.tolist() == kat["miss_host_rows"] and md.tolist() == kat["miss_device_rows"]
        assert tags.tolist() == kat["tags_after"] and lru.tolist() == kat["lru_after"]


def test_vectors_hold_the_edge_cases(vectors):
    """The seeded cases are not degenerate: short requests, misses, padding."""
    for name in make_golden.RESOLVE_CASES:
        steps = get_scalars(vectors, f"{name}.args")["steps"]
        misses = sum(int(get(vectors, f"{name}.step{s}.counts")[:, 2].sum()) for s in range(steps))
        hits = sum(int(get(vectors, f"{name}.step{s}.counts")[:, 1].sum()) for s in range(steps))
        assert misses > 0 and hits > 0, name
        assert (get(vectors, f"{name}.step0.physical") == -1).any(), name
    for name in make_golden.QUEST_CASES:
        assert (get(vectors, f"{name}.positions") == -1).any(), name  # the short request pads
    for name in make_golden.ATTEND_CASES:
        assert (get(vectors, f"{name}.rows") == -1).any(), name


# ---- GPU: the HIP kernels reproduce the fixtures -------------------------------------------------


@pytest.mark.gpu
def test_hip_reference_known_answers(gpu, kats):
    from nano_hisparse import row_kernels as rk

    log_case(test="golden-kats")
    for kat in kats["quest"]:
        q = torch.tensor(kat["query"], device=gpu)[None]
        mn = torch.tensor(kat["minimum"], device=gpu)[None]
        mx = torch.tensor(kat["maximum"], device=gpu)[None]
        pages, pos, _ = rk.quest_batched(q, mn, mx, kat["length"], kat["page_size"], kat["top_pages"],
                                         keep_sink=kat["keep_sink"])
        assert pages[0].tolist() == kat["pages"] and pos[0].tolist() == kat["positions"]
    for kat in kats["resolve"]:
        t32 = lambda v: torch.tensor([v], dtype=torch.int32, device=gpu)  # noqa: E731
        tags, lru = t32(kat["tags"]), torch.tensor([kat["lru"]], dtype=torch.int64, device=gpu)
        positions = torch.tensor([kat["positions"]], dtype=torch.int64, device=gpu)
        phys, mh, md, counts = rk.resolve_batched(positions, t32(kat["source"]), t32(kat["resident"]),
                                                  t32(kat["hot"]), tags, lru, kat["length"], kat["page_size"])
        assert phys[0].tolist() == kat["physical_rows"] and counts[0].tolist() == kat["counts"]
        assert mh[0].tolist() == kat["miss_host_rows"] and md[0].tolist() == kat["miss_device_rows"]
        assert tags[0].tolist() == kat["tags_after"] and lru[0].tolist() == kat["lru_after"]


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(make_golden.QUEST_CASES))
def test_hip_quest_vectors(gpu, vectors, name):
    from nano_hisparse import row_kernels as rk

    log_case(test="golden-quest", name=name)
    args = get_scalars(vectors, f"{name}.args")
    P, top = args["page_size"], args["top_pages"]
    q, mn, mx, lengths = (get(vectors, f"{name}.{k}") for k in ("query", "minimum", "maximum", "lengths"))
    pages, pos, scores = rk.quest_batched(q.to(gpu), mn.to(gpu), mx.to(gpu), lengths.to(gpu), P, top,
                                          args["keep_sink"])
    assert torch.equal(pages.cpu(), get(vectors, f"{name}.pages"))
    assert torch.equal(pos.cpu(), get(vectors, f"{name}.positions"))
    e_scores = get(vectors, f"{name}.scores")
    for b in range(q.shape[0]):
        count = -(-int(lengths[b]) // P)
        if top < count:  # scored pages (a request with fewer pages than the budget takes them all)
            assert torch.equal(scores.cpu()[b, :count].view(torch.int32), e_scores[b, :count].view(torch.int32))


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(make_golden.MEAN_CASES))
def test_hip_mean_select_vectors(gpu, vectors, name):
    from nano_hisparse import row_kernels as rk

    log_case(test="golden-mean", name=name)
    args = get_scalars(vectors, f"{name}.args")
    q, summ, lengths = (get(vectors, f"{name}.{k}") for k in ("query", "summaries", "lengths"))
    pages, pos, _ = rk.mean_batched(q.to(gpu), summ.to(gpu), lengths.to(gpu), args["page_size"], args["top_pages"])
    assert torch.equal(pages.cpu(), get(vectors, f"{name}.pages"))
    assert torch.equal(pos.cpu(), get(vectors, f"{name}.positions"))


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(make_golden.RESOLVE_CASES))
def test_hip_resolver_vectors(gpu, vectors, name):
    from nano_hisparse import row_kernels as rk

    log_case(test="golden-resolve", name=name)
    args = get_scalars(vectors, f"{name}.args")
    P = args["page_size"]
    src, res, hot = (get(vectors, f"{name}.{k}").to(gpu, torch.int32) for k in ("source", "resident", "hot"))
    tags = get(vectors, f"{name}.tags").to(gpu, torch.int32)
    lru = get(vectors, f"{name}.lru").to(gpu)
    lengths = get(vectors, f"{name}.lengths").to(gpu)
    for s in range(args["steps"]):
        pos = get(vectors, f"{name}.step{s}.positions").to(gpu)
        outs = rk.resolve_batched(pos, src, res, hot, tags, lru, lengths, P)
        for out, k in zip(outs, ("physical", "miss_host", "miss_device", "counts")):
            assert torch.equal(out.cpu(), get(vectors, f"{name}.step{s}.{k}")), (s, k)
        assert torch.equal(tags.cpu().long(), get(vectors, f"{name}.step{s}.tags_after")), s
        assert torch.equal(lru.cpu(), get(vectors, f"{name}.step{s}.lru_after")), s


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(make_golden.GATHER_CASES))
def test_hip_gather_vectors(gpu, vectors, name):
    from nano_hisparse import row_kernels as rk

    log_case(test="golden-gather", name=name)
    P = get_scalars(vectors, f"{name}.args")["page_size"]
    host = get(vectors, f"{name}.host").pin_memory()
    pool = get(vectors, f"{name}.pool").to(gpu)
    mh, md = get(vectors, f"{name}.miss_host").to(gpu), get(vectors, f"{name}.miss_device").to(gpu)
    rk.gather_plan(rk.MappedHost(host), pool, mh, md, P)
    torch.cuda.synchronize()
    assert torch.equal(pool.cpu().view(torch.uint8), get(vectors, f"{name}.pool_after").view(torch.uint8))


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(make_golden.ATTEND_CASES))
def test_hip_attention_vectors(gpu, vectors, name):
    from nano_hisparse import row_kernels as rk

    log_case(test="golden-attend", name=name)
    P = get_scalars(vectors, f"{name}.args")["page_size"]
    q, pool, rows = (get(vectors, f"{name}.{k}") for k in ("query", "pool", "rows"))
    out = rk.attend_batched(q.to(gpu), pool.to(gpu), rows.to(gpu), P)
    err = (out.cpu().float() - get(vectors, f"{name}.out")).abs().max().item()
    assert err <= ATTN_TOL[pool.dtype], err


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(make_golden.APPEND_CASES))
def test_hip_append_vectors(gpu, vectors, name):
    from nano_hisparse import row_kernels as rk

    log_case(test="golden-append", name=name)
    args = get_scalars(vectors, f"{name}.args")
    keys, vals = get(vectors, f"{name}.keys"), get(vectors, f"{name}.values")
    P, Hkv, D = keys.shape
    pool = torch.zeros(2, 2, P, Hkv, D, dtype=keys.dtype, device=gpu)
    summary = torch.zeros(Hkv, D, device=gpu)
    lo = torch.full((Hkv, D), float("inf"), device=gpu).to(keys.dtype)
    hi = torch.full((Hkv, D), float("-inf"), device=gpu).to(keys.dtype)
    within = 0
    for i, count in enumerate(args["counts"]):
        rk.append_page(keys[within: within + count].to(gpu), vals[within: within + count].to(gpu), pool, 1,
                       within, None, 0, summary, lo, hi)
        within += count
        torch.cuda.synchronize()
        assert torch.equal(summary.cpu(), get(vectors, f"{name}.append{i}.summary")), i
        assert torch.equal(lo.float().cpu(), get(vectors, f"{name}.append{i}.minimum")), i
        assert torch.equal(hi.float().cpu(), get(vectors, f"{name}.append{i}.maximum")), i
    assert torch.equal(pool[1, 0, :within].cpu().view(torch.uint8), keys[:within].view(torch.uint8))
    assert torch.equal(pool[1, 1, :within].cpu().view(torch.uint8), vals[:within].view(torch.uint8))
