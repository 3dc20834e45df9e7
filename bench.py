#!/usr/bin/env python3
"""Sparse decode step benchmark on one MI355X.

Workload (one decode step of one layer for a batch, Llama-3-8B head shape):
16 requests x 32 query heads / 8 KV heads x head_dim 128, bf16, 32768 tokens
of context per request in pages of 64 (512 pages), Quest selects 32 pages
(2048 rows, sink and last page forced). Residency over the selected pages:
16 resident in the pool (the last two pages among them), 8 already in the hot
buffer, 8 missing (their rows come from pinned host memory). The hot buffer
holds H = 4096 rows per request, fully occupied, in a random LRU order. Q/K/V
are N(0,1) from a seeded generator.

One step = one layer's batched sparse decode (nano_hisparse.batch_step):
Quest score + top-k (nhs_quest_select) and row resolution
(nhs_resolve_rows) for the whole batch, then the host-row gather
(nhs_gather_rows) and attention (nhs_attend_rows). Four layers are built,
each with its own query, Quest bounds, KV pool and tables over one shared
pinned host store, and step i runs layer i mod 4: between two visits of a
layer ~600 MB of other layers' data pass through the caches, more than the
256 MB Infinity Cache holds, so every launch reads cold data as in a real
multi-layer decode. `value` is that step's time in microseconds (the
metric's "sparse-attn+gather step µs": one layer's quest select + resolve +
gather + attention for the whole batch of 16, lower is better);
`roofline_warm` repeats layer 0 alone for comparison. With --chunks n the
gathers run on a side stream in n groups of requests and each group's
attention starts when its gather event fires, overlapping the next group's
gather; with one chunk everything runs in order on one stream (--side-stream
moves the gather to a second stream ordered by events). Every timed step
resolves against its own copy of its layer's starting tags/LRU, made before
the timed region, so every step has the same 25% misses. In the timed
region the gather and attention launches stamp timing events (the two
roofline kernels' launch times); the Quest and resolver times come from a
second, fully stamped pass. The CPU baseline then runs layer 0's step on
16 host threads and on one: the C port of the reference CPU path (Quest
select, resolver, gather loop, and the reference's float32 masked-softmax
attention), in microseconds per step like `value`; its rows and attention
outputs are checked against the GPU's. The default line ends with
`model_decode`: the whole-model decode below at the workload's 256 decode
steps (decode tokens/s).
Prints one JSON line.

`--workload attention-shapes` times the row attention alone, cold, at four
batch shapes (run_attention_shapes), one JSON line per shape.

`--copy-calibration` instead runs a plain 256 MiB device-to-device copy three
times: the known-size kernel that scales the FETCH_SIZE / WRITE_SIZE
counters of a rocprofv3 --pmc run to bytes.

`--workload model` instead measures whole-model greedy decode: a random-init
Llama-3-8B-shaped decoder (32 layers, hidden 4096, 32/8 heads x 128, MLP
14336, vocab 128256, bf16; q/k/v biases and RoPE theta 1e4 as the reference
model) serving 8 requests with 16384-token random prompts through the engine
with batched decode (Engine(batch_decode=True)): pages of 64, 2048 hot rows,
Quest top-32 pages, a pool of the admission credits plus 30% of the
history. All prompts are prefilled first (untimed); a step is one engine
step giving every request one token.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "nano-hisparse_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "decode tokens/s at 1 GPU; sparse-attn+gather step µs; achieved HBM/PCIe GB/s"
HBM_PEAK = 8.0e12  # MI355X HBM3E, bytes/s
PCIE_PEAK = 64.0e9  # PCIe Gen5 x16, one direction, bytes/s


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-steps", type=int, default=20,
                    help="steps of the CPU oracle baseline, one request per host thread (0 to skip)")
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--context", type=int, default=32768)
    ap.add_argument("--seed", type=int, default=42)
    ap.add_argument("--chunks", type=int, default=1, help="request chunks pipelined against the gather")
    ap.add_argument("--side-stream", action="store_true",
                    help="run the gather on a side stream ordered by events (the default with --chunks > 1)")
    ap.add_argument("--copy-calibration", action="store_true", help="run the PMC calibration copy and exit")
    ap.add_argument("--workload", choices=("kernel", "miss-heavy", "model", "resolver-stress", "attention-shapes"),
                    default="kernel",
                    help="kernel: one-layer sparse decode step (default); miss-heavy: the same step at batch 4, "
                    "128K context, 4096-row budget, ~90%% of rows gathered; model: whole-model batched decode")
    ap.add_argument("--warm-steps", type=int, default=None,
                    help="kernel workloads: steps of the warm single-layer pass (default --steps; 0: none, as for "
                    "a kernel-trace profile whose attention dispatches should all be cold)")
    ap.add_argument("--cold-layers", type=int, default=4,
                    help="kernel workloads: layers with their own device state cycled by the timed steps")
    ap.add_argument("--model-steps", type=int, default=256,
                    help="default line: timed steps of the whole-model decode (model_decode key; 0 to skip)")
    ap.add_argument("--layers", type=int, default=32, help="model workload: decoder layers")
    ap.add_argument("--prompt", type=int, default=16384, help="model workload: prompt tokens per request")
    ap.add_argument("--requests", type=int, default=8, help="model workload: concurrent requests")
    ap.add_argument("--graph", type=int, default=1, choices=(0, 1),
                    help="model workloads: 1 replays each decode step from a captured HIP graph")
    ap.add_argument("--micro-batches", type=int, default=1, choices=(1, 2),
                    help="model workload: 2 pipelines two halves of the batch (gathers beside compute)")
    return ap.parse_args()


class HostStore:
    """The batch's pinned host KV store and the Quest bounds computed from it.

    Host page b * n_pages + p holds request b's logical page p. K/V are
    N(0,1) from a seeded generator; page_offset_std adds a per-page N(0, std)
    offset so Quest scores spread out."""

    q_heads, kv_heads, head_dim, page = 32, 8, 128, 64

    def __init__(self, batch, context, seed, device, page_offset_std=0.0):
        import torch

        self.batch, self.context, self.device = batch, context, device
        B, Hkv, D, P = batch, self.kv_heads, self.head_dim, self.page
        self.n_pages = n_pages = context // P
        dtype = torch.bfloat16
        gen = torch.Generator(device=device).manual_seed(seed)
        self.host = torch.empty(B * n_pages, 2, P, Hkv, D, dtype=dtype, pin_memory=True)
        mn = torch.empty(B, n_pages, Hkv, D, dtype=dtype, device=device)
        mx = torch.empty_like(mn)
        chunk = 256
        for start in range(0, B * n_pages, chunk):
            blk = torch.randn(min(chunk, B * n_pages - start), 2, P, Hkv, D, generator=gen, device=device)
            if page_offset_std:
                blk += page_offset_std * torch.randn(blk.shape[0], 1, 1, 1, 1, generator=gen, device=device)
            blk = blk.to(dtype)
            self.host[start : start + blk.shape[0]].copy_(blk)
            mn.view(B * n_pages, Hkv, D)[start : start + blk.shape[0]] = blk[:, 0].amin(1)
            mx.view(B * n_pages, Hkv, D)[start : start + blk.shape[0]] = blk[:, 0].amax(1)
        self.minimum, self.maximum = mn, mx
        self.lengths = torch.full((B,), context, dtype=torch.int64, device=device)
        self.row_bytes = 2 * Hkv * D * 2


class Layer:
    """One layer's device state over a shared host store: its own query, its
    own copy of the Quest bounds, KV pool and resolver tables, so the layers
    of a pass touch disjoint device memory, as the layers of a model do.

    Selected pages: resident_pages resident (the last two among them),
    hot_pages in the hot buffer, the rest missing. The hot buffer holds
    H = 2 x the selected rows per request, fully occupied (rows of unselected
    pages elsewhere), in a random LRU order."""

    def __init__(self, store, seed, top_pages=32, resident_pages=16, hot_pages=8, chunks=1, compute=None,
                 transfer=None):
        import torch

        from nano_hisparse import row_kernels as rk
        from nano_hisparse.batch_step import BatchTables, SparseDecodeBatch

        self.store = store
        self.top_pages, self.resident_pages, self.hot_pages = top_pages, resident_pages, hot_pages
        self.batch, self.context, self.device = store.batch, store.context, store.device
        self.q_heads, self.kv_heads, self.head_dim, self.page = store.q_heads, store.kv_heads, store.head_dim, store.page
        self.n_pages, self.host, self.lengths, self.row_bytes = store.n_pages, store.host, store.lengths, store.row_bytes
        B, Hq, Hkv, D, P, n_pages, device = (self.batch, self.q_heads, self.kv_heads, self.head_dim, self.page,
                                              self.n_pages, self.device)
        self.K = top_pages * P
        self.H = 2 * self.K
        dtype = torch.bfloat16
        gen = torch.Generator(device=device).manual_seed(seed)
        self.minimum, self.maximum = store.minimum.clone(), store.maximum.clone()
        mn, mx = self.minimum, self.maximum
        self.q = torch.randn(B, Hq, D, generator=gen, device=device).to(dtype)

        pages, _, _ = rk.quest_batched(self.q, mn, mx, self.lengths, P, top_pages)
        pages = pages.cpu()
        rng = torch.Generator().manual_seed(seed + 1)
        hot_blocks = self.H // P
        per_req_blocks = hot_blocks + resident_pages
        self.pool = rk.padded_pool(B * per_req_blocks, P, Hkv, D, dtype, device)
        source = torch.arange(B * n_pages, dtype=torch.int32).view(B, n_pages)
        resident = torch.full((B, n_pages), -1, dtype=torch.int32)
        hot = torch.empty(B, hot_blocks, dtype=torch.int32)
        tags = torch.full((B, self.H), -1, dtype=torch.int32)
        lru = torch.empty(B, self.H, dtype=torch.int64)
        self.classes = []
        for b in range(B):
            sel = pages[b].tolist()
            tail = [p for p in sel if p >= n_pages - 2]
            rest = [p for p in sel if p < n_pages - 2]
            order = [rest[i] for i in torch.randperm(len(rest), generator=rng).tolist()]
            res_pages = tail + order[: resident_pages - len(tail)]
            hot_pg = order[resident_pages - len(tail) : resident_pages - len(tail) + hot_pages]
            miss_pg = order[resident_pages - len(tail) + hot_pages :]
            self.classes.append((res_pages, hot_pg, miss_pg))
            base = b * per_req_blocks
            hot[b] = torch.arange(base, base + hot_blocks, dtype=torch.int32)
            for i, p in enumerate(res_pages):
                blk = base + hot_blocks + i
                resident[b, p] = blk
                self.pool[blk].copy_(self.host[b * n_pages + p])
            # hot rows of the hot-hit pages at random slots; every other slot
            # holds a row of some unselected, non-resident page
            slots = torch.randperm(self.H, generator=rng)
            wanted = torch.tensor([(b * n_pages + p) * P + o for p in hot_pg for o in range(P)], dtype=torch.int32)
            selected = set(sel)
            others = torch.tensor([p for p in range(n_pages) if p not in selected], dtype=torch.int64)
            filler_pages = others[torch.randperm(others.numel(), generator=rng)]
            filler = (b * n_pages + filler_pages[:, None]) * P + torch.arange(P)
            filler = filler.flatten()[: self.H - wanted.numel()].to(torch.int32)
            tags[b, slots[: wanted.numel()]] = wanted
            tags[b, slots[wanted.numel() :]] = filler
            lru[b] = torch.randperm(self.H, generator=rng)
            # load the hot rows' contents into their hot-buffer rows
            for s in slots[: wanted.numel()].tolist():
                host_row = int(tags[b, s])
                hb, ho = divmod(host_row, P)
                db = int(hot[b, s // P])
                self.pool[db, :, s % P].copy_(self.host[hb, :, ho])
        self.source = source.to(device)
        self.resident = resident.to(device)
        self.hot = hot.to(device)
        self.tags0, self.lru0 = tags.to(device), lru.to(device)
        self.tables = BatchTables(self.source, self.resident, self.hot, self.tags0.clone(), self.lru0.clone(),
                                  mn, mx, self.lengths)
        self.out = torch.empty(B, Hq, D, dtype=dtype, device=device)
        self.selected_pages = pages
        self.step = SparseDecodeBatch(self.pool, self.host, self.tables, P, top_pages, chunks=chunks,
                                      compute=compute, transfer=transfer)

    # algorithmic bytes of one attention launch over `requests` requests
    def attention_bytes(self, valid_rows, requests):
        return valid_rows * self.row_bytes + requests * (2 * self.q_heads * self.head_dim * 2 + 8 * self.K)

    def quest_bytes(self):
        return self.batch * (self.n_pages * self.kv_heads * self.head_dim * 2 * 2 + self.q_heads * self.head_dim * 2)


def fresh_state(w):
    """A copy of layer w's starting hot-row tags and LRU order, made before a
    timed region, so that every timed step resolves against the same state
    with no copy kernel inside the region."""
    return (w.tags0.clone(), w.lru0.clone())


def run_step(w, events=None, state=None):
    """One sparse decode step of layer `w` for the whole batch, from the
    starting tags/LRU: `state` is a fresh copy of them, else they are copied
    back first."""
    if state is None:
        w.tables.tags.copy_(w.tags0)
        w.tables.lru.copy_(w.lru0)
    else:
        w.tables.tags, w.tables.lru = state
    return w.step.step(w.q, out=w.out, events=events)[1]


def copy_calibration():
    """A plain 256 MiB device copy, three times: reads and writes 256 MiB each."""
    import torch

    src = torch.ones(256 << 20, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print("copy calibration: 3 x 268435456-byte device copies", flush=True)


def cpu_model_name():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def cpu_threads(batch):
    """Host threads for the CPU baseline: one request per task, at most 16
    (one GPU's share of its host) and at most the CPUs this process may use."""
    return max(1, min(16, len(os.sched_getaffinity(0)), batch))


def cpu_baseline(w, steps, threads):
    """The C oracle (a port of the reference CPU path: Quest select, resolve,
    gather and the reference's float32 attention arithmetic) on layer w's inputs, one
    request per task on `threads` host threads (the oracle's C calls release
    the GIL; a request's gather writes only its own hot blocks, which only
    its attention reads). Returns (median step seconds, physical rows
    [B, K], attention outputs [B, Hq, D] fp32) of the last step."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np
    import torch

    import oracle

    q = w.q.cpu()
    mn, mx = w.minimum.cpu(), w.maximum.cpu()
    lengths = w.lengths.cpu()
    pool = w.pool.cpu()
    source, resident, hot = w.source.cpu().numpy(), w.resident.cpu().numpy(), w.hot.cpu().numpy()
    tags0 = w.tags0.cpu().numpy().astype(np.int64)
    lru0 = w.lru0.cpu().numpy()
    oracle.lib()  # load once, before the threads

    def one_request(b, tags, lru):
        _, _, positions = oracle.quest_select(q[b : b + 1], mn[b : b + 1], mx[b : b + 1], lengths[b : b + 1], w.page,
                                              w.top_pages)
        ph, mh, md, _ = oracle.resolve_rows(
            positions[0].numpy(), source[b], resident[b], hot[b], tags[b], lru[b], int(lengths[b]), w.page
        )
        oracle.gather_rows(w.host, pool, mh, md, w.page)
        out = oracle.attend_rows(q[b : b + 1], pool, torch.from_numpy(ph[None]), w.page, arithmetic="float32")
        return ph, out[0]

    times = []
    results = None
    with ThreadPoolExecutor(threads) as ex:
        for _ in range(steps):
            tags, lru = tags0.copy(), lru0.copy()
            t0 = time.perf_counter()
            results = list(ex.map(lambda b: one_request(b, tags, lru), range(w.batch)))
            times.append(time.perf_counter() - t0)
    physical = np.stack([r[0] for r in results])
    outputs = torch.stack([r[1] for r in results])
    return float(np.median(times)), physical, outputs


def traffic_from_profile(kernel_tag, name="sparse_decode_b16_ctx32k_pmc_traffic.txt", key="traffic_bytes"):
    """Bytes per launch of a kernel from a committed rocprofv3 --pmc summary
    (HBM bytes: FETCH_SIZE and WRITE_SIZE scaled by a plain copy of known
    size; host-link bytes: TCC_EA0_RDREQ_IO_32B x 32), or None when no
    summary is present."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            for line in f:
                fields = line.split()
                if len(fields) >= 3 and fields[0] == key and fields[1] == kernel_tag:
                    return int(fields[2])
    except OSError:
        pass
    return None


ATTENTION_SHAPES = {
    # name: (requests, query heads, KV heads, head_dim, page size, rows per request)
    "b16-32q8kv-2048rows": (16, 32, 8, 128, 64, 2048),  # the default workload's attention
    "b4-32q8kv-4096rows": (4, 32, 8, 128, 64, 4096),  # the miss-heavy step: 128K context, top-64 pages
    "b8-32q8kv-2048rows": (8, 32, 8, 128, 64, 2048),  # the model decode's per-layer attention
    "b64-28q4kv-1024rows": (64, 28, 4, 128, 32, 1024),  # Qwen2-7B heads, top-32 pages of 32
}


def run_attention_shapes(args):
    """Cold row attention alone at four batch shapes. Per shape, n disjoint
    sets of whole pages of distinct pool blocks (bf16 N(0,1) K/V) are
    cycled, n chosen so that at least 512 MB of other rows (twice the
    256 MB Infinity Cache) are read between two visits of a set. The first
    visits are untimed (--warmup launches, at least n), then --steps timed
    launches are stamped with their own dispatch events, then 10 launches
    of one set repeated (warm). One JSON line per shape."""
    import torch

    from nano_hisparse import _hip
    from nano_hisparse import row_kernels as rk

    _hip.load()
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(args.seed)
    for name, (B, Hq, Hkv, D, P, N) in ATTENTION_SHAPES.items():
        pages = N // P
        nbytes = B * N * 2 * Hkv * D * 2 + B * (2 * Hq * D * 2 + 8 * N)
        n_sets = max(4, -(-(512 << 20) // nbytes) + 1)
        blocks = n_sets * B * pages
        pool = rk.padded_pool(blocks, P, Hkv, D, torch.bfloat16, dev)
        for i in range(0, blocks, 512):
            pool[i:i + 512].normal_(generator=g)
        perm = torch.randperm(blocks, generator=g, device=dev)
        sets = []
        for k in range(n_sets):
            blk = perm[k * B * pages:(k + 1) * B * pages].view(B, pages)
            sets.append((blk[:, :, None] * P + torch.arange(P, device=dev)).view(B, N).sort(1).values.long())
        q = torch.randn(B, Hq, D, generator=g, device=dev).to(torch.bfloat16)
        out = torch.empty_like(q)
        for i in range(max(args.warmup, n_sets)):
            rk.attend_batched(q, pool, sets[i % n_sets], P, out=out)
        events = [rk.timing_events() for _ in range(args.steps)]
        torch.cuda.synchronize()
        for i, ev in enumerate(events):
            rk.set_launch_events(*ev)
            rk.attend_batched(q, pool, sets[i % n_sets], P, out=out)
        torch.cuda.synchronize()
        cold = [1e3 * a.elapsed_time(b) for a, b in events]
        warm_events = [rk.timing_events() for _ in range(10)]
        for ev in warm_events:
            rk.set_launch_events(*ev)
            rk.attend_batched(q, pool, sets[0], P, out=out)
        torch.cuda.synchronize()
        warm = [1e3 * a.elapsed_time(b) for a, b in warm_events]
        us, wus = sum(cold) / len(cold), sum(warm) / len(warm)
        print(json.dumps({
            "metric": "cold row-attention launch time", "shape": name, "unit": "us", "value": round(us, 2),
            "higher_is_better": False, "steps": args.steps, "warmup": args.warmup, "algorithmic_bytes": nbytes,
            "achieved_gbs": round(nbytes / us / 1e3, 1), "frac": round(nbytes / us / 1e6 / (HBM_PEAK / 1e12), 4),
            "warm_us": round(wus, 2), "warm_frac": round(nbytes / wus / 1e6 / (HBM_PEAK / 1e12), 4),
            "config": {"requests": B, "q_heads": Hq, "kv_heads": Hkv, "head_dim": D, "page_size": P,
                       "rows_per_request": N, "dtype": "bf16", "row_sets_cycled": n_sets},
        }), flush=True)
        del pool, sets
        torch.cuda.empty_cache()


def run_resolver_stress(args):
    """Quest selection + row resolution for 64 requests with Qwen2-7B heads
    (28 query / 4 KV heads x 128, bf16), contexts uniform in [4096, 65536]
    (seeded), pages of 32, 32 pages = 1024 rows selected, 2048 hot rows per
    request all occupied (every step replaces LRU rows), fresh queries every
    step; prints one JSON line (the step is selection + resolve only: Quest
    scoring, then selection + resolution in one launch when the shape fits
    it, as the batched decode runs them). The timed steps replay captured
    HIP graphs; per-launch times come from an eager pass."""
    import numpy as np
    import torch

    from nano_hisparse import _hip
    from nano_hisparse import row_kernels as rk

    _hip.load()
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    B, Hq, Hkv, D, P, K, H = 64, 28, 4, 128, 32, 1024, 2048
    top = K // P
    g = torch.Generator(device=device).manual_seed(args.seed)
    rng = np.random.default_rng(args.seed)
    lengths = rng.integers(4096, 65536 + 1, size=B)
    n_pages = int(-(-lengths.max() // P))
    counts = -(-lengths // P)
    minimum = torch.empty(B, n_pages, Hkv, D, dtype=torch.bfloat16, device=device)
    maximum = torch.empty_like(minimum)
    for b in range(B):
        keys = torch.randn(n_pages, P, Hkv, D, generator=g, device=device).to(torch.bfloat16)
        minimum[b], maximum[b] = keys.amin(1), keys.amax(1)
    source = np.full((B, n_pages), -1, np.int32)
    resident = np.full((B, n_pages), -1, np.int32)
    hot = np.zeros((B, H // P), np.int32)
    tags = np.full((B, H), -1, np.int32)
    next_host, next_block = 0, 0
    for b in range(B):
        c = int(counts[b])
        source[b, :c] = np.arange(next_host, next_host + c)
        next_host += c
        hot[b] = np.arange(next_block, next_block + H // P)
        next_block += H // P
        res = rng.permutation(c)[: (3 * c) // 10]
        resident[b, res] = np.arange(next_block, next_block + res.size)
        next_block += res.size
        nonres = np.flatnonzero(resident[b, :c] < 0)
        cand = (source[b, nonres][:, None].astype(np.int64) * P + np.arange(P)).ravel()
        tags[b] = rng.choice(cand, size=H, replace=False)
    lru = np.stack([rng.permutation(H) for _ in range(B)])
    to = lambda x: torch.from_numpy(x).to(device)  # noqa: E731
    g_len, g_src, g_res, g_hot, g_tags, g_lru = (to(x) for x in (lengths, source, resident, hot, tags, lru))
    queries = [torch.randn(B, Hq, D, generator=g, device=device).to(torch.bfloat16)
               for _ in range(args.warmup + 2 * args.steps)]
    totals = torch.zeros(3, dtype=torch.int64, device=device)
    ev = [[rk.timing_events(), rk.timing_events()] for _ in range(args.steps)]

    # as the batched decode runs them: Quest scoring, then the selection
    # inside the resolver launch when the shape fits it
    fused = rk.fused_select_fits(n_pages, top, P)

    def step(i, events=None):
        if events:
            rk.set_launch_events(*events[0])
        if fused:
            _, _, scores = rk.quest_batched(queries[i], minimum, maximum, g_len, P, top, select=False)
            if events:
                rk.set_launch_events(*events[1])
            return rk.select_resolve_batched(scores, g_src, g_res, g_hot, g_tags, g_lru, g_len, P, top,
                                             counts_total=totals)[2]
        _, positions, _ = rk.quest_batched(queries[i], minimum, maximum, g_len, P, top)
        if events:
            rk.set_launch_events(*events[1])
        return rk.resolve_batched(positions, g_src, g_res, g_hot, g_tags, g_lru, g_len, P, counts_total=totals)[0]

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # per-launch times and row counts from an eager pass that stamps every launch
    totals.zero_()
    for i in range(args.steps):
        step(args.warmup + i, ev[i])
    torch.cuda.synchronize()
    quest_us = 1e3 * sum(e[0][0].elapsed_time(e[0][1]) for e in ev) / args.steps
    resolve_us = 1e3 * sum(e[1][0].elapsed_time(e[1][1]) for e in ev) / args.steps
    resident_hits, hot_hits, misses = (t / args.steps for t in totals.tolist())
    # The timed pass: the next K steps, each captured into its own HIP graph
    # (its query baked in) and replayed in order, as the batched decode
    # replays its steps, so the host's Python launch path (~100 us a step,
    # against ~46 us of kernels) is not what is measured. The resolver state
    # (tags, LRU) keeps evolving from step to step.
    side = torch.cuda.Stream(device=device)
    side.wait_stream(torch.cuda.current_stream(device))
    pool = torch.cuda.graph_pool_handle()
    graphs = []
    for i in range(args.steps):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side, pool=pool):
            physical = step(args.warmup + args.steps + i)
        graphs.append(graph)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for graph in graphs:
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps

    # attention at the same shape (untimed by the step above): the last
    # step's rows over a pool of random bf16 K/V, per-launch time from events
    pool = rk.padded_pool(next_block, P, Hkv, D, torch.bfloat16, device)
    for i in range(0, next_block, 512):
        pool[i:i + 512].copy_(torch.randn(pool[i:i + 512].shape, generator=g, device=device))
    out = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=device)
    attn_q = queries[-1]
    for _ in range(3):
        rk.attend_batched(attn_q, pool, physical, P, out=out)
    attn_ev = [rk.timing_events() for _ in range(args.steps)]
    torch.cuda.synchronize()
    for e in attn_ev:
        rk.set_launch_events(*e)
        rk.attend_batched(attn_q, pool, physical, P, out=out)
    torch.cuda.synchronize()
    attn_us = 1e3 * sum(a.elapsed_time(b) for a, b in attn_ev) / args.steps
    valid_rows = int((physical >= 0).sum())
    attn_bytes = valid_rows * 2 * Hkv * D * 2 + B * (2 * Hq * D * 2 + 8 * K)
    del pool
    result = {
        "metric": METRIC,
        "value": round(ms * 1e3, 2),  # one layer's selection + resolution for the batch, not a decode rate
        "unit": "µs per step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "resolver stress: Quest selection + row resolution (no gather/attention; the selection "
            "inside the resolver launch, as the batched decode runs it) for 64 requests, "
            "Qwen2-7B heads 28q/4kv/128, bf16, contexts uniform in [4096, 65536], page 32, 1024 rows selected, "
            "2048 hot rows per request fully occupied, fresh queries every step",
            "batch": B,
            "parallelism": "single GPU",
        },
        # from the eager stamped pass; fused: "quest" is the scoring launch and
        # "resolve" the selection + resolution launch; otherwise Quest scoring +
        # selection, then the resolver
        "kernel_us": {"quest": round(quest_us, 2), "resolve": round(resolve_us, 2)},
        "timing": "graph replay, one captured graph per step",
        "fused_selection": fused,
        "rows_per_step": {"resident_hits": resident_hits, "hot_hits": hot_hits, "misses": misses},
        # attention over the same selections, timed separately (not part of value)
        "attention": {"launch_us": round(attn_us, 2), "algorithmic_bytes": attn_bytes,
                      "achieved_gbs": round(attn_bytes / (attn_us * 1e-6) / 1e9, 1),
                      "frac_of_hbm_peak": round(attn_bytes / (attn_us * 1e-6) / HBM_PEAK, 4)},
    }
    print(json.dumps(result), flush=True)


def run_model_decode(args):
    """Whole-model batched decode; prints one JSON line."""
    print(json.dumps(model_decode(args, args.requests, args.layers, args.prompt, args.steps, args.warmup)), flush=True)


def model_decode(args, B, L, T, K, W):
    """Whole-model batched greedy decode of B requests with T-token prompts
    through an L-layer Llama-3-8B-shaped model: K timed engine steps after W
    warm-up steps. Returns the result dict."""
    from math import ceil

    import torch

    from nano_hisparse import _hip
    from nano_hisparse.config import CacheConfig
    from nano_hisparse.engine import Engine
    from nano_hisparse.hybrid import HotConfig, HybridKVCache
    from nano_hisparse.model import Model, ModelConfig

    _hip.load()
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    cfg = ModelConfig(vocab_size=128256, hidden_size=4096, intermediate_size=14336, num_hidden_layers=L,
                      num_attention_heads=32, num_key_value_heads=8, rope_theta=10000.0)
    t0 = time.perf_counter()
    torch.manual_seed(args.seed)
    default_dtype = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(device):
            model = Model(cfg).eval()
    finally:
        torch.set_default_dtype(default_dtype)
    weight_bytes = sum(p.numel() * p.element_size() for p in model.parameters())
    print(f"[bench] model init {time.perf_counter() - t0:.1f} s, {weight_bytes / 1e9:.2f} GB of weights",
          file=sys.stderr, flush=True)
    P, H, top = 64, 2048, 32
    new_tokens = B + W + K + 2  # nobody finishes before the timed steps end
    pages = ceil((T + new_tokens) / P)
    hot = HotConfig(H, H)
    resident = int(0.3 * B * L * pages)
    kv = CacheConfig(gpu_pages=B * hot.admission_blocks(P, L) + resident, host_pages=B * L * pages, page_size=P,
                     kv_heads=8, head_dim=128, dtype=torch.bfloat16, device=str(device),
                     index_budget_bytes=1 << 31)
    t0 = time.perf_counter()
    cache = HybridKVCache(kv, hot)
    print(f"[bench] cache: {kv.gpu_pages} pool blocks ({kv.gpu_pages * kv.row_bytes * P / 2**30:.1f} GiB), "
          f"{kv.host_pages} host pages ({kv.host_pages * kv.row_bytes * P / 2**30:.1f} GiB pinned), "
          f"{time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
    graph = bool(args.graph)
    engine = Engine(model, cache, top_k=top, batch_decode=True, micro_batches=args.micro_batches, graph=graph)
    gen = torch.Generator().manual_seed(args.seed)
    for b in range(B):
        engine.add_request(f"r{b}", torch.randint(0, cfg.vocab_size, (T,), generator=gen).tolist(), new_tokens)
    t0 = time.perf_counter()
    while engine.waiting:  # one prefill per engine step; admitted requests decode meanwhile
        engine.step()
        torch.cuda.synchronize()
        print(f"[bench] admitted {B - len(engine.waiting)}/{B} at {time.perf_counter() - t0:.1f} s",
              file=sys.stderr, flush=True)
    admit_s = time.perf_counter() - t0
    for _ in range(W):
        engine.step()
    torch.cuda.synchronize()
    stats0 = cache.row_stats.tolist()
    compute = torch.cuda.current_stream(device)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(compute)
    for _ in range(K):
        emitted = engine.step()
        if len(emitted) != B:
            raise RuntimeError("a request finished inside the timed steps")
    end.record(compute)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = start.elapsed_time(end) / K
    resident_hits, hot_hits, misses = (a - b for a, b in zip(cache.row_stats.tolist(), stats0))
    row_bytes = kv.row_bytes
    selected_rows = B * L * top * P  # every context holds more than 32 pages
    hbm_bytes = weight_bytes + selected_rows * row_bytes + B * L * pages * 8 * 128 * 2 * 2
    pcie_bytes = misses * row_bytes / K
    ideal_ms = 1e3 * max(hbm_bytes / HBM_PEAK, pcie_bytes / PCIE_PEAK)
    result = {
        "metric": METRIC,
        "value": round(B / (ms_per_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights, random prompt tokens)",
        "config": {
            "workload": f"whole-model batched greedy decode, Llama-3-8B shape ({L} layers, hidden 4096, 32q/8kv x 128, "
            f"MLP 14336, vocab 128256), {B} requests x {T}-token prompts, page 64, hot rows 2048, Quest top-32 "
            f"pages, pool = admission credits + 30% of history",
            "requests": B,
            "prompt": T,
            "layers": L,
            "micro_batches": args.micro_batches,
            "decode_graph": graph,
            "parallelism": "single GPU",
        },
        "rows_per_step": {"resident_hits": resident_hits / K, "hot_hits": hot_hits / K, "misses": misses / K},
        "pcie_gbs": round(pcie_bytes / (ms_per_step * 1e-3) / 1e9, 2),
        "step_roofline": {"ideal_ms": round(ideal_ms, 3), "frac": round(ideal_ms / ms_per_step, 4),
                          "hbm_bytes": hbm_bytes, "pcie_bytes": round(pcie_bytes)},
        "wall_s_timed": round(wall, 3),
        "admit_s": round(admit_s, 2),  # untimed: every prompt prefilled, admitted requests decoding meanwhile
    }
    del engine, cache, model
    torch.cuda.empty_cache()
    return result


def main():
    args = parse_args()
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the sparse decode step shards by "
            "request with no exchange, so the N-GPU figure would be N independent copies of this one)",
            file=sys.stderr,
        )
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return
    if args.workload == "model":
        run_model_decode(args)
        return
    if args.workload == "resolver-stress":
        run_resolver_stress(args)
        return
    if args.workload == "attention-shapes":
        run_attention_shapes(args)
        return
    import torch

    from nano_hisparse import _hip

    _hip.load()
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    miss_heavy = args.workload == "miss-heavy"
    if miss_heavy:
        args.batch, args.context = 4, 131072
    L = args.cold_layers
    print(f"[bench] building workload batch={args.batch} context={args.context} layers={L}", file=sys.stderr,
          flush=True)
    store = HostStore(args.batch, args.context, args.seed, device, page_offset_std=0.5 if miss_heavy else 0.0)
    compute = torch.cuda.current_stream(device)
    transfer = torch.cuda.Stream(device=device) if args.side_stream else None
    # miss-heavy: the two tail pages resident, 4 pages hot, 58 of 64 missing
    kw = dict(top_pages=64, resident_pages=2, hot_pages=4) if miss_heavy else {}
    layers = [Layer(store, args.seed + 1000 * l, chunks=args.chunks, compute=compute, transfer=transfer, **kw)
              for l in range(L)]
    w = layers[0]
    names = ("quest", "resolve", "gather", "attention")

    def layer_of(i):  # step i runs layer i mod L: a layer's data is cold at every visit
        return layers[i % L]

    results = {}
    for i in range(max(args.warmup, L)):
        results[i % L] = run_step(layer_of(i))
    torch.cuda.synchronize()
    per_layer = []
    for l, layer in enumerate(layers):
        r = results[l]
        counts_sum = r.counts.sum(0).tolist()
        valid = [int((r.physical[c] >= 0).sum()) for c in r.chunks]
        requests = [c.stop - c.start for c in r.chunks]
        per_layer.append({"counts": counts_sum, "valid": valid, "requests": requests,
                          "attn_bytes": sum(layer.attention_bytes(v, n) for v, n in zip(valid, requests)),
                          "gather_bytes": counts_sum[2] * layer.row_bytes})
    n_chunks = len(results[0].chunks)
    print(f"[bench] layer 0 counts resident/hot/miss = {per_layer[0]['counts']}, valid rows "
          f"{sum(per_layer[0]['valid'])}, chunks {per_layer[0]['requests']}", file=sys.stderr, flush=True)

    def timed_pass(layer_for_step, events):
        """K steps bracketed by a barrier and a synchronisation on both sides;
        returns (ms per step, host enqueue seconds, wall seconds)."""
        states = [fresh_state(layer_for_step(i)) for i in range(args.steps)]
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        start.record(compute)
        for i in range(args.steps):
            run_step(layer_for_step(i), events[i] if events else None, states[i])
        end.record(compute)
        enqueue_s = time.perf_counter() - t0
        torch.cuda.synchronize()
        return start.elapsed_time(end) / args.steps, enqueue_s, time.perf_counter() - t0

    def launch_us(events, name):
        """Mean launch time of stage `name` over the steps' launches (chunks)."""
        pairs = [pair for ev in events for pair in ev[name]]
        return 1e3 * sum(a.elapsed_time(b) for a, b in pairs) / len(pairs)

    # The timed region: K steps cycling over the L layers. The launches of
    # the two roofline kernels, gather and attention, stamp timing events
    # here (measured: with the gather unstamped, the attention's own stamps
    # read ~1.7 us longer). A stamped launch costs a few microseconds, so the
    # Quest and resolver times come from a second pass stamped at every
    # launch.
    cold_events = []
    for i in range(args.steps):
        full = layer_of(i).step.timing_events()
        cold_events.append({"gather": full["gather"], "attention": full["attention"]})
    ms_per_step, enqueue_s, wall = timed_pass(layer_of, cold_events)
    attn_us = launch_us(cold_events, "attention")
    gather_us = n_chunks * launch_us(cold_events, "gather")  # per step: all of its chunks
    stamped = [layer_of(i).step.timing_events() for i in range(args.steps)]
    stamped_ms, _, _ = timed_pass(layer_of, stamped)
    kernel_us = {n: len(stamped[0][n]) * launch_us(stamped, n) for n in names}
    kernel_us["gather"] = gather_us  # from the timed pass, like the attention's launch time
    # warm: every step on layer 0, whose data the previous step left in the caches
    warm_steps = args.steps if args.warm_steps is None else args.warm_steps
    if warm_steps > 0:
        warm_events = []
        for _ in range(warm_steps):
            full = w.step.timing_events()
            warm_events.append({"gather": full["gather"], "attention": full["attention"]})
        steps, args.steps = args.steps, warm_steps
        warm_ms, _, _ = timed_pass(lambda i: w, warm_events)
        args.steps = steps
        warm_attn_us = launch_us(warm_events, "attention")

    # measured pinned H2D copy ceiling (copy engine), for reference
    probe = torch.empty(256 << 20, dtype=torch.uint8, pin_memory=True)
    dst = torch.empty(probe.shape, dtype=torch.uint8, device=device)
    dst.copy_(probe, non_blocking=True)
    torch.cuda.synchronize()
    h2d = []
    for _ in range(3):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        dst.copy_(probe, non_blocking=True)
        b.record()
        torch.cuda.synchronize()
        h2d.append(probe.numel() / (a.elapsed_time(b) * 1e-3))
    del probe, dst

    # algorithmic bytes per launch, averaged over the layers (each is visited equally often)
    attn_launch_bytes = sum(x["attn_bytes"] for x in per_layer) / L / n_chunks
    w0_attn_launch_bytes = per_layer[0]["attn_bytes"] / n_chunks
    gather_bytes = sum(x["gather_bytes"] for x in per_layer) / L
    quest_bytes = w.quest_bytes()
    step_us = ms_per_step * 1e3
    # ideal step: every HBM byte at the HBM peak, or every host byte at the PCIe peak
    ideal_us = 1e6 * max((attn_launch_bytes * n_chunks + quest_bytes + gather_bytes) / HBM_PEAK,
                         gather_bytes / PCIE_PEAK)
    # the committed PMC summaries cover the default workload only
    default = (not miss_heavy and (args.batch, args.context, args.seed, n_chunks, L) == (16, 32768, 42, 1, 4))
    traffic = traffic_from_profile("attend_mfma_kernel") if default else None
    host_traffic = (
        traffic_from_profile("gather_rows_kernel", "sparse_decode_b16_ctx32k_pmc_host_link.txt", "host_read_bytes")
        if default else None
    )
    result = {
        "metric": METRIC,
        "value": round(step_us, 2),
        "unit": "µs per step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": (
                "sparse decode step of one layer (quest select + resolve + host-row gather + attention), "
                "Llama-3-8B heads 32q/8kv/128, bf16, page 64, 32 pages = 2048 rows selected of 32768, "
                "selected pages 50% resident / 25% hot / 25% host misses, hot rows 4096 per request"
                if not miss_heavy else
                "miss-heavy sparse decode step of one layer, Llama-3-8B heads 32q/8kv/128, bf16, page 64, "
                "64 pages = 4096 rows selected of 131072, selected pages: 2 tail pages resident, 4 hot, 58 host "
                "misses; K/V N(0,1) plus a per-page offset N(0, 0.5); hot rows 8192 per request"
            ),
            "value": "one layer's sparse decode step for the whole batch (quest select + resolve + host-row "
                     "gather + attention), microseconds per step; whole-model decode tokens/s: model_decode",
            "step": f"one layer's step; step i runs layer i mod {L}, each layer with its own device pool, "
                    "bounds and tables (shared pinned host store), so every step reads data the other layers "
                    "evicted from the 256 MB Infinity Cache",
            "batch": w.batch,
            "context": w.context,
            "layers_cycled": L,
            "chunks": n_chunks,
            "gather_stream": "side" if w.step.transfer is not w.step.compute else "compute",
            "parallelism": "single GPU",
        },
        "step_us": round(step_us, 2),
        # per-stage launch times (cold): gather from the timed pass, the
        # others from a second pass of K steps that stamps every launch (its
        # step time: stamped_step_us)
        "kernel_us": {n: round(v, 2) for n, v in kernel_us.items()},
        # the sparse-attention + gather step: resolve (with the page selection
        # in the same launch) + gather + attention, the launches that follow
        # the Quest scoring on the step's critical path
        "sparse_attn_gather_step_us": round(sum(kernel_us[n] for n in ("resolve", "gather", "attention")), 2),
        "stamped_step_us": round(stamped_ms * 1e3, 2),
        "roofline": {
            "kernel": "nhs_attend_rows (attend_mfma_kernel)",
            "bound": "hbm",
            "achieved": round(attn_launch_bytes / (attn_us * 1e-6) / 1e9, 1),
            "peak": HBM_PEAK / 1e9,
            "unit": "GB/s",
            "frac": round(attn_launch_bytes / (attn_us * 1e-6) / HBM_PEAK, 4),
            "traffic": traffic,
            "algorithmic_bytes": round(attn_launch_bytes),
            "launch_us": round(attn_us, 2),
            "cache": "cold: the launch's rows, bounds and tables untouched for >600 MB of other traffic",
        },
        "roofline_warm": {
            "frac": round(w0_attn_launch_bytes / (warm_attn_us * 1e-6) / HBM_PEAK, 4),
            "launch_us": round(warm_attn_us, 2),
            "step_us": round(warm_ms * 1e3, 2),
            "cache": "warm: layer 0 repeated, ~202 MB per step (below the 256 MB Infinity Cache)",
        } if warm_steps > 0 else None,
        "gather_roofline": {
            "kernel": "nhs_gather_rows (gather_rows_kernel)",
            "bound": "pcie",
            "achieved": round(gather_bytes / (kernel_us["gather"] * 1e-6) / 1e9, 2),
            "peak": PCIE_PEAK / 1e9,
            "unit": "GB/s",
            "frac": round(gather_bytes / (kernel_us["gather"] * 1e-6) / PCIE_PEAK, 4),
            "measured_h2d_copy_gbs": round(max(h2d) / 1e9, 2),
            "algorithmic_bytes": round(gather_bytes),
            "traffic": host_traffic,
        },
        "step_roofline": {"ideal_us": round(ideal_us, 1), "frac": round(ideal_us / step_us, 4)},
        "quest_gbs": round(quest_bytes / (kernel_us["quest"] * 1e-6) / 1e9, 1),
        "wall_s_timed": round(wall, 3),
        "host_enqueue_us_per_step": round(enqueue_s * 1e6 / args.steps, 1),
    }
    if args.cpu_steps > 0:
        threads = cpu_threads(w.batch)
        print(f"[bench] CPU oracle baseline: {args.cpu_steps} steps on {threads} threads, then 1 thread",
              file=sys.stderr, flush=True)
        r0 = run_step(w)  # layer 0's pool, rows and output as the CPU leg starts from them
        torch.cuda.synchronize()
        cpu_s, cpu_physical, cpu_out = cpu_baseline(w, args.cpu_steps, threads)
        if not (torch.from_numpy(cpu_physical) == r0.physical.cpu()).all():
            raise RuntimeError("GPU resolved rows differ from the CPU oracle")
        attn_err = (w.out.cpu().float() - cpu_out).abs().max().item()
        if attn_err > 2e-2:
            raise RuntimeError(f"GPU attention differs from the CPU oracle by {attn_err} (max-abs)")
        one_steps = max(1, min(3, args.cpu_steps))
        cpu1_s, _, _ = cpu_baseline(w, one_steps, 1)
        result["cpu_baseline"] = {
            "value": round(cpu_s * 1e6, 1),
            "unit": "µs per step",
            "cores": threads,
            "kind": "port",
            "sample": f"{args.cpu_steps} full steps of layer 0's inputs (the whole batch of {w.batch}), one "
                      f"request per thread; median step",
            "arithmetic": "the C port of the reference CPU path: fp32 Quest scores, integer resolver, byte "
                          "gather loop, the reference's float32 masked-softmax attention (attention.py:26-35)",
            "single_thread": {"value": round(cpu1_s * 1e6, 1), "unit": "µs per step", "cores": 1,
                              "sample": f"{one_steps} full steps, median"},
            "host": f"{cpu_model_name()} ({os.cpu_count()} CPUs visible)",
        }
        result["parity"] = {"rows_bit_exact": True, "attention_max_abs": float(f"{attn_err:.3g}")}
    if not miss_heavy and args.model_steps > 0:
        del layers, w, store, results
        torch.cuda.empty_cache()
        print(f"[bench] whole-model decode: 8 requests x 16384-token prompts, {args.model_steps} timed steps",
              file=sys.stderr, flush=True)
        try:
            m = model_decode(args, 8, 32, 16384, args.model_steps, 2)
            result["model_decode"] = {
                "value": m["value"], "unit": "tokens/s", "ms_per_step": m["ms_per_step"], "steps": m["steps"],
                "workload": m["config"]["workload"], "step_roofline": m["step_roofline"],
                "rows_per_step": m["rows_per_step"], "pcie_gbs": m["pcie_gbs"], "admit_s": m["admit_s"],
                "decode_graph": m["config"]["decode_graph"],
            }
        except Exception as exc:  # the kernel line stands on its own
            result["model_decode"] = {"error": f"{type(exc).__name__}: {exc}"}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
