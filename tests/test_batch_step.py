"""The batched decode step (nano_hisparse.batch_step, gathers pipelined with
attention in chunks of requests on a side stream) against the C
oracle run request by request: selected positions, resolved rows, the
gathered pool bytes and the tags/LRU state bit-exact; attention within 2e-2
(bf16 KV) or 1e-4 (fp32 KV) max-abs of the oracle's float64 softmax.
"""

import numpy as np
import pytest
import torch

import oracle


def build(batch, n_pages, page, kv_heads, head_dim, q_heads, top_pages, hot_rows, dtype, seed, pinned=True):
    """Stacked tables for `batch` requests of n_pages pages each: a random
    half of the pages resident, hot rows filled with random host rows of the
    request (some of them rows Quest will select), random LRU order."""
    from nano_hisparse.batch_step import BatchTables

    g = torch.Generator().manual_seed(seed)
    B, P, H = batch, page, hot_rows
    host = torch.empty(B * n_pages, 2, P, kv_heads, head_dim, dtype=dtype, pin_memory=pinned)
    host.copy_(torch.randn(host.shape, generator=g).to(dtype))
    keys = host[:, 0].view(B, n_pages, P, kv_heads, head_dim)
    minimum, maximum = keys.amin(2), keys.amax(2)
    hot_blocks = -(-H // P)
    resident_per_req = n_pages // 2
    blocks_per_req = hot_blocks + resident_per_req
    pool = torch.zeros(B * blocks_per_req, 2, P, kv_heads, head_dim, dtype=dtype)
    source = torch.arange(B * n_pages, dtype=torch.int32).view(B, n_pages)
    resident = torch.full((B, n_pages), -1, dtype=torch.int32)
    hot = torch.empty(B, hot_blocks, dtype=torch.int32)
    tags = torch.full((B, H), -1, dtype=torch.int32)
    lru = torch.empty(B, H, dtype=torch.int64)
    for b in range(B):
        base = b * blocks_per_req
        hot[b] = torch.arange(base, base + hot_blocks, dtype=torch.int32)
        chosen = torch.randperm(n_pages, generator=g)[:resident_per_req]
        for i, p in enumerate(chosen.tolist()):
            resident[b, p] = base + hot_blocks + i
            pool[base + hot_blocks + i] = host[b * n_pages + p]
        rows = (b * n_pages * P + torch.randperm(n_pages * P, generator=g)[: H - H // 4]).to(torch.int32)
        slots = torch.randperm(H, generator=g)[: rows.numel()]
        tags[b, slots] = rows
        for s, r in zip(slots.tolist(), rows.tolist()):
            hb, ho = divmod(r, P)
            pool[int(hot[b, s // P]), :, s % P] = host[hb, :, ho]
        lru[b] = torch.randperm(H, generator=g)
    lengths = torch.full((B,), n_pages * P, dtype=torch.int64)
    lengths[0] -= P // 2  # a partial last page
    q = torch.randn(B, q_heads, head_dim, generator=g).to(dtype)
    tables = BatchTables(source, resident, hot, tags, lru, minimum, maximum, lengths)
    return host, pool, tables, q


def oracle_step(host, pool, tables, q, page, top_pages, tags, lru):
    """Request by request: Quest select, resolve, gather, attend (CPU)."""
    B = q.shape[0]
    _, _, positions = oracle.quest_select(q, tables.minimum, tables.maximum, tables.lengths, page, top_pages)
    physical = np.empty((B, positions.shape[1]), np.int64)
    for b in range(B):
        ph, mh, md, _ = oracle.resolve_rows(
            positions[b].numpy(), tables.source[b].numpy(), tables.resident[b].numpy(), tables.hot[b].numpy(),
            tags[b], lru[b], int(tables.lengths[b]), page,
        )
        oracle.gather_rows(host, pool, mh, md, page)
        physical[b] = ph
    out = oracle.attend_rows(q, pool, torch.from_numpy(physical), page)
    return positions, physical, out


@pytest.mark.gpu
@pytest.mark.parametrize(
    "batch,n_pages,page,kv_heads,head_dim,q_heads,top_pages,hot_rows,dtype,chunks,tol",
    [
        (6, 40, 16, 2, 128, 8, 8, 256, torch.bfloat16, 3, 2e-2),
        (5, 33, 8, 4, 64, 16, 6, 96, torch.bfloat16, 2, 2e-2),
        (4, 20, 16, 2, 64, 4, 5, 160, torch.float32, 4, 1e-4),
        (3, 64, 64, 8, 128, 32, 4, 512, torch.bfloat16, 1, 2e-2),
    ],
)
def test_pipelined_step_matches_oracle(gpu, batch, n_pages, page, kv_heads, head_dim, q_heads, top_pages,
                                       hot_rows, dtype, chunks, tol):
    from nano_hisparse.batch_step import BatchTables, SparseDecodeBatch

    host, pool, tables, q = build(batch, n_pages, page, kv_heads, head_dim, q_heads, top_pages, hot_rows, dtype, 7)
    dev = BatchTables(*(t.to(gpu) for t in (tables.source, tables.resident, tables.hot, tables.tags, tables.lru,
                                            tables.minimum, tables.maximum, tables.lengths)))
    dpool = pool.to(gpu)
    step = SparseDecodeBatch(dpool, host, dev, page, top_pages, chunks=chunks)
    tags = tables.tags.numpy().astype(np.int64)
    lru = tables.lru.numpy().copy()
    cpool = pool.clone()
    for it in range(3):  # the tables evolve: later steps hit rows earlier steps gathered
        query = q if it == 0 else torch.randn(q.shape, generator=torch.Generator().manual_seed(it)).to(dtype)
        out, result = step.step(query.to(gpu))
        positions, physical, counts = result.positions, result.physical, result.counts
        torch.cuda.synchronize()
        e_pos, e_phys, e_out = oracle_step(host, cpool, tables, query, page, top_pages, tags, lru)
        assert torch.equal(positions.cpu(), e_pos), f"step {it}: positions"
        assert np.array_equal(physical.cpu().numpy(), e_phys), f"step {it}: rows"
        assert np.array_equal(dev.tags.cpu().numpy(), tags), f"step {it}: tags"
        assert np.array_equal(dev.lru.cpu().numpy(), lru), f"step {it}: lru"
        assert torch.equal(dpool.cpu().view(torch.uint8), cpool.view(torch.uint8)), f"step {it}: pool bytes"
        err = (out.float().cpu() - e_out).abs().max().item()
        assert err <= tol, f"step {it}: attention max-abs {err}"
        assert int(counts.sum()) == int((physical >= 0).sum())
