"""CPU: host logic of the drop-in boundary and the workloads (no kernels run).

Arena/page-table invariants restate the reference's own tests
(``tests/test_paged_hybrid.py:214-225, 750-794``) for the device page pools;
pools are placed on the CPU here because only host bookkeeping is exercised.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from pkv import ops, workloads  # noqa: E402
from pkv.arena import SEGMENT_PAGES, PersistentPageTable, SegmentedPageArena  # noqa: E402
from pkv.block_cache import BlockId  # noqa: E402
from pkv.cache_errors import CacheCapacityError, CacheCorruptionError  # noqa: E402
from pkv.modes import ModelCapabilityUnsupported  # noqa: E402
from pkv.paged import PagedKVCache  # noqa: E402


def _cache(arena, bits=8, group=64):
    return PagedKVCache(arena, dtype="bfloat16", bits=bits, group_size=group)


def _plan(cache, tokens, heads=2, dim=64):
    return cache._plan_append(tokens, cache.layout_for(heads, dim))


def test_block_id_packing():
    b = BlockId((5 << 96) | (7 << 32) | 9)
    assert (b.epoch, b.slot, b.generation) == (5, 7, 9)


def test_pages_segments_and_table_updates():
    arena = SegmentedPageArena(2**40, block_tokens=16, device="cpu")
    cache = _cache(arena)
    _plan(cache, 257)
    assert cache.offset == 257 and len(cache._blocks) == 17
    assert len(arena.segments) == 2                       # 257 tokens -> 2 segments of 16 pages
    assert all(r.block.immutable for r in cache._blocks[:16])
    assert not cache._blocks[-1].block.immutable and cache._blocks[-1].block.token_count == 1
    assert cache.page_table.pages == [r.block.page for r in cache._blocks]
    prefix_chunk = cache.page_table.chunks[0]
    branch = cache.page_table.fork()
    assert branch.chunks[0] is prefix_chunk                # forks share chunks
    before = arena.table_update_bytes
    _plan(cache, 1)
    assert arena.table_update_bytes - before == SEGMENT_PAGES * 4 * 4   # one 256-byte chunk
    assert cache.page_table.chunks[0] is prefix_chunk
    cache.page_table.validate(cache._blocks)


def test_refcounts_seal_and_release():
    arena = SegmentedPageArena(2**40, block_tokens=16, device="cpu")
    cache = _cache(arena)
    _plan(cache, 40)
    shared = cache._blocks[0].fork()
    assert cache._blocks[0].block.references == 2
    cache.reset()
    assert shared.block.references == 1
    shared.close()
    with pytest.raises(CacheCorruptionError):
        shared.close()                                      # double close
    with pytest.raises(CacheCorruptionError):
        _ = shared.block
    assert arena.stats()["block_live"] == 0
    with pytest.raises(CacheCorruptionError):
        arena.seal(arena.allocate(None, 3, layout=cache.layout_for(2, 64)))  # partial page


def test_shared_mutable_tail_is_rejected():
    arena = SegmentedPageArena(2**40, block_tokens=16, device="cpu")
    cache = _cache(arena)
    _plan(cache, 5)
    other = cache._blocks[-1].fork()
    with pytest.raises(ValueError, match="shared"):
        _plan(cache, 1)
    other.close()


def test_trim_adopt_and_layout_checks():
    arena = SegmentedPageArena(2**40, block_tokens=16, device="cpu")
    cache = _cache(arena)
    _plan(cache, 50)
    with pytest.raises(ModelCapabilityUnsupported):
        cache.trim(3)                                       # not page aligned
    cache.trim(2)                                           # 48 tokens: whole pages
    assert cache.offset == 48 and len(cache.page_table.pages) == 3
    refs = [r.fork() for r in cache._blocks]
    other = _cache(arena)
    other.adopt(refs)
    assert other.offset == 48 and other.page_table.pages == cache.page_table.pages
    wrong = _cache(arena, bits=4)
    with pytest.raises(ModelCapabilityUnsupported):
        wrong.adopt([r.fork() for r in cache._blocks])
    with pytest.raises(ModelCapabilityUnsupported):
        cache.update(None, None)
    with pytest.raises(ModelCapabilityUnsupported):
        cache.state()
    with pytest.raises(ModelCapabilityUnsupported):
        PagedKVCache(arena, dtype="float32")


def test_capacity_error_and_page_reuse():
    fmt_bytes = ops.PageFormat(2, 64, 16, 8, 64, torch.bfloat16).page_bytes
    arena = SegmentedPageArena(3 * fmt_bytes, block_tokens=16, device="cpu")
    cache = _cache(arena)
    _plan(cache, 48)
    with pytest.raises(CacheCapacityError):
        _plan(_cache(arena), 1)
    pages = list(cache.page_table.pages)
    cache.reset()
    again = _cache(arena)
    _plan(again, 48)
    assert sorted(again.page_table.pages) == sorted(pages)   # freed pages are reused


def test_page_table_truncate():
    arena = SegmentedPageArena(2**40, block_tokens=16, device="cpu")
    cache = _cache(arena)
    _plan(cache, 16 * 20)
    table = cache.page_table
    table.truncate(17)
    assert len(table.pages) == 17 and max(table.entries) == 16 and set(table.chunks) == {0, 1}


# ---------------------------------------------------------------- workloads


def test_workloads_are_seeded_and_follow_configs():
    a = workloads.generate(workloads.get("c2"), kv=False)
    b = workloads.generate(workloads.get("c2"), kv=False)
    assert np.array_equal(a.context, b.context) and np.array_equal(a.table, b.table)
    assert a.context.min() >= 1024 and a.context.max() <= 8192 and len(a.context) == 32
    used = a.table[a.table >= 0]
    assert len(np.unique(used)) == len(used)                 # distinct pages per sequence
    c1 = workloads.generate(workloads.get("c1"), kv=False)
    assert c1.num_pages == 128 and list(c1.context) == [128, 256, 384, 512]
    c4 = workloads.generate(workloads.get("c4"), kv=False)
    assert np.all(c4.table[:, :16] == c4.table[0, :16])       # 256-token shared prefix
    assert c4.positions.shape == (16, 5)
    c5 = workloads.generate(workloads.get("c5"), kv=False)
    assert c5.positions.shape == (4, 512)
    assert np.all(c5.positions[:, 0] == 4096) and np.all(c5.positions[:, -1] == 4607)


def test_workload_waves():
    """C3's 512-token partitions as waves: one per partition of every (sequence, KV head)."""
    import bench

    c3 = workloads.get("c3")
    assert bench.workload_waves(c3, [32768] * 8) == 8 * 64 * 4
    assert bench.workload_waves(workloads.get("c2"), [5000] * 32) == 0   # library default


def test_prefill_flops_match_the_causal_count():
    """C5 flops: the closed form 4*D*H*B*(512*4096 + 512*513/2) and a brute-force
    count of (query, visible token) pairs on a small chunk."""
    import bench

    c5 = workloads.get("c5")
    assert bench.is_prefill(c5) and not bench.is_prefill(workloads.get("c4"))
    assert bench.attention_flops(c5, [4608] * 4) == 4 * 128 * 32 * 4 * (512 * 4096 + 512 * 513 // 2)
    small = workloads.get("c5", batch=2, num_queries=7, heads=2, kv_heads=1, head_dim=3)
    lengths = [20, 9]
    pairs = sum(1 for n in lengths for q in range(7) for t in range(n) if t <= n - 7 + q)
    assert bench.attention_flops(small, lengths) == 4 * 3 * 2 * pairs


def test_bench_bytes_match_the_configs():
    """Algorithmic bytes of bench.py against the per-config figures (C2 at E[L], C3 exact)."""
    import bench

    w = workloads.get("c2")
    assert bench.kv_bytes_per_token(w) == 2176
    lengths = [4608 + 1] * 32
    attn, step = bench.algorithmic_bytes(w, lengths)
    want = 2176 * sum(lengths) + 32 * (8192 + 8192) + 4 * sum(math.ceil(x / 16) for x in lengths)
    assert attn == want and step == want + 32 * 4096
    assert abs(step / 1e6 - 321.6) < 1.0
    w3 = workloads.get("c3")
    assert bench.kv_bytes_per_token(w3) == 576
    attn3, _ = bench.algorithmic_bytes(w3, [32768] * 8)
    assert attn3 - 4 * 8 * 1024 == 150_994_944 + 131_072


def test_profiled_traffic_matches_algorithmic_bytes():
    """The committed PMC profile of the C2 attention launch: HBM traffic within
    5% of the algorithmic bytes (no re-reads), as bench.py reports it."""
    import bench

    traffic = bench.measured_traffic("c2")
    assert traffic is not None
    w = workloads.get("c2")
    inst = workloads.generate(w, kv=False)
    attn, _ = bench.algorithmic_bytes(w, inst.context + w.append_tokens)
    assert 1.0 <= traffic / attn < 1.05


def test_page_pool_stays_within_the_byte_budget_and_reuses_lowest_ids():
    """A pool grows by doubling but never past the arena's budget in pages;
    freed pages come back lowest id first."""
    arena = SegmentedPageArena(10 * 34816, block_tokens=16, device="cpu")   # 10 C2 pages
    cache = _cache(arena, bits=8, group=64)
    layout = cache.layout_for(8, 128)
    pool = arena.pool_for(layout)
    assert pool.page_bytes == 34816 and pool.max_pages == 10
    _plan(cache, 160, heads=8, dim=128)                  # 10 pages: the whole budget
    assert pool.capacity == 10 and pool.buffer.shape[0] == 10
    with pytest.raises(CacheCapacityError):
        _plan(cache, 1, heads=8, dim=128)
    freed = [cache._blocks[i].block.page for i in (7, 3, 5)]
    for i in sorted((7, 3, 5), reverse=True):
        cache._blocks.pop(i).close()
    assert [pool.take() for _ in range(3)] == sorted(freed)


def _recount(arena):
    """The pool's statistics recomputed from every live block."""
    blocks = list(arena._blocks.values())
    nbytes = sum(b.nbytes for b in blocks)
    return {"block_total": len(blocks), "block_live": sum(b.references > 0 for b in blocks),
            "block_prefix": sum(b.pins > 0 for b in blocks),
            "block_shared": sum(b.references > 1 for b in blocks),
            "block_pinned": sum(b.pins > 0 for b in blocks), "live_bytes": nbytes,
            "retained_free_bytes": arena.allocated_nbytes - nbytes,
            "evictable_bytes": sum(b.nbytes for b in blocks if b.references == 0 and b.pins == 1),
            "shared_page_savings_bytes": sum(b.nbytes * max(b.references - 1, 0) for b in blocks),
            "pinned_bytes": sum(b.nbytes for b in blocks if b.pins),
            "page_payload_bytes": sum(b.nbytes * b.token_count // arena.block_tokens
                                      for b in blocks),
            "segment_count": len(arena.segments)}


def test_running_pool_statistics_match_a_recount():
    """stats() is kept incrementally (it runs every runner step): through
    appends that fill and seal tails, forks, pins of evicted-to-prefix pages,
    rollbacks of partial tails and releases, it equals a recount of the live
    blocks."""
    rng = np.random.default_rng(7)
    arena = SegmentedPageArena(2**40, block_tokens=16, device="cpu")
    caches = [_cache(arena) for _ in range(4)]
    held, pinned = [], []
    for step in range(120):
        op = int(rng.integers(6))
        c = caches[int(rng.integers(len(caches)))]
        if op <= 1:
            _plan(c, int(rng.integers(1, 40)))
        elif op == 2 and any(r.block.immutable for r in c._blocks):
            sealed = [r for r in c._blocks if r.block.immutable]     # a mutable tail stays unshared
            held.append(sealed[int(rng.integers(len(sealed)))].fork())
        elif op == 3 and held:
            ref = held.pop(int(rng.integers(len(held))))
            arena.pin(ref.block_id)
            ref.close()                                  # pinned only: evictable
            if rng.integers(2):
                arena.unpin(ref.block_id)
            else:
                pinned.append(ref.block_id)
        elif op == 4:
            mark = c.checkpoint()
            _plan(c, int(rng.integers(1, 20)))
            c.rollback(mark)
        elif op == 5 and rng.integers(4) == 0:
            c.reset()
        got = arena.stats()
        want = _recount(arena)
        assert {k: got[k] for k in want} == want, step
    for ref in held:
        ref.close()
    for c in caches:
        c.reset()
    for block_id in pinned:
        arena.unpin(block_id)
    assert arena.stats()["block_total"] == 0 and arena.stats()["page_payload_bytes"] == 0
    assert _recount(arena)["live_bytes"] == 0 == arena.stats()["evictable_bytes"]
