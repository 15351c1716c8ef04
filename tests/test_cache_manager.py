"""Host logic of the paged ``CacheManager`` and ``PagedRunner`` validation (no GPU).

Restates the reference's paged branches (``engine/cache_manager.py:152-200``
create_handle precision rules, :255-262 quantized growth formula) and the
runner's batch checks (``engine/paged.py:308-335``).
"""

from __future__ import annotations

import pytest

from pkv.cache_errors import CacheCapacityError, CacheCorruptionError, KVQuantizationUnsupported
from pkv.cache_manager import CacheConfig, CacheManager
from pkv.layer import ModelSpec
from pkv.paged import PagedKVCache
from pkv.runner import ForwardRequest, PagedRunner, RunnerOutput


class _Bundle:
    def __init__(self, spec):
        self.spec = spec
        self.activation_dtype = spec.dtype


def _manager(**kw):
    spec = ModelSpec(hidden=256, query_heads=8, kv_heads=2, head_dim=64, num_layers=3,
                     dtype=kw.pop("dtype", "bfloat16"))
    return CacheManager(_Bundle(spec), CacheConfig(**kw), device="cpu")


def test_create_handle_precision_rules():
    cm = _manager()
    h = cm.create_handle("r1", key_type="q8_0", value_type="q8_0")
    assert len(h.bundle.entries) == 3
    assert all(isinstance(e, PagedKVCache) for e in h.bundle.entries)
    assert [e.layer_id for e in h.bundle.entries] == [0, 1, 2]
    assert {e.bits for e in h.bundle.entries} == {8} and {e.dtype for e in h.bundle.entries} == {"float16"}
    h4 = cm.create_handle("r2", key_type="q4_0", value_type="q4_0")
    assert {e.bits for e in h4.bundle.entries} == {4}
    hb = cm.create_handle("r3", key_type="bf16", value_type="bf16")
    assert {e.dtype for e in hb.bundle.entries} == {"bfloat16"} and {e.bits for e in hb.bundle.entries} == {None}
    with pytest.raises(KVQuantizationUnsupported):
        cm.create_handle("r4", key_type="q8_0", value_type="f16")
    with pytest.raises(KVQuantizationUnsupported):
        cm.create_handle("r5", key_type="q2_k", value_type="q2_k")
    assert cm.stats().live_handles == 3


def test_estimate_growth_matches_the_reference_formula():
    cm = _manager(block_size_tokens=16, group_size=32)
    h = cm.create_handle("r", key_type="q8_0", value_type="q8_0")
    # HK * tokens * sum over (Dk, Dv) ceil(D/32) * (32*bits/8 + 4), per layer,
    # plus bytes_per_token * block * 16 (cache_manager.py:255-262)
    per_layer = 2 * 100 * 2 * ((64 + 31) // 32) * (32 * 8 // 8 + 4)
    allowance = 3 * 2 * 2 * 64 * 2 * 16 * 16
    assert cm.estimate_growth(h, 60, 40) == 3 * per_layer + allowance
    hf = cm.create_handle("f", key_type="f16", value_type="f16")
    assert cm.estimate_growth(hf, 10) == 3 * 2 * 2 * 64 * 2 * 10


def test_budget_reservations_and_release():
    cm = _manager(memory_budget_bytes=1000)
    h = cm.create_handle("r", key_type="bf16", value_type="bf16")
    r = cm.reserve(h, 600)
    with pytest.raises(CacheCapacityError):
        cm.reserve(h, 500)
    with pytest.raises(CacheCapacityError):
        with cm.transient_reservation(500):
            pass
    cm.release_reservation(r)
    with cm.transient_reservation(900) as n:
        assert n == 900 and cm.stats().transient_bytes == 900
    assert cm.stats().transient_bytes == 0
    cm.release(h)
    with pytest.raises(CacheCorruptionError):
        cm.release(h)
    with pytest.raises(CacheCorruptionError):
        cm.estimate_growth(h, 1)
    cm.close()
    with pytest.raises(CacheCorruptionError):
        cm.create_handle("late", key_type="bf16", value_type="bf16")


class _Hidden:
    def __init__(self, tokens, hidden):
        self.shape = (tokens, hidden)


class _Model:
    def __init__(self, spec):
        self.spec, self.activation_dtype = spec, spec.dtype


def test_runner_rejects_inconsistent_batches():
    cm = _manager()
    runner = PagedRunner(_Model(cm.bundle.spec))
    h1 = cm.create_handle("a", key_type="bf16", value_type="bf16")
    h2 = cm.create_handle("b", key_type="bf16", value_type="bf16")
    ok = ForwardRequest(None, (), h1.bundle.entries, runtime=cm, handle=h1, request_id="a",
                        hidden=_Hidden(1, 256))
    with pytest.raises(ValueError):
        runner.execute([])
    with pytest.raises(ValueError):        # another phase in the batch
        runner._validate(runner.model, [ok, ForwardRequest(None, (), h2.bundle.entries,
                                             phase="prefill", runtime=cm, handle=h2, request_id="b",
                                             hidden=_Hidden(1, 256))])
    with pytest.raises(ValueError):        # layers out of order
        runner._validate(runner.model, [ForwardRequest(None, (), h1.bundle.entries[::-1],
                                         runtime=cm, request_id="a", hidden=_Hidden(1, 256))])
    with pytest.raises(ValueError):        # the request does not own its caches
        runner._validate(runner.model, [ForwardRequest(None, (), h2.bundle.entries, runtime=cm,
                                         handle=h1, request_id="a", hidden=_Hidden(1, 256))])
    with pytest.raises(ValueError):        # hidden size of another model
        runner._validate(runner.model, [ForwardRequest(None, (), h1.bundle.entries, runtime=cm,
                                         handle=h1, request_id="a", hidden=_Hidden(1, 128))])
    hq = cm.create_handle("q", key_type="q8_0", value_type="q8_0")   # f16 pages, bf16 model
    from pkv.modes import ModelCapabilityUnsupported
    with pytest.raises(ModelCapabilityUnsupported):
        runner._validate(runner.model, [ForwardRequest(None, (), hq.bundle.entries, runtime=cm,
                                         handle=hq, request_id="q", hidden=_Hidden(1, 256))])
    runner._validate(runner.model, [ok])
    with pytest.raises(ValueError):
        RunnerOutput(("a", "a"), (None, None), (1, 1))


def test_in_place_append_rolls_back_by_length():
    """checkpoint / rollback undo page allocation, tail fill and sealing."""
    cm = _manager(block_size_tokens=16)
    h = cm.create_handle("r", key_type="bf16", value_type="bf16")
    cache = h.bundle.entries[0]
    layout = cache.layout_for(2, 64)
    cache._plan_append(10, layout)               # one partial page
    before_pages = list(cache.page_table.pages)
    live_before = cm.block_pool.stats()["block_live"]
    mark = cache.checkpoint()
    cache._plan_append(40, layout)               # fills + seals the tail, two more pages
    assert cache.offset == 50 and len(cache._blocks) == 4
    assert cache._blocks[0].block.immutable
    cache.rollback(mark)
    assert cache.offset == 10 and len(cache._blocks) == 1
    tail = cache._blocks[0].block
    assert tail.token_count == 10 and not tail.immutable
    assert list(cache.page_table.pages) == before_pages
    assert cm.block_pool.stats()["block_live"] == live_before
    cache._plan_append(6, layout)                # appends continue from the restored tail
    assert cache.offset == 16 and cache._blocks[0].block.immutable


# ---------------------------------------------------------------- shared prefixes
# BlockPrefixIndex / adopt_prefix / publish_prefix (engine/prefix_cache.py:186-348,
# engine/cache_manager.py:415-497, :633-667), on the host bookkeeping alone.


def _prefilled(cm, request_id, tokens):
    h = cm.create_handle(request_id, key_type="q8_0", value_type="q8_0")
    for cache in h.bundle.entries:
        cache._plan_append(len(tokens), cache.layout_for(2, 64))
    h.token_count = len(tokens)
    return h


def test_published_prefix_is_adopted_by_a_later_request():
    cm = _manager(prefix_cache_enabled=True, block_size_tokens=16)
    fp = cm.fingerprint(key_type="q8_0", value_type="q8_0")
    prompt = tuple(range(1000, 1053))                    # 3 complete pages + 5 tokens
    first = _prefilled(cm, "a", prompt)
    assert cm.publish_prefix(first, fp, prompt)
    assert cm.block_prefix.stats()["entries"] == 3
    second = cm.create_handle("b", key_type="q8_0", value_type="q8_0")
    assert cm.adopt_prefix(second, fp, prompt + (7, 8)) == 48
    for mine, theirs in zip(second.bundle.entries, first.bundle.entries, strict=True):
        assert mine.offset == 48
        assert [r.block_id for r in mine._blocks] == [r.block_id for r in theirs._blocks[:3]]
        assert all(r.block.references == 2 for r in mine._blocks)
    # the publisher goes away: the index's pins keep the pages for the next request
    cm.release(first)
    third = cm.create_handle("c", key_type="q8_0", value_type="q8_0")
    assert cm.adopt_prefix(third, fp, prompt) == 48
    assert cm.block_prefix.stats()["hits"] == 2


def test_prefix_lookup_stops_at_the_first_different_block_and_never_takes_the_last_token():
    cm = _manager(prefix_cache_enabled=True, block_size_tokens=16)
    fp = cm.fingerprint(key_type="q8_0", value_type="q8_0")
    prompt = tuple(range(64))
    cm.publish_prefix(_prefilled(cm, "a", prompt), fp, prompt)
    index = cm.block_prefix
    assert index.longest_prefix_tokens(fp, prompt) == 48            # last token stays
    assert index.longest_prefix_tokens(fp, prompt + (1,)) == 64
    changed = prompt[:20] + (999,) + prompt[21:]
    assert index.longest_prefix_tokens(fp, changed) == 16
    other = cm.fingerprint(key_type="q4_0", value_type="q4_0")
    assert index.longest_prefix_tokens(other, prompt + (1,)) == 0
    h = cm.create_handle("b", key_type="q8_0", value_type="q8_0")
    assert cm.adopt_prefix(h, fp, prompt + (1,), minimum_tokens=80) == 0
    assert index.stats()["misses"] == 1


def test_prefix_index_evicts_leaves_under_its_budget():
    cm = _manager(prefix_cache_enabled=True, block_size_tokens=16)
    page = cm.block_pool.pool_for(cm.create_handle("x", key_type="q8_0", value_type="q8_0")
                                  .bundle.entries[0].layout_for(2, 64)).page_bytes
    cm.block_prefix.capacity_bytes = 3 * 2 * page       # two blocks of three layers
    fp = cm.fingerprint(key_type="q8_0", value_type="q8_0")
    prompt = tuple(range(49))
    h = _prefilled(cm, "a", prompt)
    assert cm.publish_prefix(h, fp, prompt)
    stats = cm.block_prefix.stats()
    assert stats["entries"] == 2 and stats["evictions"] == 1
    assert cm.block_prefix.longest_prefix_tokens(fp, prompt) == 32   # the leaf went first
    cm.release(h)
    cm.block_prefix.clear()
    assert cm.block_pool.nbytes == 0                     # unpinned pages were freed


def _pins(cm):
    return {int(b): blk.pins for b, blk in cm.block_pool._blocks.items() if blk.pins}


def test_prefix_index_keeps_recently_looked_up_prompts_and_drops_stale_leaves():
    """Two prompts of three pages share their first page; after a lookup of
    the first, a third prompt's publication over budget drops the second
    prompt's pages (least recently used leaves first), never a page some
    kept page extends."""
    cm = _manager(prefix_cache_enabled=True, block_size_tokens=16)
    fp = cm.fingerprint(key_type="q8_0", value_type="q8_0")
    index = cm.block_prefix
    a = tuple(range(49))
    b = a[:16] + tuple(range(500, 533))
    c = tuple(range(900, 949))
    ha, hb, hc = _prefilled(cm, "a", a), _prefilled(cm, "b", b), _prefilled(cm, "c", c)
    assert index.publish(fp, a, tuple(x.full_block_refs for x in ha.bundle.entries)) == 3
    # b's first page is a's (same tokens): only its last two are new nodes
    assert index.publish(fp, b, tuple(x.full_block_refs for x in hb.bundle.entries)) == 2
    assert index.stats()["entries"] == 5
    page_set = index.stats()["bytes"] // 5
    assert index.lookup(fp, a) is not None                   # a is now the most recent
    index.capacity_bytes = 6 * page_set
    assert index.publish(fp, c, tuple(x.full_block_refs for x in hc.bundle.entries)) == 3
    stats = index.stats()
    assert stats["entries"] == 6 and stats["evictions"] == 2
    assert index.longest_prefix_tokens(fp, a) == 48
    assert index.longest_prefix_tokens(fp, b) == 16          # only the shared first page
    assert index.longest_prefix_tokens(fp, c) == 48
    # every node pins one page per layer; b's own pages are unpinned again
    assert sum(_pins(cm).values()) == 6 * 3
    for cache in hb.bundle.entries:
        assert all(r.block.pins == 0 for r in cache._blocks)


def test_prefix_index_metadata_budget_and_stale_heap_items():
    cm = _manager(prefix_cache_enabled=True, block_size_tokens=16)
    fp = cm.fingerprint(key_type="q8_0", value_type="q8_0")
    index = cm.block_prefix
    prompt = tuple(range(81))                                 # five complete pages
    h = _prefilled(cm, "a", prompt)
    assert index.publish(fp, prompt, tuple(x.full_block_refs for x in h.bundle.entries)) == 5
    per_node = index.stats()["metadata_bytes"] // 5
    for _ in range(500):                                      # each lookup re-stamps the path
        assert index.lookup(fp, prompt).token_count == 80
    assert len(index._leaves) <= 4 * 5 + 64
    index.metadata_capacity_bytes = 3 * per_node
    index.publish(fp, prompt, tuple(x.full_block_refs for x in h.bundle.entries))
    assert index.stats()["entries"] == 3 and index.longest_prefix_tokens(fp, prompt) == 48
    assert index.stats()["metadata_bytes"] == 3 * per_node


def test_prefix_publication_that_fails_to_pin_leaves_the_index_as_it_was(monkeypatch):
    cm = _manager(prefix_cache_enabled=True, block_size_tokens=16)
    fp = cm.fingerprint(key_type="q8_0", value_type="q8_0")
    index = cm.block_prefix
    first = tuple(range(33))
    h = _prefilled(cm, "a", first)
    index.publish(fp, first, tuple(x.full_block_refs for x in h.bundle.entries))
    before, pins = index.stats(), _pins(cm)
    longer = tuple(range(81))
    h2 = _prefilled(cm, "b", longer)
    original, calls = cm.block_pool.pin, [0]

    def pin(block_id):
        calls[0] += 1
        if calls[0] == 5:                                     # the second new node, 2nd layer
            raise MemoryError("injected pin failure")
        return original(block_id)

    monkeypatch.setattr(cm.block_pool, "pin", pin)
    with pytest.raises(MemoryError):
        index.publish(fp, longer, tuple(x.full_block_refs for x in h2.bundle.entries))
    assert index.stats() == before and _pins(cm) == pins
    assert index.longest_prefix_tokens(fp, longer) == 32
    monkeypatch.setattr(cm.block_pool, "pin", original)
    assert index.publish(fp, longer, tuple(x.full_block_refs for x in h2.bundle.entries)) == 3
    assert index.longest_prefix_tokens(fp, longer) == 80
    index.clear()
    assert _pins(cm) == {} and index.stats()["entries"] == 0 and index.nbytes == 0


def test_prefix_keys_chain_from_the_fingerprint_digest():
    """A node's key is the reference's chained key: sha256 over the parent's
    key and the page's tokens, starting from the fingerprint digest."""
    import hashlib
    import json

    from pkv.prefix_cache import chain_key

    cm = _manager(prefix_cache_enabled=True, block_size_tokens=16)
    fp = cm.fingerprint(key_type="q8_0", value_type="q8_0")
    prompt = tuple(range(40))
    h = _prefilled(cm, "a", prompt)
    cm.block_prefix.publish(fp, prompt, tuple(x.full_block_refs for x in h.bundle.entries))
    keys, node = [], cm.block_prefix._roots[fp]
    while node.children:
        (node,) = node.children.values()
        keys.append(node.key)
    parent, want = fp.digest, []
    for i in range(2):
        body = json.dumps(list(prompt[16 * i:16 * i + 16]), separators=(",", ":"))
        parent = hashlib.sha256(parent.encode() + b":" + body.encode()).hexdigest()
        want.append(parent)
    assert keys == want == [chain_key(fp.digest, prompt[:16]),
                            chain_key(want[0], prompt[16:32])]


def test_prefix_reuse_rules():
    from pkv.cache_errors import PrefixReuseUnsupported

    cm = _manager(prefix_cache_enabled=False)
    fp = cm.fingerprint(key_type="q8_0", value_type="q8_0")
    h = _prefilled(cm, "a", tuple(range(40)))
    assert cm.publish_prefix(h, fp, tuple(range(40))) is False
    assert cm.adopt_prefix(cm.create_handle("b"), fp, tuple(range(40))) == 0
    cm2 = _manager(prefix_cache_enabled=True)
    mm = cm2.fingerprint(key_type="q8_0", value_type="q8_0", multimodal_identity="img")
    with pytest.raises(PrefixReuseUnsupported):
        cm2.adopt_prefix(cm2.create_handle("c"), mm, (1, 2, 3))
    h2 = _prefilled(cm2, "d", tuple(range(40)))
    assert cm2.publish_prefix(h2, mm, tuple(range(40))) is False
    assert cm2.publish_prefix(h2, fp, tuple(range(39))) is False    # length must match
    assert fp.digest == cm2.fingerprint(key_type="q8_0", value_type="q8_0").digest
    assert fp.digest != cm2.fingerprint(key_type="q8_0", value_type="q8_0", namespace="x").digest


# ------------------------------------------------- allocation failure sweep
# The reference injects a failure at every page allocation of a step and
# checks that offsets, live blocks and reserved bytes are unchanged
# (tests/test_paged_hybrid.py:349-374).  Here the batched attend plans pages
# for every row before its one append launch; a failure at any allocation
# (or at the launch itself, which has no GPU to run on in this suite) must
# roll every row back.


def _sweep_rows(cm):
    rows = []
    for request_id, tokens in (("a", 20), ("b", 9)):
        h = cm.create_handle(request_id, key_type="q8_0", value_type="q8_0")
        cache = h.bundle.entries[0]
        cache._plan_append(tokens, cache.layout_for(2, 64))
        rows.append(cache)
    return rows


def _row_state(cache):
    tail = cache._blocks[-1].block if cache._blocks else None
    return (cache.offset, [r.block_id for r in cache._blocks], list(cache.page_table.pages),
            dict(cache.page_table.entries), tail.token_count if tail else 0,
            tail.immutable if tail else False)


@pytest.mark.parametrize("fail_at", range(1, 6))
def test_every_allocation_of_a_batched_attend_rolls_back(monkeypatch, fail_at):
    from pkv.paged import PagedBatchCache

    cm = _manager(block_size_tokens=16)
    rows = _sweep_rows(cm)
    before = [_row_state(c) for c in rows]
    live = cm.block_pool.stats()["block_live"]
    original, calls = cm.block_pool.allocate_ref, [0]

    def allocate(*args, **kwargs):
        calls[0] += 1
        if calls[0] == fail_at:
            raise MemoryError("injected page allocation")
        return original(*args, **kwargs)

    monkeypatch.setattr(cm.block_pool, "allocate_ref", allocate)
    # 32 new tokens per row: 12 (a) / 7 (b) fill the tails, then two new pages
    # per row -- four allocations; fail_at = 5 fails at the launch instead
    import torch

    batch = PagedBatchCache(tuple(rows), (32, 32), {})
    q = torch.zeros((2, 8, 32, 64), dtype=torch.float16)
    kv = torch.zeros((2, 2, 32, 64), dtype=torch.float16)
    with pytest.raises((MemoryError, ValueError)):
        batch.attend(q, kv, kv, scale=0.125, position_ids=None)
    assert calls[0] == min(fail_at, 4)
    assert [_row_state(c) for c in rows] == before
    assert cm.block_pool.stats()["block_live"] == live
    for cache in rows:
        cache.page_table.validate(cache._blocks)
    # the rows still grow normally afterwards
    monkeypatch.setattr(cm.block_pool, "allocate_ref", original)
    for cache in rows:
        cache._plan_append(32, cache.layout_for(2, 64))
    assert [c.offset for c in rows] == [52, 41]


@pytest.mark.parametrize("fail_at", range(1, 4))
def test_every_allocation_of_a_single_append_rolls_back(monkeypatch, fail_at):
    cm = _manager(block_size_tokens=16)
    cache = _sweep_rows(cm)[0]
    before = _row_state(cache)
    live = cm.block_pool.stats()["block_live"]
    original, calls = cm.block_pool.allocate_ref, [0]

    def allocate(*args, **kwargs):
        calls[0] += 1
        if calls[0] == fail_at:
            raise MemoryError("injected page allocation")
        return original(*args, **kwargs)

    monkeypatch.setattr(cm.block_pool, "allocate_ref", allocate)
    import torch

    k = torch.zeros((1, 2, 40, 64), dtype=torch.float16)   # 12 + 16 + 12: two new pages
    with pytest.raises((MemoryError, ValueError)):
        cache.append(k, k)
    assert _row_state(cache) == before
    assert cm.block_pool.stats()["block_live"] == live
