"""GPU: the reference-named API (``CacheManager`` + ``PagedRunner.execute``) on
the device page arena (``CacheConfig(page_arena="device")``).

The same steps through a host-bookkept manager and a device-arena manager give
the same outputs bit for bit (same kernels, same work split); graph replays of
repeated decode steps equal eager steps; a failing step, an out-of-pages step
and released handles leave the arena consistent; published prefixes are
adopted by reference and give the steps of a recomputed prompt.
"""

from __future__ import annotations

import pytest

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from pkv import _native

    _native.load()


def _setup(page_arena, *, budget=1 << 28, prefix=False, key_type="q8_0", seed=5, pages=0):
    from pkv.cache_manager import CacheConfig, CacheManager
    from pkv.layer import AttentionStack, ModelSpec

    spec = ModelSpec(hidden=256, query_heads=8, kv_heads=2, head_dim=64, num_layers=2,
                     dtype="float16")
    model = AttentionStack(spec, device="cuda", seed=seed)
    cm = CacheManager(model, CacheConfig(block_size_tokens=16, key_type=key_type,
                                         value_type=key_type, group_size=32,
                                         memory_budget_bytes=budget, page_arena=page_arena,
                                         prefix_cache_enabled=prefix, max_sequences=8,
                                         max_sequence_tokens=512, device_pages=pages))
    return model, cm


def _run(runner, cm, handles, xs, phase="prefill"):
    from pkv.runner import ForwardRequest

    return runner.execute([ForwardRequest(None, (), h.bundle.entries, phase=phase,
                                          runtime=cm, handle=h, return_all_logits=True,
                                          request_id=h.request_id, hidden=x)
                           for h, x in zip(handles, xs)])


@pytest.mark.parametrize("key_type", ["q8_0", "q4_0", "f16"])
def test_device_manager_steps_equal_host_manager_steps(key_type):
    from pkv.device_cache import SlotLayerCache
    from pkv.runner import PagedRunner

    model, host_cm = _setup("host", key_type=key_type)
    _, dev_cm = _setup("device", key_type=key_type)
    hh = [host_cm.create_handle(f"r{i}", key_type=key_type, value_type=key_type)
          for i in range(3)]
    dh = [dev_cm.create_handle(f"r{i}", key_type=key_type, value_type=key_type)
          for i in range(3)]
    assert all(isinstance(e, SlotLayerCache) for h in dh for e in h.bundle.entries)
    host, dev, graphs = PagedRunner(model), PagedRunner(model), PagedRunner(model, graphs=True)
    gen = torch.Generator(device="cuda").manual_seed(3)
    widths_seq = [(40, 17, 3), (1, 1, 1), (5, 1, 9)] + [(1, 1, 1)] * 4
    gh = [dev_cm.create_handle(f"g{i}", key_type=key_type, value_type=key_type)
          for i in range(3)]
    for step, widths in enumerate(widths_seq):
        xs = [torch.randn((n, 256), generator=gen, device="cuda").half() for n in widths]
        phase = "decode" if max(widths) == 1 else "prefill"
        a = _run(host, host_cm, hh, xs, phase)
        b = _run(dev, dev_cm, dh, xs, phase)
        c = _run(graphs, dev_cm, gh, xs, phase)          # graph replays from the 2nd decode
        torch.cuda.synchronize()
        for i in range(3):
            assert torch.equal(a.logits[i], b.logits[i]), (step, i)
            assert torch.equal(a.logits[i], c.logits[i]), (step, i)
        assert [h.token_count for h in hh] == [h.token_count for h in dh] == \
            [h.token_count for h in gh]
    assert graphs.last_trace["graph_replay"] and graphs.last_trace["page_arena"] == "device"
    arena = dh[0].bundle.entries[0].arena
    mirror = list(arena.lengths)
    arena.sync_lengths()
    assert arena.lengths == mirror
    free = arena.check()
    for h in dh + gh:
        dev_cm.release(h)
    assert arena.check() > free
    assert dev_cm.stats().live_handles == 0


def test_device_manager_failed_and_out_of_page_steps_change_nothing():
    from pkv.cache_errors import CacheCapacityError
    from pkv.runner import PagedRunner

    # 12 pages per layer: two sequences of 40 tokens take 6
    model, cm = _setup("device", pages=12)
    hs = [cm.create_handle(f"r{i}", key_type="q8_0", value_type="q8_0") for i in range(2)]
    runner = PagedRunner(model)
    gen = torch.Generator(device="cuda").manual_seed(1)
    _run(runner, cm, hs, [torch.randn((40, 256), generator=gen, device="cuda").half()] * 2)
    arena = hs[0].bundle.entries[0].arena
    lens, table = arena.lens.clone(), arena.table.clone()
    free = arena.check()

    class Boom(RuntimeError):
        pass

    forward = model.forward
    model.forward = lambda *a, **k: (_ for _ in ()).throw(Boom())
    with pytest.raises(Boom):
        _run(runner, cm, hs, [torch.zeros((1, 256), device="cuda").half()] * 2, "decode")
    model.forward = forward
    assert [h.token_count for h in hs] == [40, 40] and arena.lengths[:2] == [40, 40]
    assert torch.equal(arena.lens, lens) and arena.check() == free
    with pytest.raises(CacheCapacityError):                # 2 x 60 more tokens: 8 pages
        _run(runner, cm, hs, [torch.zeros((60, 256), device="cuda").half()] * 2)
    assert arena.lengths[:2] == [40, 40] and torch.equal(arena.lens, lens)
    assert torch.equal(arena.table, table) and arena.check() == free
    assert cm.stats().transient_bytes == 0
    out = _run(runner, cm, hs, [torch.randn((1, 256), generator=gen, device="cuda").half()] * 2,
               "decode")
    assert out.committed_token_counts == (1, 1) and [h.token_count for h in hs] == [41, 41]


def test_device_arenas_of_several_precisions_share_one_budget():
    """Each precision's device arena is charged against the one byte budget:
    sized from the budget, the first arena takes all of it and a second
    precision is refused; with pages per arena given, arenas open while they
    fit and the bytes allocated never pass the budget."""
    from pkv.cache_errors import CacheCapacityError
    from pkv.ops import PageFormat

    # two layers of int8 pages: 100 of them and 64 bytes, which fit no page
    per_page = 2 * PageFormat(2, 64, 16, 8, 32, torch.float16).page_bytes
    budget = 100 * per_page + 64
    _, cm = _setup("device", budget=budget)
    cm.create_handle("a", key_type="q8_0", value_type="q8_0")
    assert [dev.capacity for dev, _ in cm.device_arenas.values()] == [100]
    with pytest.raises(CacheCapacityError):
        cm.create_handle("b", key_type="q4_0", value_type="q4_0")
    assert cm.stats().allocated_bytes == 100 * per_page
    assert cm.stats().live_handles == 1

    budget = 1 << 20
    _, cm = _setup("device", budget=budget, pages=40)
    cm.create_handle("a", key_type="q8_0", value_type="q8_0")
    cm.create_handle("b", key_type="q4_0", value_type="q4_0")
    cm.create_handle("c", key_type="q8_0", value_type="q8_0")   # same arena: no new bytes
    pools = [(dev.capacity, len(dev.pools), dev.fmt.page_bytes)
             for dev, _ in cm.device_arenas.values()]
    assert [c for c, _, _ in pools] == [40, 40]
    allocated = sum(c * n * b for c, n, b in pools)
    assert cm.stats().allocated_bytes == allocated <= budget
    with pytest.raises(CacheCapacityError):                     # 40 f16 pages do not fit
        cm.create_handle("d", key_type="f16", value_type="f16")
    assert cm.stats().allocated_bytes == allocated and len(cm.device_arenas) == 2


def test_device_manager_prefix_adoption_gives_the_steps_of_a_recomputed_prompt():
    from pkv.runner import PagedRunner

    model, cm = _setup("device", prefix=True, seed=9)
    fp = cm.fingerprint(key_type="q8_0", value_type="q8_0")
    runner = PagedRunner(model)
    gen = torch.Generator(device="cuda").manual_seed(4)
    prompt = tuple(range(500, 553))                       # 53 tokens: 3 pages + 5
    hidden = torch.randn((53, 256), generator=gen, device="cuda").half()
    a = cm.create_handle("a", key_type="q8_0", value_type="q8_0")
    c = cm.create_handle("c", key_type="q8_0", value_type="q8_0")
    for h in (a, c):
        _run(runner, cm, [h], [hidden[:48]])
        _run(runner, cm, [h], [hidden[48:]])
    assert cm.publish_prefix(a, fp, prompt)
    assert not cm.publish_prefix(a, fp, prompt)           # already held
    b = cm.create_handle("b", key_type="q8_0", value_type="q8_0")
    assert cm.adopt_prefix(b, fp, prompt) == 48
    arena = a.bundle.entries[0].arena
    sa, sb = a.bundle.entries[0].slot, b.bundle.entries[0].slot
    assert arena.table[sb, :3].tolist() == arena.table[sa, :3].tolist()    # shared pages
    refs = arena.refcounts()
    assert all(int(refs[p]) == 3 for p in arena.table[sa, :3].tolist())    # a, b, the index
    _run(runner, cm, [b], [hidden[48:]])
    cm.release(a)                                         # b and the index keep the pages
    for _ in range(3):
        x = torch.randn((1, 256), generator=gen, device="cuda").half()
        out_b, out_c = _run(runner, cm, [b], [x], "decode"), _run(runner, cm, [c], [x], "decode")
        torch.cuda.synchronize()
        assert torch.equal(out_b.logits[0], out_c.logits[0])
    assert b.token_count == c.token_count == 56
    other = cm.create_handle("x", key_type="q8_0", value_type="q8_0")
    assert cm.adopt_prefix(other, fp, prompt[:20] + (7,) * 9) == 16      # one page matches
    assert cm.adopt_prefix(cm.create_handle("y", key_type="q8_0", value_type="q8_0"), fp,
                           prompt[:16]) == 0              # never the last token
    cm.close()
