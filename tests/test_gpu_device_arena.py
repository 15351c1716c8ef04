"""GPU: device-side page allocation (``pkv_arena_*``, ``pkv.device_arena``).

Checked against a host model of the same ownership rules (free pages,
reference counts, copy-on-write of a shared tail) and the invariants they
imply: every page is either free or referenced, a page's count equals the
number of slot tables holding it, no page appears twice on the free stack.
Attention through device-allocated pages must equal attention through
host-allocated pages bit for bit (same kernels, same bytes; only page ids
differ) and the oracle within the attention tolerance; graph replays of a
reserve + append + attention step must equal the same steps run eagerly.
"""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from paged_case import assert_attention_close, fill_pages, oracle_attention, scale_of, to_torch  # noqa: E402


def _fmt(w=None, **kw):
    from pkv.ops import PageFormat

    if w is not None:
        return PageFormat(w.kv_heads, w.head_dim, w.page_tokens, w.bits, w.group_size,
                          torch.bfloat16)
    base = dict(num_kv_heads=2, head_dim=64, page_tokens=16, bits=8, group_size=32,
                dtype=torch.bfloat16)
    base.update(kw)
    return PageFormat(**base)


def _arena(capacity=64, **kw):
    from pkv.device_arena import DevicePageArena

    return DevicePageArena(_fmt(), capacity, **kw)


def _invariants(arena):
    """Free stack + references account for every page exactly once."""
    torch.cuda.synchronize()
    free, err = arena.status()
    assert err == 0, f"error bits {err:#x}"
    refs = arena.refcounts().numpy()
    stack = arena.free_stack().numpy()
    assert len(set(stack.tolist())) == len(stack) == free
    held = {}
    lens = arena.lens.cpu().numpy()
    table = arena.table.cpu().numpy()
    for s in range(arena.max_slots):
        n = -(-int(lens[s]) // arena.page_tokens)
        assert (table[s, :n] >= 0).all() and (table[s, n:] == -1).all()
        for p in table[s, :n]:
            held[int(p)] = held.get(int(p), 0) + 1
        assert int(lens[s]) == arena.lengths[s]
    for p in range(arena.capacity):
        assert refs[p] == held.get(p, 0), f"page {p}: count {refs[p]}, held {held.get(p, 0)}"
        assert (refs[p] == 0) == (p in set(stack.tolist()))


def test_reserve_hands_out_pages_in_order_and_fills_tails_first():
    arena = _arena(64, max_slots=8, max_tokens=256)
    res = arena.reserve([0, 1, 2], [20, 5, 40])
    torch.cuda.synchronize()
    assert arena.pages(0) == [0, 1] and arena.pages(1) == [2] and arena.pages(2) == [3, 4, 5]
    assert res.starts.tolist() == [0, 0, 0] and res.lens.tolist() == [20, 5, 40]
    table = res.table.cpu().numpy()
    assert table[0, :2].tolist() == [0, 1] and table[2, :3].tolist() == [3, 4, 5]
    arena.reserve([0], [12])            # 20 -> 32: fills page 1, no new page
    assert arena.pages(0) == [0, 1]
    res = arena.reserve([0, 1], [1, 11])  # 32 -> 33 opens a page; 5 -> 16 fills slot 1's
    assert arena.pages(0) == [0, 1, 6] and arena.pages(1) == [2]
    assert res.starts.tolist() == [32, 5] and res.lens.tolist() == [33, 16]
    assert arena.check() == 64 - 7
    _invariants(arena)


def test_fork_shares_pages_and_copies_a_shared_tail_on_first_write():
    arena = _arena(32, num_layers=3, max_slots=8, max_tokens=128)
    arena.reserve([1], [21])                       # pages [0, 1], tail 1 holds 5 tokens
    for i, pool in enumerate(arena.pools):         # distinct bytes per layer and page
        pool.copy_(torch.randint(0, 256, pool.shape, generator=torch.Generator().manual_seed(i),
                                 dtype=torch.uint8).cuda())
    before = [pool[1].clone() for pool in arena.pools]
    arena.fork([1], [3])
    assert arena.pages(3) == [0, 1] and arena.refcounts()[:2].tolist() == [2, 2]
    arena.reserve([3], [2])                        # first write into the shared tail: copy
    torch.cuda.synchronize()
    new = arena.pages(3)[1]
    assert arena.pages(1) == [0, 1] and arena.pages(3)[0] == 0 and new not in (0, 1)
    for pool, old in zip(arena.pools, before):
        assert torch.equal(pool[1], old) and torch.equal(pool[new], old)
    assert arena.refcounts()[[0, 1, new]].tolist() == [2, 1, 1]
    _invariants(arena)
    # two sharers of one tail writing in the same call: exactly one copies
    arena.fork([1], [4])
    pages_before = 32 - arena.check()
    arena.reserve([1, 4], [1, 1])
    assert 32 - arena.check() == pages_before + 1
    assert arena.pages(1)[1] != arena.pages(4)[1]
    _invariants(arena)


def test_truncate_and_release_return_pages():
    arena = _arena(16, max_slots=4, max_tokens=256)
    arena.reserve([0, 1], [40, 16])
    arena.fork([0], [2])
    arena.truncate([0], [17])                      # keeps 2 pages; page 2 still held by slot 2
    assert arena.pages(0) == [0, 1] and arena.refcounts()[2].item() == 1
    arena.release([2])                             # page 2 freed, 0 and 1 drop to one reference
    assert arena.refcounts()[:3].tolist() == [1, 1, 0]
    assert arena.check() == 16 - 3
    _invariants(arena)
    arena.release([0, 1])
    assert arena.check() == 16
    _invariants(arena)


def test_out_of_pages_and_full_table_change_nothing():
    from pkv.cache_errors import CacheCapacityError

    arena = _arena(4, max_slots=4, max_tokens=64)
    arena.reserve([0], [30])                       # 2 pages
    res = arena.reserve([1, 2], [20, 20])          # needs 4, 2 free: nothing grows
    torch.cuda.synchronize()
    assert res.lens.tolist() == [0, 0] and (res.table[:, :2].cpu().numpy() == -1).all()
    with pytest.raises(CacheCapacityError):
        arena.check()
    arena.lengths[1] = arena.lengths[2] = 0        # the host mirror counted the failed growth
    _invariants(arena)
    res = arena.reserve([0], [1])                  # 30 -> 31 fits in its tail page
    assert res.lens.tolist() == [31]
    arena.reserve(torch.tensor([0], dtype=torch.int32, device="cuda"),
                  torch.tensor([100], dtype=torch.int32, device="cuda"))  # past max_tokens
    with pytest.raises(CacheCapacityError):
        arena.check()
    assert arena.lens[0].item() == 31


def test_a_blocked_decode_step_overwrites_no_cached_token():
    """Regression: slots whose length is a multiple of the page size (one of
    them sharing forked pages) and no free page.  A one-token step cannot
    grow them; it must raise CacheCapacityError and leave every pool byte,
    reference count, table, length and the free stack as they were, both run
    eagerly (fused append + attention) and replayed from captured graphs.
    A blocked row once kept its old length L as the batch length, and the
    single-token append (positioned at length - 1) overwrote token L - 1 of
    a valid, shared page in every layer."""
    from pkv.cache_errors import CacheCapacityError
    from pkv.device_arena import DevicePageArena, DeviceRunner
    from pkv.layer import AttentionStack, ModelSpec
    from pkv.ops import PageFormat

    spec = ModelSpec(hidden=256, query_heads=8, kv_heads=2, head_dim=64, num_layers=2,
                     dtype="float16")
    model = AttentionStack(spec, device="cuda", seed=6)
    fmt = PageFormat(2, 64, 16, 8, 32, torch.float16)
    arena = DevicePageArena(fmt, 5, num_layers=2, max_slots=4, max_tokens=256)
    runner = DeviceRunner(model, arena)
    a, c, d = arena.open_slot(), arena.open_slot(), arena.open_slot()
    gen = torch.Generator(device="cuda").manual_seed(6)
    x0 = torch.randn((3, 32, 256), generator=gen, device="cuda").half()
    runner.execute([a, c, d], x0, [32, 16, 20])    # pages: a 2, c 1, d 2 -> 5 of 5
    b = arena.open_slot()
    arena.fork([a], [b])                           # b shares a's two full pages
    assert arena.check() == 0
    slots = [a, b, c, d]                           # a, b, c need a page; d's tail has room

    def snapshot():
        torch.cuda.synchronize()
        return ([p.clone() for p in arena.pools], arena.refcounts(), arena.free_stack(),
                arena.table.clone(), arena.lens.clone())

    def assert_unchanged(before, what):
        after = snapshot()
        for l, (p0, p1) in enumerate(zip(before[0], after[0])):
            assert torch.equal(p0, p1), f"{what}: layer {l}'s pool changed"
        for name, x0_, x1_ in zip(("refcounts", "free stack", "table", "lengths"),
                                  before[1:], after[1:]):
            assert torch.equal(x0_, x1_), f"{what}: {name} changed"

    before = snapshot()
    mirror = list(arena.lengths)
    x1 = torch.randn((4, 1, 256), generator=gen, device="cuda").half()
    with pytest.raises(CacheCapacityError):
        runner.execute(slots, x1)
    assert arena.lengths == mirror
    assert_unchanged(before, "eager step")

    step = runner.capture_decode(slots, x1.clone(), warm=False)
    for i in range(2):
        step.replay()
        with pytest.raises(CacheCapacityError):
            arena.check()
        assert_unchanged(before, f"replay {i}")
    arena.sync_lengths()
    assert arena.lengths == mirror
    _invariants(arena)


def test_random_operations_keep_the_invariants():
    rng = np.random.default_rng(7)
    arena = _arena(96, max_slots=12, max_tokens=320)
    live = set()
    for step in range(60):
        op = rng.integers(0, 4)
        free_slots = [s for s in range(arena.max_slots) if s not in live]
        if op == 0 and free_slots:                              # new sequences grow
            slots = list(rng.choice(free_slots, size=min(3, len(free_slots)), replace=False))
            live.update(int(s) for s in slots)
            arena.reserve([int(s) for s in slots], [int(x) for x in rng.integers(1, 60, len(slots))])
        elif op == 1 and live:                                   # a batch step of live ones
            slots = sorted(live)[: int(rng.integers(1, len(live) + 1))]
            widths = [int(min(x, 320 - arena.lengths[s])) for s, x in
                      zip(slots, rng.integers(0, 20, len(slots)))]
            arena.reserve(slots, widths)
        elif op == 2 and live and free_slots:                    # fork
            src = int(rng.choice(sorted(live)))
            dst = int(free_slots[0])
            arena.fork([src], [dst])
            live.add(dst)
        elif op == 3 and live:                                   # truncate or release
            s = int(rng.choice(sorted(live)))
            if rng.random() < 0.5:
                arena.release([s])
                live.discard(s)
            else:
                arena.truncate([s], [int(rng.integers(0, arena.lengths[s] + 1))])
        free, err = arena.status()
        if err:                                                  # out of pages: undo the mirror
            arena.state[1:2].zero_()
            for s in range(arena.max_slots):
                arena.lengths[s] = int(arena.lens[s].item())
        _invariants(arena)


@pytest.mark.parametrize("chunk", [None, 100, 7])
def test_attention_over_device_pages_equals_host_pages(chunk):
    from pkv import ops, workloads
    from pkv.device_arena import DevicePageArena

    w = workloads.get("c2", batch=5, length_range=(30, 700))
    inst = workloads.generate(w)
    fmt = _fmt(w)
    lengths = [k.shape[1] for k in inst.keys]
    arena = DevicePageArena(fmt, sum(-(-n // 16) for n in lengths) + 8, max_slots=8,
                            max_tokens=max(lengths))
    slots = [arena.open_slot() for _ in range(w.batch)]
    longest = max(lengths)
    step = chunk or longest
    for start in range(0, longest, step):         # append the contexts in chunks
        width = [int(np.clip(n - start, 0, step)) for n in lengths]
        res = arena.reserve(slots, width)
        k = np.zeros((w.batch, w.kv_heads, step, w.head_dim), np.float32)
        v = np.zeros_like(k)
        for b in range(w.batch):
            k[b, :, :width[b]] = inst.keys[b][:, start:start + width[b]]
            v[b, :, :width[b]] = inst.values[b][:, start:start + width[b]]
        ops.append_quantize(fmt, arena.pools[0], to_torch(k, fmt.dtype), to_torch(v, fmt.dtype),
                            res.table, res.starts, res.widths)
    arena.check()
    res = arena.reserve(slots, [0] * w.batch)     # the batch's operands, nothing grows
    q = to_torch(inst.queries, fmt.dtype)
    q_pos = torch.from_numpy(inst.positions).cuda()
    scale = scale_of(w.head_dim)
    got = ops.paged_attention(fmt, arena.pools[0], q, res.table, res.lens, scale=scale, q_pos=q_pos)
    pool, table, lens = fill_pages(fmt, inst, chunk=chunk)
    want = ops.paged_attention(fmt, pool, q, table, lens, scale=scale, q_pos=q_pos)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert_attention_close(got.float().cpu().numpy(),
                           oracle_attention(fmt, inst, inst.positions,
                                            np.full(w.batch, w.num_queries, np.int32), scale))
    _invariants(arena)


def test_graph_replays_of_a_decode_step_equal_eager_steps():
    from pkv import ops
    from pkv.device_arena import DeviceBatchCache, DevicePageArena

    fmt = _fmt(num_kv_heads=2, head_dim=64, page_tokens=16, bits=8, group_size=32)
    batch, heads = 4, 8
    gen = torch.Generator(device="cuda").manual_seed(3)

    def make():
        arena = DevicePageArena(fmt, 64, max_slots=batch, max_tokens=512)
        slots = [arena.open_slot() for _ in range(batch)]
        res = arena.reserve(slots, [37, 16, 5, 90])
        k = torch.randn((batch, 2, 90, 64), generator=torch.Generator(device="cuda").manual_seed(1),
                        device="cuda").to(fmt.dtype)
        ops.append_quantize(fmt, arena.pools[0], k, k * 0.5, res.table, res.starts, res.widths)
        return arena, slots

    qs = torch.randn((6, batch, heads, 1, 64), generator=gen, device="cuda").to(fmt.dtype)
    kvs = torch.randn((6, 2, batch, 2, 1, 64), generator=gen, device="cuda").to(fmt.dtype)
    scale = 0.125

    eager, eslots = make()
    want = []
    for i in range(4):
        res = eager.reserve(eslots, [1] * batch)
        want.append(DeviceBatchCache(eager, 0, res).attend(qs[i], kvs[i, 0], kvs[i, 1], scale=scale))
    torch.cuda.synchronize()

    arena, slots = make()
    slots_d = torch.tensor(slots, dtype=torch.int32, device="cuda")
    widths_d = torch.ones(batch, dtype=torch.int32, device="cuda")
    q_in, k_in, v_in = qs[0].clone(), kvs[0, 0].clone(), kvs[0, 1].clone()
    res = arena.reserve(slots_d, widths_d)          # step 0 eagerly: sizes the buffers
    out = DeviceBatchCache(arena, 0, res).attend(q_in, k_in, v_in, scale=scale)
    torch.cuda.synchronize()
    assert torch.equal(out, want[0])
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            res_g = arena.reserve(slots_d, widths_d, out=res)
            out_g = DeviceBatchCache(arena, 0, res_g).attend(q_in, k_in, v_in, scale=scale)
    torch.cuda.current_stream().wait_stream(stream)
    for i in range(1, 4):                           # each replay is one more decode step
        q_in.copy_(qs[i])
        k_in.copy_(kvs[i, 0])
        v_in.copy_(kvs[i, 1])
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, want[i]), f"replay {i}"
        arena.status()                              # eager work between replays
    assert arena.lens[slots].tolist() == [37 + 4, 16 + 4, 5 + 4, 90 + 4]
    arena.lengths = [int(x) for x in arena.lens.cpu()]
    _invariants(arena)


def test_device_runner_matches_the_host_runner_and_rolls_back():
    """The same layer steps through PagedRunner (host pages) and DeviceRunner
    (device pages) give the same outputs bit for bit; a step that raises leaves
    the device slots at their lengths before it; captured decode steps equal
    eager ones."""
    from pkv.cache_manager import CacheConfig, CacheManager
    from pkv.device_arena import DevicePageArena, DeviceRunner
    from pkv.layer import AttentionStack, ModelSpec
    from pkv.ops import PageFormat
    from pkv.runner import ForwardRequest, PagedRunner

    spec = ModelSpec(hidden=256, query_heads=8, kv_heads=2, head_dim=64, num_layers=2,
                     dtype="float16")
    model = AttentionStack(spec, device="cuda", seed=5)
    cm = CacheManager(model, CacheConfig(block_size_tokens=16, key_type="q8_0", value_type="q8_0",
                                         group_size=32, memory_budget_bytes=1 << 30))
    handles = [cm.create_handle(f"r{b}", key_type="q8_0", value_type="q8_0") for b in range(3)]
    host = PagedRunner(model)
    arena = DevicePageArena(PageFormat(2, 64, 16, 8, 32, torch.float16), 64, num_layers=2,
                            max_slots=4, max_tokens=256)
    dev = DeviceRunner(model, arena)
    slots = [arena.open_slot() for _ in range(3)]
    gen = torch.Generator(device="cuda").manual_seed(2)
    for widths in ([40, 17, 3], [1, 1, 1], [5, 1, 9], [1, 1, 1]):
        width = max(widths)
        x = torch.randn((3, width, 256), generator=gen, device="cuda").half()
        for b, n in enumerate(widths):
            x[b, n:] = 0
        got = dev.execute(slots, x, widths)
        phase = "prefill" if width > 1 else "decode"
        out = host.execute([ForwardRequest(None, (), h.bundle.entries, phase=phase,
                                           runtime=cm, handle=h, return_all_logits=True,
                                           request_id=h.request_id, hidden=x[b, :n])
                            for b, (h, n) in enumerate(zip(handles, widths))])
        torch.cuda.synchronize()
        for b, n in enumerate(widths):
            assert torch.equal(got[b, :n], out.logits[b][0]), (widths, b)
    arena.check()
    assert arena.lengths[:3] == [h.token_count for h in handles]

    before = list(arena.lengths)

    class Boom(RuntimeError):
        pass

    def broken(*_a, **_k):
        raise Boom

    forward = model.forward
    model.forward = broken
    with pytest.raises(Boom):
        dev.execute(slots, torch.zeros((3, 1, 256), device="cuda").half())
    model.forward = forward
    arena.sync_lengths()
    assert arena.lengths == before
    _invariants(arena)

    x = torch.randn((3, 1, 256), generator=gen, device="cuda").half()
    step = dev.capture_decode(slots, x)                # one eager step, then the graph
    out = step.out
    host.execute([ForwardRequest(None, (), h.bundle.entries, runtime=cm, handle=h,
                                 request_id=h.request_id, hidden=x[b])
                  for b, h in enumerate(handles)])     # the host runner takes the same step
    # the graph's split-K partials live in a workspace the step holds: dropping
    # and refilling the shared per-device workspace must not reach the replays
    from pkv import ops

    assert step.workspace is not None and step.waves > 0
    assert all(step.workspace is not ws for ws in ops._WORKSPACES.values())
    junk = []
    for i in range(3):
        if i == 1:
            ops._WORKSPACES.clear()
            ops.attention_workspace(torch.device("cuda"), 32 << 20).fill_(255)
            junk.append(torch.full((8 << 20,), -1.0, device="cuda"))
        x.copy_(torch.randn((3, 1, 256), generator=gen, device="cuda").half())
        step.replay()
        ref = host.execute([ForwardRequest(None, (), h.bundle.entries, runtime=cm,
                                           handle=h, request_id=h.request_id,
                                           hidden=x[b]) for b, h in enumerate(handles)])
        torch.cuda.synchronize()
        for b in range(3):
            assert torch.equal(out[b, 0], ref.logits[b][0, 0]), (i, b)
    arena.sync_lengths()
    assert arena.lengths[:3] == [h.token_count for h in handles]
    _invariants(arena)
