"""GPU: ``PagedRunner.execute`` + ``CacheManager`` handles driving attention layers.

A batch goes through prefill (ragged widths) and decode steps; every step's
outputs are checked against a float32 restatement of the same layers on the
CPU (projections rounded to the activation dtype as the GPU GEMMs do, RoPE,
the history quantized and dequantized by the numpy oracle for q8_0 / q4_0
caches, causal GQA attention by the oracle, output projection).
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import numpy_ref

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from pkv import _native

    _native.load()


def _rope(x, positions, inv_freq):
    """x [H, T, D] float32, positions [T] -> rotate-half RoPE (float32)."""
    ang = positions[None, :, None].astype(np.float32) * inv_freq[None, None, :]
    cos, sin = np.cos(ang), np.sin(ang)
    half = x.shape[-1] // 2
    a, b = x[..., :half], x[..., half:]
    return np.concatenate([a * cos - b * sin, b * cos + a * sin], -1).astype(np.float32)


class Reference:
    """float32 CPU restatement of the stack; keeps each request's K/V history."""

    def __init__(self, model, bits, group, batch):
        self.spec, self.bits, self.group = model.spec, bits, group
        self.w = [(l.wq.float().cpu().numpy(), l.wk.float().cpu().numpy(),
                   l.wv.float().cpu().numpy(), l.wo.float().cpu().numpy()) for l in model.layers]
        self.inv = model.layers[0].inv_freq.cpu().numpy()
        s = self.spec
        self.k = [[np.zeros((s.kv_heads, 0, s.head_dim), np.float32) for _ in range(batch)]
                  for _ in model.layers]
        self.v = [[np.zeros((s.kv_heads, 0, s.head_dim), np.float32) for _ in range(batch)]
                  for _ in model.layers]
        self.round = (lambda a: a.astype(np.float16).astype(np.float32)) if s.dtype == "float16" \
            else numpy_ref.bf16_round

    def _seen(self, x):
        if self.bits is None:
            return x
        return numpy_ref.dequantize_page(
            numpy_ref.quantize_page(x.astype(np.float16), self.bits, self.group), self.bits,
            x.shape[-1], self.group).astype(np.float32)

    def step(self, hidden):
        """hidden: list of [T_b, hidden] float32 -> list of outputs [T_b, hidden]."""
        s = self.spec
        xs = [self.round(h) for h in hidden]
        for li, (wq, wk, wv, wo) in enumerate(self.w):
            outs = []
            for b, x in enumerate(xs):
                t = x.shape[0]
                start = self.k[li][b].shape[1]
                pos = np.arange(start, start + t)
                q = self.round(x @ wq).reshape(t, s.query_heads, s.head_dim).transpose(1, 0, 2)
                k = self.round(x @ wk).reshape(t, s.kv_heads, s.head_dim).transpose(1, 0, 2)
                v = self.round(x @ wv).reshape(t, s.kv_heads, s.head_dim).transpose(1, 0, 2)
                q, k = self.round(_rope(q, pos, self.inv)), self.round(_rope(k, pos, self.inv))
                self.k[li][b] = np.concatenate([self.k[li][b], self._seen(k)], 1)
                self.v[li][b] = np.concatenate([self.v[li][b], self._seen(v)], 1)
                att = numpy_ref.paged_attention(q[None], [self.k[li][b]], [self.v[li][b]],
                                                [pos], [t], scale=1.0 / math.sqrt(s.head_dim))
                att = self.round(att[0].astype(np.float32)).transpose(1, 0, 2).reshape(t, -1)
                outs.append(self.round(att @ wo))
            xs = outs
        return xs


def _close(got, want, max_rel, mean_rel):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    scale = float(np.abs(want).max()) + 1e-6
    err = np.abs(got - want) / scale
    assert np.isfinite(got).all()
    assert err.max() <= max_rel, f"max rel error {err.max():.3e}"
    assert err.mean() <= mean_rel, f"mean rel error {err.mean():.3e}"


CASES = {
    # name: (spec kwargs, key type, prefill widths, decode steps, block tokens, max_rel)
    "small_f16": (dict(hidden=256, query_heads=8, kv_heads=2, head_dim=64, num_layers=2,
                       dtype="float16"), "f16", (37, 5, 20), 3, 16, 2e-2),
    "small_bf16": (dict(hidden=256, query_heads=8, kv_heads=2, head_dim=64, num_layers=2,
                        dtype="bfloat16"), "bf16", (17, 33), 2, 32, 3e-2),
    "small_q8": (dict(hidden=256, query_heads=8, kv_heads=2, head_dim=64, num_layers=2,
                      dtype="float16"), "q8_0", (37, 5, 20), 3, 16, 2e-2),
    "small_q4": (dict(hidden=256, query_heads=8, kv_heads=2, head_dim=64, num_layers=2,
                      dtype="float16"), "q4_0", (24, 9), 2, 16, 4e-2),
    "llama3_8b_layer_q8": (dict(num_layers=1, dtype="float16"), "q8_0", (40, 3), 2, 16, 2e-2),
}


@pytest.mark.parametrize("copy_on_write", [False, True])
@pytest.mark.parametrize("case", sorted(CASES))
def test_runner_prefill_then_decode_matches_reference(case, copy_on_write):
    from pkv.cache_manager import CacheConfig, CacheManager
    from pkv.layer import AttentionStack, ModelSpec
    from pkv.runner import ForwardRequest, PagedRunner

    kw, key_type, prefill, steps, block, max_rel = CASES[case]
    spec = ModelSpec(**kw)
    model = AttentionStack(spec, seed=3)
    cm = CacheManager(model, CacheConfig(block_size_tokens=block, key_type=key_type,
                                         value_type=key_type, memory_budget_bytes=1 << 30))
    handles = [cm.create_handle(f"r{i}", key_type=key_type, value_type=key_type)
               for i in range(len(prefill))]
    bits = {"q8_0": 8, "q4_0": 4}.get(key_type)
    ref = Reference(model, bits, 32, len(prefill))
    runner = PagedRunner(model, copy_on_write=copy_on_write)
    rng = np.random.default_rng(11)
    dtype = getattr(torch, spec.dtype)
    widths_seq = [prefill] + [(1,) * len(prefill)] * steps
    for step, widths in enumerate(widths_seq):
        hidden = [rng.standard_normal((w, spec.hidden)).astype(np.float32) for w in widths]
        reqs = [ForwardRequest(None, (), h.bundle.entries, phase="prefill" if step == 0 else "decode",
                               runtime=cm, handle=h, return_all_logits=step == 0,
                               request_id=h.request_id,
                               hidden=torch.from_numpy(x).to("cuda", dtype))
                for h, x in zip(handles, hidden)]
        out = runner.execute(reqs)
        want = ref.step(hidden)
        assert out.committed_token_counts == tuple(widths)
        for i, w in enumerate(widths):
            got = out.logits[i][0].float().cpu().numpy()
            _close(got, want[i][-got.shape[0]:], max_rel, max_rel / 10)
        offsets = [sum(ws[i] for ws in widths_seq[:step + 1]) for i in range(len(prefill))]
        assert [h.token_count for h in handles] == offsets
        assert [h.bundle.offset for h in handles] == offsets
    for h in handles:
        cm.release(h)
    assert cm.stats().live_handles == 0


class _FailAfterFirstLayer:
    """A stack that raises after its first layer has appended and attended."""

    def __init__(self, model):
        self.model, self.spec, self.activation_dtype = model, model.spec, model.activation_dtype

    def forward(self, x, *, cache, position_ids):
        self.model.layers[0](x, cache[0], position_ids)
        raise RuntimeError("planted failure")


@pytest.mark.parametrize("copy_on_write", [False, True])
def test_failed_step_leaves_caches_unchanged(copy_on_write):
    """A step that fails mid-way rolls back (or drops its clones); the next step
    matches a reference that never saw it."""
    from pkv.cache_manager import CacheConfig, CacheManager
    from pkv.layer import AttentionStack, ModelSpec
    from pkv.runner import ForwardRequest, PagedRunner

    spec = ModelSpec(hidden=256, query_heads=8, kv_heads=2, head_dim=64, num_layers=2,
                     dtype="float16")
    model = AttentionStack(spec, seed=5)
    cm = CacheManager(model, CacheConfig(block_size_tokens=16, key_type="q8_0",
                                         value_type="q8_0"))
    handles = [cm.create_handle(f"r{i}", key_type="q8_0", value_type="q8_0") for i in range(2)]
    ref = Reference(model, 8, 32, 2)
    good, bad = PagedRunner(model, copy_on_write=copy_on_write), PagedRunner(
        _FailAfterFirstLayer(model), copy_on_write=copy_on_write)
    rng = np.random.default_rng(5)

    def requests(widths, phase):
        hidden = [rng.standard_normal((w, spec.hidden)).astype(np.float32) for w in widths]
        return hidden, [ForwardRequest(None, (), h.bundle.entries, phase=phase, runtime=cm,
                                       handle=h, request_id=h.request_id,
                                       hidden=torch.from_numpy(x).to("cuda", torch.float16))
                        for h, x in zip(handles, hidden)]

    hidden, reqs = requests((15, 16), "prefill")   # a partial page and a page just filled
    good.execute(reqs)
    ref.step(hidden)
    state = [[(c.offset, len(c._blocks), list(c.page_table.pages)) for c in h.bundle.entries]
             for h in handles]
    _, reqs = requests((1, 1), "decode")
    with pytest.raises(RuntimeError, match="planted failure"):
        bad.execute(reqs)
    assert [[(c.offset, len(c._blocks), list(c.page_table.pages)) for c in h.bundle.entries]
            for h in handles] == state
    assert [h.token_count for h in handles] == [15, 16]
    hidden, reqs = requests((1, 1), "decode")
    out = good.execute(reqs)
    want = ref.step(hidden)
    for i in range(2):
        _close(out.logits[i][0].float().cpu().numpy(), want[i][-1:], 2e-2, 2e-3)


def test_adopted_prefix_pages_give_the_same_steps_as_computed_ones():
    """Request B adopts the prefix pages request A published; request C computes
    the same prompt itself.  Same chunks, same shapes: B's and C's later steps
    must agree bit for bit (the shared pages are A's, which equal C's)."""
    from pkv.cache_manager import CacheConfig, CacheManager
    from pkv.layer import AttentionStack, ModelSpec
    from pkv.runner import ForwardRequest, PagedRunner

    spec = ModelSpec(hidden=256, query_heads=8, kv_heads=2, head_dim=64, num_layers=2,
                     dtype="float16")
    model = AttentionStack(spec, device="cuda", seed=9)
    cm = CacheManager(model, CacheConfig(block_size_tokens=16, key_type="q8_0", value_type="q8_0",
                                         group_size=32, prefix_cache_enabled=True,
                                         memory_budget_bytes=1 << 30))
    fp = cm.fingerprint(key_type="q8_0", value_type="q8_0")
    runner = PagedRunner(model)
    gen = torch.Generator(device="cuda").manual_seed(4)
    prompt = tuple(range(500, 553))                          # 53 tokens: 3 pages + 5
    hidden = torch.randn((53, 256), generator=gen, device="cuda").half()

    def run(handle, x, phase):
        return runner.execute([ForwardRequest(None, (), handle.bundle.entries,
                                              phase=phase, runtime=cm, handle=handle,
                                              request_id=handle.request_id, hidden=x)])

    a = cm.create_handle("a", key_type="q8_0", value_type="q8_0")
    c = cm.create_handle("c", key_type="q8_0", value_type="q8_0")
    for h in (a, c):
        run(h, hidden[:48], "prefill")
        run(h, hidden[48:], "prefill")
    assert cm.publish_prefix(a, fp, prompt)
    b = cm.create_handle("b", key_type="q8_0", value_type="q8_0")
    assert cm.adopt_prefix(b, fp, prompt) == 48
    assert [r.block_id for r in b.bundle.entries[0]._blocks] == \
        [r.block_id for r in a.bundle.entries[0]._blocks[:3]]
    run(b, hidden[48:], "prefill")
    cm.release(a)                                            # B keeps A's pages alive
    for _ in range(3):
        x = torch.randn((1, 256), generator=gen, device="cuda").half()
        out_b, out_c = run(b, x, "decode"), run(c, x, "decode")
        torch.cuda.synchronize()
        assert torch.equal(out_b.logits[0], out_c.logits[0])
    assert b.token_count == c.token_count == 56


def test_snapshot_restore_gives_the_same_steps(tmp_path):
    """A request's caches saved to disk and restored into a fresh arena take the
    next steps exactly as the originals do; the reference-format export equals
    gather_pages of the same pages."""
    from pkv import ops
    from pkv.cache_manager import CacheConfig, CacheManager
    from pkv.layer import AttentionStack, ModelSpec
    from pkv.runner import ForwardRequest, PagedRunner
    from pkv.snapshot import load_snapshot, save_snapshot

    spec = ModelSpec(hidden=256, query_heads=8, kv_heads=2, head_dim=64, num_layers=2,
                     dtype="float16")
    model = AttentionStack(spec, device="cuda", seed=11)
    config = CacheConfig(block_size_tokens=16, key_type="q4_0", value_type="q4_0", group_size=32,
                         memory_budget_bytes=1 << 30)
    cm, cm2 = CacheManager(model, config), CacheManager(model, config)
    runner = PagedRunner(model)
    gen = torch.Generator(device="cuda").manual_seed(6)
    a = cm.create_handle("a", key_type="q4_0", value_type="q4_0")
    runner.execute([ForwardRequest(None, (), a.bundle.entries, phase="prefill", runtime=cm,
                                   handle=a, request_id="a",
                                   hidden=torch.randn((45, 256), generator=gen, device="cuda").half())])
    manifest = save_snapshot(tmp_path, a.bundle, identity="m", reference_pages=True)
    restored = load_snapshot(tmp_path, identity="m", expected_specs=cm2.layer_specs,
                             page_pool=cm2.block_pool, bits=4)
    b = cm2.create_handle("b", key_type="q4_0", value_type="q4_0")
    for entry in b.bundle.entries:
        entry.reset()
    b.bundle = restored
    b.token_count = restored.offset
    # the reference-format pages in the payload, before any step writes more tokens
    data = np.load(tmp_path / manifest["payload"])
    cache = restored.entries[0]
    pool = cache.pool.pool_for(cache.layout)
    ids = torch.tensor([r.block.page for r in cache._blocks], dtype=torch.int32, device="cuda")
    exported = ops.gather_pages(pool.fmt, pool.buffer, ids)
    for name, value in zip(("k_codes", "k_scale", "k_bias", "v_codes", "v_scale", "v_bias"),
                           exported, strict=True):
        assert np.array_equal(data[f"layer_0_reference_{name}"], value.cpu().numpy()), name
    for _ in range(3):
        x = torch.randn((1, 256), generator=gen, device="cuda").half()
        out_a = runner.execute([ForwardRequest(None, (), a.bundle.entries, runtime=cm, handle=a,
                                               request_id="a", hidden=x)])
        out_b = runner.execute([ForwardRequest(None, (), b.bundle.entries, runtime=cm2, handle=b,
                                               request_id="b", hidden=x)])
        torch.cuda.synchronize()
        assert torch.equal(out_a.logits[0], out_b.logits[0])


@pytest.mark.parametrize("copy_on_write", [False, True])
def test_every_page_allocation_of_a_step_rolls_back(copy_on_write, monkeypatch):
    """The reference's allocation sweep (tests/test_paged_hybrid.py:349-374): a
    request with a few cached tokens takes a 32-token step through a 3-layer
    stack; a failure injected at each page allocation of the step in turn
    leaves offsets, live blocks, page tables and reservations unchanged, and
    the next step equals the same step on a manager that never failed."""
    from pkv.cache_manager import CacheConfig, CacheManager
    from pkv.layer import AttentionStack, ModelSpec
    from pkv.runner import ForwardRequest, PagedRunner

    spec = ModelSpec(hidden=256, query_heads=8, kv_heads=2, head_dim=64, num_layers=3,
                     dtype="float16")
    model = AttentionStack(spec, seed=8)
    config = CacheConfig(block_size_tokens=16, key_type="q8_0", value_type="q8_0",
                         memory_budget_bytes=1 << 30)
    gen = torch.Generator(device="cuda").manual_seed(8)
    first = torch.randn((2, 256), generator=gen, device="cuda").half()
    step = torch.randn((32, 256), generator=gen, device="cuda").half()
    nxt = torch.randn((1, 256), generator=gen, device="cuda").half()
    runner = PagedRunner(model, copy_on_write=copy_on_write)

    def fresh():
        cm = CacheManager(model, config)
        h = cm.create_handle("r", key_type="q8_0", value_type="q8_0")
        runner.execute([ForwardRequest(None, (), h.bundle.entries, phase="prefill",
                                       runtime=cm, handle=h, request_id="r", hidden=first)])
        return cm, h

    def run(cm, h, x):
        return runner.execute([ForwardRequest(None, (), h.bundle.entries, phase="prefill",
                                              runtime=cm, handle=h, return_all_logits=True,
                                              request_id="r", hidden=x)])

    # the untouched twin, and the number of allocations the step makes
    cm0, h0 = fresh()
    calls = [0]
    original = cm0.block_pool.allocate_ref

    def counting(*a, **k):
        calls[0] += 1
        return original(*a, **k)

    monkeypatch.setattr(cm0.block_pool, "allocate_ref", counting)
    run(cm0, h0, step)
    monkeypatch.undo()
    total = calls[0]
    assert total == (9 if copy_on_write else 6)     # clones' tails + two new pages per layer
    want = run(cm0, h0, nxt).logits[0]
    for fail_at in range(1, total + 1):
        cm, h = fresh()
        state = [(c.offset, [r.block_id for r in c._blocks], list(c.page_table.pages))
                 for c in h.bundle.entries]
        live = cm.block_pool.stats()["block_live"]
        count, base = [0], cm.block_pool.allocate_ref

        def failing(*a, **k):
            count[0] += 1
            if count[0] == fail_at:
                raise MemoryError("injected page allocation")
            return base(*a, **k)

        cm.block_pool.allocate_ref = failing
        with pytest.raises(MemoryError, match="allocation"):
            run(cm, h, step)
        cm.block_pool.allocate_ref = base
        assert [(c.offset, [r.block_id for r in c._blocks], list(c.page_table.pages))
                for c in h.bundle.entries] == state, fail_at
        assert cm.block_pool.stats()["block_live"] == live
        assert h.token_count == 2
        stats = cm.stats()
        assert stats.reserved_bytes == 0 and stats.transient_bytes == 0
        run(cm, h, step)
        got = run(cm, h, nxt).logits[0]
        torch.cuda.synchronize()
        assert torch.equal(got, want), fail_at


def test_device_runner_out_of_pages_at_every_point_changes_nothing():
    """The device arena's counterpart: a step needing N new pages with only
    k - 1 free (k = 1..N) sets the out-of-pages bit, ``execute`` raises
    CacheCapacityError, and lengths (device and host mirror), tables,
    reference counts and the free stack stay as they were."""
    from pkv.cache_errors import CacheCapacityError
    from pkv.device_arena import DevicePageArena, DeviceRunner
    from pkv.layer import AttentionStack, ModelSpec
    from pkv.ops import PageFormat

    spec = ModelSpec(hidden=256, query_heads=8, kv_heads=2, head_dim=64, num_layers=2,
                     dtype="float16")
    model = AttentionStack(spec, device="cuda", seed=4)
    fmt = PageFormat(2, 64, 16, 8, 32, torch.float16)
    gen = torch.Generator(device="cuda").manual_seed(4)
    x0 = torch.randn((2, 20, 256), generator=gen, device="cuda").half()
    x1 = torch.randn((2, 40, 256), generator=gen, device="cuda").half()
    # after the 20-token prefill each slot holds 2 pages; 40 more tokens need
    # 2 more pages per slot: N = 4
    for free in range(0, 4):
        arena = DevicePageArena(fmt, 4 + free, num_layers=2, max_slots=2, max_tokens=256)
        runner = DeviceRunner(model, arena)
        slots = [arena.open_slot() for _ in range(2)]
        runner.execute(slots, x0)
        assert arena.check() == free
        lens, table = arena.lens.clone(), arena.table.clone()
        refs, stack = arena.refcounts(), arena.free_stack()
        mirror = list(arena.lengths)
        with pytest.raises(CacheCapacityError):
            runner.execute(slots, x1)
        assert arena.check() == free                   # the error bit was taken and cleared
        assert arena.lengths == mirror
        assert torch.equal(arena.lens, lens) and torch.equal(arena.table, table)
        assert torch.equal(arena.refcounts(), refs) and torch.equal(arena.free_stack(), stack)


@pytest.mark.parametrize("page_arena", ["host", "device"])
def test_reference_style_requests_trace_and_cancellation(page_arena):
    """The reference's runner tests with the real kernels, on both arenas:
    requests built positionally from token ids (the model embeds them) run
    under ``PagedRunner()``, which takes the model from the bundle, and give
    the outputs of the same steps fed as hidden states, bit for bit; the trace
    carries the reference's keys (``tests/test_paged_hybrid.py:162-163``,
    ``tests/test_p1_runtime.py:517``); a request cancelled while its forward
    runs keeps its caches (``tests/test_paged_hybrid.py:183-186``), so its next
    step gives what it gives in a run where the cancelled step never happened."""
    import threading

    from pkv.cache_manager import CacheConfig, CacheManager
    from pkv.layer import AttentionStack, ModelSpec
    from pkv.runner import ForwardRequest, PagedRunner

    spec = ModelSpec(hidden=256, query_heads=8, kv_heads=2, head_dim=64, num_layers=2,
                     dtype="float16", vocab_size=1000)
    model = AttentionStack(spec, device="cuda", seed=7)

    def manager():
        return CacheManager(model, CacheConfig(block_size_tokens=16, key_type="q8_0",
                                               value_type="q8_0", group_size=32,
                                               memory_budget_bytes=1 << 26, page_arena=page_arena,
                                               max_sequences=4, max_sequence_tokens=256))

    prompts = [tuple(range(1, 18)), (4, 5, 6)]
    cm_t, cm_h, cm_c = manager(), manager(), manager()
    by_tokens, by_hidden, clean = [], [], []
    for i, ids in enumerate(prompts):
        for cm, out in ((cm_t, by_tokens), (cm_h, by_hidden), (cm_c, clean)):
            h = cm.create_handle(str(i), key_type="q8_0", value_type="q8_0")
            out.append(ForwardRequest(model, ids, h.bundle.entries, "prefill", ids, cm, h,
                                      request_id=str(i)))
    for r in by_hidden:
        r.hidden = model.embed(r.token_ids)
    runner, runner_h, runner_c = PagedRunner(), PagedRunner(), PagedRunner()

    def step(requests, rn, tokens=None):
        if tokens is not None:
            for r in requests:
                r.phase, r.token_ids = "decode", tokens
                if r.hidden is not None:
                    r.hidden = model.embed(tokens)
        return rn.execute(tuple(requests))

    a, b = step(by_tokens, runner), step(by_hidden, runner_h)
    step(clean, runner_c)
    torch.cuda.synchronize()
    for x, y in zip(a.logits, b.logits):
        assert torch.equal(x, y)
    trace = runner.last_trace
    assert trace["history_materializations"] == 0 and trace["direct_attention_calls"] == 2
    assert trace["history_lengths"] == [0, 0] and trace["layer_layouts"][1]["key_dim"] == 64
    for k in range(2):
        a, b = step(by_tokens, runner, (9 + k,)), step(by_hidden, runner_h, (9 + k,))
        step(clean, runner_c, (9 + k,))
        torch.cuda.synchronize()
        for x, y in zip(a.logits, b.logits):
            assert torch.equal(x, y), k
        assert runner.last_trace["history_lengths"] == [17 + k, 3 + k]
        assert runner.last_trace["history_materializations"] == 0
    before = [r.cache[0].offset for r in by_tokens]
    by_tokens[0].cancel = threading.Event()
    forward = model.forward

    def cancelling(*args, **kwargs):
        out = forward(*args, **kwargs)
        by_tokens[0].cancel.set()
        return out

    model.forward = cancelling
    try:
        step(by_tokens, runner, (40,))
    finally:
        model.forward = forward
    assert [r.cache[0].offset for r in by_tokens] == [before[0], before[1] + 1]
    assert by_tokens[0].handle.token_count == before[0]
    assert runner.last_trace["cancelled_request_ids"] == ["0"]
    # the clean run: request 1 takes the step request 0 missed, alone
    clean[1].phase, clean[1].token_ids = "decode", (40,)
    runner_c.execute((clean[1],))
    by_tokens[0].cancel = None
    a, c = step(by_tokens, runner, (41,)), step(clean, runner_c, (41,))
    torch.cuda.synchronize()
    assert [r.cache[0].offset for r in by_tokens] == [r.cache[0].offset for r in clean]
    # request 0's caches saw the same steps in both runs: the same bits
    assert torch.equal(a.logits[0], c.logits[0])
    # request 1 took token 40 in a batch of one in the clean run, where the
    # projection GEMM may round differently
    torch.testing.assert_close(a.logits[1], c.logits[1], atol=2e-2, rtol=0)
