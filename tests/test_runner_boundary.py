"""Host logic of ``PagedRunner`` at the reference's boundary (no GPU).

The reference builds requests positionally -- ``ForwardRequest(bundle,
token_ids, cache, phase, prompt_ids, runtime, handle, request_id=...)``
(``tests/test_paged_hybrid.py:132-138``, ``engine/batching.py:49-65``) -- runs
``PagedRunner()`` without a model (it takes the batch's bundle), reads
``last_trace`` (``tests/test_paged_hybrid.py:162-163``,
``tests/test_paged_architectures.py:62-63``, ``tests/test_p1_runtime.py:196,
325, 517``) and cancels a request while its forward runs, after which that
request's caches keep their length and the others commit
(``tests/test_paged_hybrid.py:170-187``, ``engine/transactions.py:79-82``).

Both runner paths are driven here with their kernel launches stubbed out:
the host path's append, tail-copy and attention calls do nothing (the
attention returns zeros), and the device
path's arena and step runner are host stand-ins that only move lengths.
Everything else -- validation, page planning, transactions, the trace -- is
the product code.  ``tests/test_gpu_runner.py`` repeats the assertions with
the real kernels.
"""

from __future__ import annotations

import threading
import time

import pytest

torch = pytest.importorskip("torch")

from pkv.cache_manager import CacheConfig, CacheManager  # noqa: E402
from pkv.layer import ModelSpec  # noqa: E402
from pkv.runner import ForwardRequest, PagedRunner, request_cancelled  # noqa: E402

# the reference's trace keys (engine/paged.py:348-350, 406-416)
TRACE_KEYS = {"direct_attention_calls", "history_materializations", "conversion_bytes",
              "kernel_version", "synchronized_kernel_dispatch_ms", "gpu_timestamp_latency_ms",
              "arena", "phase", "request_ids", "batch_size", "history_lengths", "real_tokens",
              "padded_tokens", "padding_efficiency", "transient_reserved_bytes",
              "layer_layouts", "adapter_transient_bound_bytes", "duration_ms"}


class _StubModel:
    """The attention stack's interface (spec, activation dtype, embed, forward)
    on the CPU: each layer calls ``cache.attend`` with zero q/k/v, and
    ``pause`` (if set) runs during the forward, as the reference's test
    model's does."""

    def __init__(self, spec):
        self.spec, self.activation_dtype = spec, spec.dtype
        self.pause = None
        self.calls = []

    def embed(self, token_ids):
        return torch.full((len(token_ids), self.spec.hidden), 0.5, dtype=torch.float16)

    def forward(self, x, *, cache, position_ids):
        s = self.spec
        batch, width, _ = x.shape
        self.calls.append((batch, width))
        for layer in cache:
            q = torch.zeros((batch, s.query_heads, width, s.head_dim), dtype=torch.float16)
            kv = torch.zeros((batch, s.kv_heads, width, s.head_dim), dtype=torch.float16)
            layer.attend(q, kv, kv, scale=0.125, position_ids=position_ids)
        if self.pause is not None:
            self.pause()
        return x + 1


@pytest.fixture
def host_stubs(monkeypatch):
    """The host path's kernel calls (append, tail copy, attention), replaced by
    no-ops; the attention returns zeros."""
    import pkv.ops as ops
    import pkv.paged_attention as pa

    monkeypatch.setattr(ops, "append_quantize", lambda *a, **k: None)
    monkeypatch.setattr(ops, "copy_pages", lambda *a, **k: None)
    monkeypatch.setattr(pa, "paged_attention", lambda queries, *a, **k: torch.zeros_like(queries))


def _host_setup(num_layers=2, key_dim=64):
    spec = ModelSpec(hidden=256, query_heads=8, kv_heads=2, head_dim=key_dim,
                     num_layers=num_layers, dtype="float16")
    model = _StubModel(spec)
    cm = CacheManager(model, CacheConfig(block_size_tokens=16, key_type="q8_0",
                                         value_type="q8_0"), device="cpu")
    return model, cm


def _requests(model, cm, prompts):
    """The reference's helper, argument for argument (tests/test_paged_hybrid.py:132-138)."""
    out = []
    for i, ids in enumerate(prompts):
        h = cm.create_handle(str(i), key_type="q8_0", value_type="q8_0")
        out.append(ForwardRequest(model, tuple(ids), h.bundle.entries, "prefill", tuple(ids), cm,
                                  h, request_id=str(i)))
    return out


def test_forward_request_takes_the_reference_fields_in_order():
    names = [f for f in ForwardRequest.__dataclass_fields__]
    assert names[:15] == ["bundle", "token_ids", "cache", "phase", "prompt_ids", "runtime",
                          "handle", "request_id", "model_epoch", "cancel", "options", "deadline",
                          "return_all_logits", "staged_verification", "generated_ids"]
    r = ForwardRequest("m", (1, 2, 3), (), "prefill", (1, 2, 3), None, None, request_id="x")
    assert r.width == 3 and r.phase == "prefill" and r.request_id == "x"
    r.phase, r.token_ids = "decode", (9,)           # requests are mutable, as the reference's
    assert r.width == 1
    assert ForwardRequest(hidden=torch.zeros((4, 8))).width == 4


def test_request_cancelled_follows_the_flag_and_the_deadline():
    r = ForwardRequest()
    assert not request_cancelled(r)
    r.cancel = threading.Event()
    assert not request_cancelled(r)
    r.deadline = time.monotonic() - 1.0
    assert request_cancelled(r) and r.cancel.is_set()   # a passed deadline sets the flag
    r2 = ForwardRequest(deadline=time.monotonic() + 60.0)
    assert not request_cancelled(r2)
    r2.cancel = threading.Event()
    r2.cancel.set()
    assert request_cancelled(r2)


@pytest.mark.parametrize("copy_on_write", [False, True])
def test_host_runner_trace_tokens_and_cancellation(host_stubs, copy_on_write):
    model, cm = _host_setup()
    requests = _requests(model, cm, [range(1, 18), (4, 5, 6)])
    runner = PagedRunner(copy_on_write=copy_on_write)   # the model comes from the bundle
    out = runner.execute(tuple(requests))
    assert model.calls[-1] == (2, 17)
    assert [tuple(x.shape) for x in out.logits] == [(1, 1, 256), (1, 1, 256)]
    trace = runner.last_trace
    assert TRACE_KEYS <= set(trace)
    assert trace["history_materializations"] == 0 and trace["conversion_bytes"] == 0
    assert trace["direct_attention_calls"] == 2
    assert trace["history_lengths"] == [0, 0] and trace["request_ids"] == ["0", "1"]
    assert trace["real_tokens"] == 20 and trace["padded_tokens"] == 34
    assert trace["padding_efficiency"] == pytest.approx(20 / 34)
    assert trace["layer_layouts"][1]["key_dim"] == 64 and trace["phase"] == "prefill"
    assert [r.cache[0].offset for r in requests] == [17, 3]
    for step in range(2):
        for r in requests:
            r.phase, r.token_ids = "decode", (step + 9,)
        runner.execute(tuple(requests))
        assert runner.last_trace["history_lengths"] == [17 + step, 3 + step]
        assert runner.last_trace["history_materializations"] == 0
    before = [r.cache[0].offset for r in requests]
    pages = [[ref.block_id for ref in c._blocks] for c in requests[0].cache]
    requests[0].cancel = threading.Event()
    model.pause = requests[0].cancel.set             # cancelled while its forward runs
    out = runner.execute(tuple(requests))
    assert [r.cache[0].offset for r in requests] == [before[0], before[1] + 1]
    assert all(c.offset == before[0] for c in requests[0].cache)
    assert [[ref.block_id for ref in c._blocks] for c in requests[0].cache] == pages
    assert requests[0].handle.token_count == before[0]
    assert out.committed_token_counts == (1, 1)      # as the reference reports them
    assert runner.last_trace["cancelled_request_ids"] == ["0"]
    # a passed deadline counts as cancellation
    model.pause = None
    requests[0].cancel = None
    requests[1].deadline = time.monotonic() - 1.0
    runner.execute(tuple(requests))
    assert [r.cache[0].offset for r in requests] == [before[0] + 1, before[1] + 1]


def test_runner_takes_one_model_per_batch(host_stubs):
    model, cm = _host_setup()
    other = _StubModel(model.spec)
    a, b = _requests(model, cm, [(1, 2), (3,)])
    with pytest.raises(ValueError):
        PagedRunner().execute((a, ForwardRequest(other, (3,), b.cache, "prefill", (3,), cm,
                                                 b.handle, request_id="1")))
    with pytest.raises(ValueError):                  # a runner model and another bundle
        PagedRunner(other).execute((a, b))
    with pytest.raises(ValueError):                  # no model anywhere
        PagedRunner().execute((ForwardRequest(None, (1,), a.cache, "prefill", (1,), cm,
                                              a.handle, request_id="0"),))
    with pytest.raises(ValueError):                  # tokens and hidden states disagree
        PagedRunner().execute((ForwardRequest(model, (1, 2), a.cache, "prefill", (1, 2), cm,
                                              a.handle, request_id="0",
                                              hidden=torch.zeros((3, 256), dtype=torch.float16)),))


# ---- the device-arena path, with host stand-ins for the arena and its step runner


class _FakeArena:
    def __init__(self, slots=4):
        from pkv.ops import PageFormat

        self.fmt = PageFormat(2, 64, 16, 8, 32, torch.float16)
        self.page_tokens, self.capacity, self.max_slots = 16, 64, slots
        self.lengths = [0] * slots

    def truncate(self, slots, keep):
        for s, k in zip(slots, keep):
            assert 0 <= k <= self.lengths[s]
            self.lengths[s] = k


class _FakeDeviceRunner:
    def __init__(self, model, arena):
        self.model, self.arena = model, arena

    def execute(self, slots, x, widths):
        y = self.model.forward(x, cache=(), position_ids=None)
        for s, w in zip(slots, widths):
            self.arena.lengths[s] += w
        return y


def test_device_runner_trace_tokens_and_cancellation(monkeypatch):
    import pkv.device_arena as device_arena
    from pkv.device_cache import SlotLayerCache
    from pkv.paged import _layout

    monkeypatch.setattr(device_arena, "DeviceRunner", _FakeDeviceRunner)
    spec = ModelSpec(hidden=256, query_heads=8, kv_heads=2, head_dim=64, num_layers=2,
                     dtype="float16")
    model = _StubModel(spec)
    arena = _FakeArena()
    requests = []
    for slot, ids in enumerate([range(1, 18), (4, 5, 6)]):
        caches = tuple(SlotLayerCache(arena, slot, layer, "float16", 8, 32,
                                      _layout(layer, 16, 2, 64, "float16", 8, 32))
                       for layer in range(2))
        requests.append(ForwardRequest(model, tuple(ids), caches, "prefill", tuple(ids),
                                       request_id=str(slot)))
    runner = PagedRunner()
    runner.execute(tuple(requests))
    trace = runner.last_trace
    assert TRACE_KEYS <= set(trace) and trace["page_arena"] == "device"
    assert trace["history_materializations"] == 0 and trace["direct_attention_calls"] == 2
    assert trace["history_lengths"] == [0, 0] and trace["request_ids"] == ["0", "1"]
    assert trace["padding_efficiency"] == pytest.approx(20 / 34)
    assert arena.lengths[:2] == [17, 3]
    for r in requests:
        r.phase, r.token_ids = "decode", (9,)
    requests[1].cancel = threading.Event()
    model.pause = requests[1].cancel.set
    runner.execute(tuple(requests))
    assert arena.lengths[:2] == [18, 3]
    assert runner.last_trace["history_lengths"] == [17, 3]
    assert runner.last_trace["cancelled_request_ids"] == ["1"]
