"""``PagedRunner.execute``: a batch step over paged caches (``engine/paged.py:285-417``).

Same checks as the reference, with this build's attention stack as the
model: validate the batch (same model, phase, layer count; every cache a
``PagedKVCache`` of its layer in the model's activation dtype; one pool and
precision), reserve the step's transient bytes on the cache manager, run the
layers over ``PagedBatchCache`` views (append + attention per layer), pick
each request's outputs (all positions for ``return_all_logits``, else the
last).  A failure anywhere leaves the request caches as they were; a request
cancelled (or past its deadline) by the time the forward has run is not
committed (``engine/transactions.py:79-82``), the others are.

Two ways to get that guarantee: the reference's (``copy_on_write=True``:
clone every layer cache -- sealed pages shared, mutable tails copied -- run on
the clones and commit them, :377-403), and the default: append in place and,
on failure or cancellation, roll the caches back to their checkpoint by
length (pages taken released, tail counts restored), which saves the
per-step tail copies.

Requests are the reference's ``ForwardRequest`` (same fields, same order).
The layers take hidden states: a request's ``hidden`` keyword (``[T,
hidden]``) when given, else the model's embedding of ``token_ids``.  The
outputs are the last layer's hidden states (the LM head sits outside the
path).
"""

from __future__ import annotations

import time
from contextlib import ExitStack
from dataclasses import dataclass

import numpy as np

from pkv.modes import ModelCapabilityUnsupported
from pkv.paged import KERNEL_VERSION, PagedBatchCache, PagedKVCache


@dataclass
class ForwardRequest:
    """``engine/batching.py:49-65``: the reference's fields in its order, plus
    ``hidden`` (keyword), the step's layer inputs when the caller has them.
    ``bundle`` is the model (None: the runner's own); ``token_ids`` are the
    step's tokens (only their count is read when ``hidden`` is given)."""

    bundle: object = None
    token_ids: tuple = ()
    cache: tuple = ()
    phase: str = "decode"
    prompt_ids: tuple = ()
    runtime: object = None         # CacheManager
    handle: object = None          # CacheHandle owning ``cache``
    request_id: str = ""
    model_epoch: int = 0
    cancel: object = None          # a threading.Event-like flag (``is_set``, ``set``)
    options: object = None
    deadline: float | None = None  # ``time.monotonic()`` seconds
    return_all_logits: bool = False
    staged_verification: bool = False
    generated_ids: tuple | None = None
    hidden: object = None          # [T, hidden] device tensor, activation dtype

    @property
    def width(self):
        """Tokens of the step."""
        return int(self.hidden.shape[0]) if self.hidden is not None else len(self.token_ids)


def request_cancelled(request):
    """``engine/batching.py:74-78``: a request is cancelled when its flag is
    set or its deadline has passed (which also sets the flag)."""
    late = request.deadline is not None and time.monotonic() >= request.deadline
    if late and request.cancel is not None:
        request.cancel.set()
    return late or bool(request.cancel is not None and request.cancel.is_set())


@dataclass(frozen=True)
class RunnerOutput:
    """``engine/contracts.py:196-210``: per request, its outputs and committed tokens."""

    request_ids: tuple
    logits: tuple                  # per request [1, n or 1, hidden]
    committed_token_counts: tuple

    def __post_init__(self):
        if len(set(self.request_ids)) != len(self.request_ids):
            raise ValueError("runner output request IDs must be unique")
        if len(self.request_ids) != len(self.committed_token_counts):
            raise ValueError("runner output mappings must align")
        if any(count < 0 for count in self.committed_token_counts):
            raise ValueError("committed counts cannot be negative")
        if len(self.logits) != len(self.request_ids):
            raise ValueError("runner logits must align with request IDs")


class PagedRunner:
    """``copy_on_write`` picks the transaction of host-bookkept caches (see the
    module docstring).  Caches of a device arena (``CacheConfig(page_arena=
    "device")``) always run as one ``DeviceRunner`` step, rolled back by
    truncation; with ``graphs=True`` their repeated decode steps (the same
    sequences, one token each) replay a captured HIP graph of the whole step.
    Without a model the runner takes each batch's (``requests[0].bundle``),
    as the reference's ``PagedRunner()`` does."""

    def __init__(self, model=None, *, copy_on_write=False, graphs=False):
        self.model = model
        self.copy_on_write = copy_on_write
        self.graphs = graphs
        self.last_trace = {}
        self._device_runners = {}
        self._captured = {}            # (arena, slots) -> CapturedStep, oldest first
        self.max_graphs = 8
        self._last_signature = None
        self._layouts = None

    def _model_of(self, requests):
        """The batch's model: the runner's, else the requests' common bundle."""
        first = requests[0]
        model = self.model if self.model is not None else first.bundle
        if model is None:
            raise ValueError("paged batch names no model (bundle)")
        for r in requests:
            if r.bundle is not first.bundle or (r.bundle is not None and r.bundle is not model):
                raise ValueError("incompatible paged batch")
        return model

    @staticmethod
    def _inputs(model, requests, widths):
        """``[B, width, hidden]`` layer inputs: each row's ``hidden`` (or its
        tokens embedded by the model), padding columns zero."""
        import torch

        rows = [r.hidden if r.hidden is not None else model.embed(r.token_ids) for r in requests]
        width = max(widths)
        first = rows[0]
        if all(n == width for n in widths) and all(
                x.dtype == first.dtype and x.device == first.device for x in rows):
            return torch.stack(rows)                           # one copy kernel
        x = torch.zeros((len(rows), width, model.spec.hidden), dtype=first.dtype,
                        device=first.device)
        for i, row in enumerate(rows):
            x[i, :widths[i]] = row
        return x

    @staticmethod
    def _check_inputs(model, r):
        if r.hidden is None:
            if not r.token_ids:
                raise ValueError("request has neither tokens nor hidden states")
            return
        if int(r.hidden.shape[0]) < 1 or int(r.hidden.shape[-1]) != model.spec.hidden:
            raise ValueError("request hidden states do not match the model")
        if r.token_ids and len(r.token_ids) != int(r.hidden.shape[0]):
            raise ValueError("request tokens and hidden states differ in length")

    def _trace(self, model, requests, widths, history, transient, started, extra):
        """``last_trace`` with the reference's keys (``engine/paged.py:348-350,
        406-416``): history is never materialised (the kernels read pages in
        place) and nothing is converted; no adapter scratch."""
        width = max(widths)
        if self._layouts is None or self._layouts[0] is not model:
            self._layouts = (model, [vars(layer) for layer in model.spec.layers])
        return {"direct_attention_calls": model.spec.num_layers,
                "history_materializations": 0, "conversion_bytes": 0,
                "kernel_version": KERNEL_VERSION, "synchronized_kernel_dispatch_ms": 0.0,
                "gpu_timestamp_latency_ms": None, **extra,
                "phase": requests[0].phase,
                "request_ids": [r.request_id for r in requests],
                "batch_size": len(requests), "history_lengths": history,
                "real_tokens": sum(widths), "padded_tokens": len(requests) * width,
                "padding_efficiency": sum(widths) / (len(requests) * width),
                "transient_reserved_bytes": transient,
                "layer_layouts": self._layouts[1],
                "adapter_transient_bound_bytes": 0,
                "duration_ms": (time.perf_counter() - started) * 1000}

    @staticmethod
    def _transient(model, batch, width):
        """Transient bytes of a step: activations and projections per layer."""
        spec = model.spec
        return batch * width * spec.num_layers * 4 * (
            spec.hidden + (spec.query_heads + 2 * spec.kv_heads) * spec.head_dim) * 2

    def _validate(self, model, requests):
        """The reference's batch checks (``paged.py:308-345``), one pass per request."""
        first = requests[0]
        layers = model.spec.layers
        activation = model.activation_dtype
        pool_key = None
        for r in requests:
            caches = r.cache
            if r.phase != first.phase or r.model_epoch != first.model_epoch \
                    or len(caches) != len(first.cache):
                raise ValueError("incompatible paged batch")
            if not caches or len(caches) != len(layers):
                raise ValueError("invalid paged layer mappings")
            offset = caches[0].offset if isinstance(caches[0], PagedKVCache) else None
            for i, c in enumerate(caches):
                if not isinstance(c, PagedKVCache) or c.offset != offset or c.layer_id != i:
                    raise ValueError("invalid paged layer mappings")
            if r.handle is not None:
                r.runtime._validate_handle(r.handle)
                if r.handle.bundle.entries is not caches:
                    raise ValueError("paged request does not own its cache mapping")
            self._check_inputs(model, r)
            for cache, layout in zip(caches, layers):
                if cache.dtype != activation:
                    raise ModelCapabilityUnsupported("paged storage differs from execution precision")
                # one layout per cache (append and adopt enforce it): its first page's
                stored = cache.layout
                if stored is not None and (stored.num_kv_heads != layout.kv_heads
                                           or stored.head_dim != layout.key_dim
                                           or stored.layer_id != layout.layer_id):
                    raise ValueError("paged layer layout differs from the model")
                key = (id(cache.pool), cache.dtype, cache.bits)
                if pool_key is None:
                    pool_key = key
                elif key != pool_key:
                    raise ValueError("incompatible paged pools or precision")
            if r.runtime is not first.runtime:
                raise ValueError("paged batch spans cache managers")

    # -- device-arena batches -------------------------------------------------------------
    def _validate_device(self, model, requests):
        """The reference's batch checks for slot-backed caches: one arena, one
        slot per request across its layers, layouts of the model."""
        from pkv.device_cache import SlotLayerCache

        first = requests[0]
        layers = model.spec.layers
        activation = model.activation_dtype
        arena = first.cache[0].arena
        slots = set()
        for r in requests:
            caches = r.cache
            if r.phase != first.phase or r.model_epoch != first.model_epoch \
                    or len(caches) != len(layers):
                raise ValueError("incompatible paged batch")
            slot = caches[0].slot if isinstance(caches[0], SlotLayerCache) else None
            for i, c in enumerate(caches):
                if (not isinstance(c, SlotLayerCache) or c.slot != slot or c.layer_id != i
                        or c.arena is not arena):
                    raise ValueError("invalid paged layer mappings")
                if c.dtype != activation:
                    raise ModelCapabilityUnsupported("paged storage differs from execution precision")
                lay = c.layout
                if lay.num_kv_heads != layers[i].kv_heads or lay.head_dim != layers[i].key_dim:
                    raise ValueError("paged layer layout differs from the model")
            if slot in slots:
                raise ValueError("a sequence appears twice in the batch")
            slots.add(slot)
            if r.handle is not None:
                r.runtime._validate_handle(r.handle)
                if r.handle.bundle.entries is not caches:
                    raise ValueError("paged request does not own its cache mapping")
            self._check_inputs(model, r)
            if r.runtime is not first.runtime:
                raise ValueError("paged batch spans cache managers")
        return arena

    def _execute_device(self, model, requests):
        from pkv.device_arena import DeviceRunner

        # a batch of the same caches as the last one skips the per-layer
        # checks (the caches of a handle never change); handles are re-checked
        signature = tuple((id(r.cache), id(r.handle), r.phase, r.model_epoch) for r in requests)
        if signature == self._last_signature and all(
                r.handle is None or (not r.handle.closed and r.handle.bundle.entries is r.cache)
                for r in requests) and all(
                r.hidden is None or (int(r.hidden.shape[-1]) == model.spec.hidden
                                     and int(r.hidden.shape[0]) >= 1)
                for r in requests):
            arena = requests[0].cache[0].arena
        else:
            arena = self._validate_device(model, requests)
            self._last_signature = signature
        first = requests[0]
        started = time.perf_counter()
        widths = tuple(r.width for r in requests)
        width = max(widths)
        slots = [r.cache[0].slot for r in requests]
        history = [arena.lengths[s] for s in slots]
        runner = self._device_runners.get(id(arena))
        if runner is None or runner.arena is not arena or runner.model is not model:
            runner = self._device_runners[id(arena)] = DeviceRunner(model, arena)
        transient = self._transient(model, len(requests), width)
        uniform = all(n == width for n in widths)
        replayed = bool(self.graphs and width == 1 and uniform)
        with ExitStack() as stack:
            if first.runtime is not None:
                stack.enter_context(first.runtime.transient_reservation(transient))
            key = (id(arena), tuple(slots))
            if replayed:
                y = self._replay_decode(runner, key, slots, requests)
            else:
                y = runner.execute(slots, self._inputs(model, requests, widths), widths)
            # cancelled (or late) requests keep their length before the step
            dropped = [(s, n) for r, s, n in zip(requests, slots, history) if request_cancelled(r)]
            if dropped:
                arena.truncate([s for s, _ in dropped], [n for _, n in dropped])
        if uniform and not any(r.return_all_logits for r in requests):
            outputs = y[:, width - 1:width].split(1)            # one call for every view
        else:
            outputs = []
            for i, n in enumerate(widths):
                begin = 0 if requests[i].return_all_logits else n - 1
                outputs.append(y[i:i + 1, begin:n])
        lengths = arena.lengths
        for r in requests:
            if r.handle is not None:
                r.handle.token_count = lengths[r.cache[0].slot]
        self.last_trace = self._trace(model, requests, widths, history, transient, started, {
            "arena": {"page_arena": "device", "capacity_pages": arena.capacity,
                      "slots": arena.max_slots},
            "page_arena": "device", "graph_replay": replayed, "slots": slots,
            "cancelled_request_ids": [r.request_id for r in requests
                                      if any(s == r.cache[0].slot for s, _ in dropped)]})
        return RunnerOutput(tuple(r.request_id for r in requests), tuple(outputs), widths)

    def _replay_decode(self, runner, key, slots, requests):
        """One decode step of ``slots`` as a graph replay (captured on first use
        for this set of sequences; the capture runs the step eagerly).  The
        reserve kernel's error bits are read before returning: a step that ran
        out of pages raises ``CacheCapacityError`` and the slots stay as they
        were (the failed reserve grew none of them)."""
        import torch

        arena = runner.arena
        step = self._captured.get(key)
        rows = [r.hidden if r.hidden is not None else runner.model.embed(r.token_ids)
                for r in requests]
        if step is None:
            # this step runs eagerly (and checks itself); the next ones replay
            x = torch.stack(rows)
            y = runner.execute(slots, x, [1] * len(slots))
            while len(self._captured) >= self.max_graphs:
                self._captured.pop(next(iter(self._captured)))
            self._captured[key] = runner.capture_decode(slots, x.clone(), warm=False)
            return y
        torch.stack(rows, out=step.hidden)
        step.reserve_graph.replay()
        probe = arena.error_probe()        # waits for the reservation only
        step.graph.replay()
        failed = arena.probe_failed(probe)
        if failed:
            # the failed reservation grew no slot; the forward appended nothing
            arena._raise(failed)
        for s in slots:
            arena.lengths[s] += 1
        return step.out.clone()

    def execute(self, requests):
        requests = tuple(requests)
        if not requests:
            raise ValueError("empty paged batch")
        model = self._model_of(requests)
        if requests[0].cache and hasattr(requests[0].cache[0], "slot"):
            return self._execute_device(model, requests)
        self._validate(model, requests)
        first = requests[0]
        widths = tuple(r.width for r in requests)
        width = max(widths)
        started = time.perf_counter()
        metrics = {"direct_attention_calls": 0, "kernel_version": KERNEL_VERSION,
                   "synchronized_kernel_dispatch_ms": 0.0}
        transient = self._transient(model, len(requests), width)
        runtime = first.runtime
        x = self._inputs(model, requests, widths)
        import torch

        # logical positions (padding columns continue the row), pinned so RoPE's
        # device copy does not stall the host
        positions = torch.empty((len(requests), width), dtype=torch.int32,
                                pin_memory=x.device.type == "cuda")
        starts = np.array([r.cache[0].offset for r in requests], np.int64)
        positions.numpy()[:] = starts[:, None] + np.arange(width)[None, :]
        outputs = []

        def run(rows):
            packed = tuple(PagedBatchCache(tuple(row[layer] for row in rows), widths, metrics)
                           for layer in range(len(first.cache)))
            y = model.forward(x, cache=packed, position_ids=positions)
            # views of this step's fresh output tensor
            for i, n in enumerate(widths):
                begin = 0 if requests[i].return_all_logits else n - 1
                outputs.append(y[i:i + 1, begin:n])

        cancelled = []
        with ExitStack() as stack:
            if runtime is not None:
                stack.enter_context(runtime.transient_reservation(transient))
            if self.copy_on_write:
                drafts = []
                try:
                    for r in requests:
                        # listed before they are filled: a clone that fails part
                        # way still leaves the earlier layers' clones to reset
                        layers = []
                        drafts.append(layers)
                        for c in r.cache:
                            layers.append(c.clone())
                    run(drafts)
                    # commit: the drafts of requests still live become the
                    # request caches (old refs closed); cancelled ones are dropped
                    for r, layers in zip(requests, drafts, strict=True):
                        if request_cancelled(r):
                            cancelled.append(r.request_id)
                            continue
                        for cache, draft in zip(r.cache, layers, strict=True):
                            cache.replace_from(draft)
                finally:
                    for layers in drafts:
                        for draft in layers:
                            draft.reset()   # no-op for committed drafts (emptied by replace_from)
            else:
                marks = [[c.checkpoint() for c in r.cache] for r in requests]
                try:
                    run([r.cache for r in requests])
                except BaseException:
                    for r, layer_marks in zip(requests, marks, strict=True):
                        for cache, mark in zip(r.cache, layer_marks, strict=True):
                            cache.rollback(mark)
                    raise
                for r, layer_marks in zip(requests, marks, strict=True):
                    if request_cancelled(r):
                        cancelled.append(r.request_id)
                        for cache, mark in zip(r.cache, layer_marks, strict=True):
                            cache.rollback(mark)
            for r in requests:
                if r.handle is not None:
                    r.handle.token_count = r.cache[0].offset
        self.last_trace = self._trace(model, requests, widths, starts.tolist(), transient, started, {
            **metrics, "arena": runtime.block_pool.stats() if runtime is not None else {},
            "cancelled_request_ids": cancelled})
        return RunnerOutput(tuple(r.request_id for r in requests), tuple(outputs), widths)
