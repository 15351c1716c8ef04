"""``PagedRunner.execute``: a batch step over paged caches (``engine/paged.py:285-417``).

Same checks as the reference, with this build's attention stack as the
model: validate the batch (same model, phase, layer count; every cache a
``PagedKVCache`` of its layer in the model's activation dtype; one pool and
precision), reserve the step's transient bytes on the cache manager, run the
layers over ``PagedBatchCache`` views (append + attention per layer), pick
each request's outputs (all positions for ``return_all_logits``, else the
last).  A failure anywhere leaves the request caches as they were.

Two ways to get that guarantee: the reference's (``copy_on_write=True``:
clone every layer cache -- sealed pages shared, mutable tails copied -- run on
the clones and commit them, :377-403), and the default: append in place and,
on failure, roll every cache back to its checkpoint by length (pages taken
released, tail counts restored), which saves the per-step tail copies.
Requests carry hidden states ``[T, hidden]`` where the reference carries
token ids: embedding and LM head sit outside the path.
"""

from __future__ import annotations

import time
from contextlib import ExitStack
from dataclasses import dataclass

import numpy as np

from pkv.modes import ModelCapabilityUnsupported
from pkv.paged import KERNEL_VERSION, PagedBatchCache, PagedKVCache


@dataclass(frozen=True)
class ForwardRequest:
    """Subset of ``engine/batching.py:50-66`` the paged runner reads."""

    request_id: str
    hidden: object                 # [T, hidden] device tensor, activation dtype
    cache: tuple                   # one PagedKVCache per layer
    phase: str = "decode"
    runtime: object = None         # CacheManager
    handle: object = None          # CacheHandle owning ``cache``
    model_epoch: int = 0
    return_all_logits: bool = False

    @property
    def token_ids(self):
        return range(int(self.hidden.shape[0]))


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
    def __init__(self, model, *, copy_on_write=False):
        self.model = model
        self.copy_on_write = copy_on_write
        self.last_trace = {}

    def _validate(self, requests):
        """The reference's batch checks (``paged.py:308-345``), one pass per request."""
        if not requests:
            raise ValueError("empty paged batch")
        first = requests[0]
        layers = self.model.spec.layers
        activation = self.model.activation_dtype
        hidden = self.model.spec.hidden
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
            if int(r.hidden.shape[0]) < 1 or int(r.hidden.shape[-1]) != hidden:
                raise ValueError("request hidden states do not match the model")
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

    def execute(self, requests):
        import torch

        requests = tuple(requests)
        self._validate(requests)
        first = requests[0]
        spec = self.model.spec
        widths = tuple(int(r.hidden.shape[0]) for r in requests)
        width = max(widths)
        started = time.perf_counter()
        metrics = {"direct_attention_calls": 0, "kernel_version": KERNEL_VERSION,
                   "synchronized_kernel_dispatch_ms": 0.0}
        # transient bytes of the step: activations and projections per layer
        transient = len(requests) * width * spec.num_layers * 4 * (
            spec.hidden + (spec.query_heads + 2 * spec.kv_heads) * spec.head_dim) * 2
        runtime = first.runtime
        device = first.hidden.device
        if all(n == width for n in widths) and all(
                r.hidden.dtype == first.hidden.dtype and r.hidden.device == device
                for r in requests):
            x = torch.stack([r.hidden for r in requests])          # one copy kernel
        else:
            x = torch.zeros((len(requests), width, spec.hidden), dtype=first.hidden.dtype,
                            device=device)
            for i, r in enumerate(requests):
                x[i, :widths[i]] = r.hidden
        # logical positions (padding columns continue the row), pinned so RoPE's
        # device copy does not stall the host
        positions = torch.empty((len(requests), width), dtype=torch.int32,
                                pin_memory=device.type == "cuda")
        starts = np.array([r.cache[0].offset for r in requests], np.int64)
        positions.numpy()[:] = starts[:, None] + np.arange(width)[None, :]
        outputs = []

        def run(rows):
            packed = tuple(PagedBatchCache(tuple(row[layer] for row in rows), widths, metrics)
                           for layer in range(len(first.cache)))
            y = self.model.forward(x, cache=packed, position_ids=positions)
            # views of this step's fresh output tensor
            for i, n in enumerate(widths):
                begin = 0 if requests[i].return_all_logits else n - 1
                outputs.append(y[i:i + 1, begin:n])

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
                    # commit: the drafts become the request caches (old refs closed)
                    for r, layers in zip(requests, drafts, strict=True):
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
            for r in requests:
                if r.handle is not None:
                    r.handle.token_count = r.cache[0].offset
        self.last_trace = {**metrics, "phase": first.phase,
                           "request_ids": [r.request_id for r in requests],
                           "batch_size": len(requests),
                           "history_lengths": [r.cache[0].offset - w for r, w in zip(requests, widths)],
                           "real_tokens": sum(widths), "padded_tokens": len(requests) * width,
                           "padding_efficiency": sum(widths) / (len(requests) * width),
                           "transient_reserved_bytes": transient,
                           "layer_layouts": [vars(layer) for layer in spec.layers],
                           "duration_ms": (time.perf_counter() - started) * 1000}
        return RunnerOutput(tuple(r.request_id for r in requests), tuple(outputs), widths)
