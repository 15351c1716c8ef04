"""Paged branch of the reference's ``CacheManager`` (``engine/cache_manager.py``).

Same names and error behaviour for the calls the paged path makes:
``create_handle`` (one ``PagedKVCache`` per layer, key/value types ``f16`` /
``bf16`` / ``q8_0`` / ``q4_0`` -> bits None/None/8/4, :152-200),
``estimate_growth`` (the quantized growth formula of :255-262, with this
build's group size in place of 32), ``reserve`` / ``commit`` / ``reconcile`` /
``release_reservation`` / ``transient_reservation`` (a byte budget; over budget
raises ``CacheCapacityError``), ``fingerprint`` / ``adopt_prefix`` /
``publish_prefix`` (shared prefix pages through ``BlockPrefixIndex``, :99-130,
:415-497, :633-667), ``release``, ``stats``, ``close``.  The arena
(``block_pool``) is a ``SegmentedPageArena`` whose pages live in device pools.
Dense / block / hybrid backends, the cold (SSD) prefix store, quality
qualification and host admission are outside the paged path.
"""

from __future__ import annotations

import hashlib
import json
import threading
import uuid
from contextlib import contextmanager
from dataclasses import dataclass, field

from pkv.arena import SegmentedPageArena
from pkv.cache_errors import (CacheCapacityError, CacheCorruptionError, CacheTopologyUnsupported,
                              KVQuantizationUnsupported, PrefixReuseUnsupported)
from pkv.paged import PagedKVCache
from pkv.prefix_cache import BlockPrefixIndex, CacheFingerprint

_BITS = {"f16": None, "bf16": None, "q8_0": 8, "q4_0": 4}


@dataclass(frozen=True)
class CacheConfig:
    backend: str = "paged"
    block_size_tokens: int = 16
    key_type: str = "bf16"
    value_type: str = "bf16"
    memory_budget_bytes: int = 8 << 30
    group_size: int = 32
    prefix_cache_enabled: bool = False
    prefix_cache_budget_bytes: int = 256 << 20
    ssd_cache_directory: str | None = None
    ssd_cache_budget_bytes: int = 1 << 30
    ssd_staging_budget_bytes: int = 256 << 20
    ssd_max_entries: int = 128
    # "host": pages owned by host bookkeeping (SegmentedPageArena + PagedKVCache,
    # the reference's structure); "device": a DevicePageArena per precision,
    # one sequence slot per handle (no host page bookkeeping per step)
    page_arena: str = "host"
    max_sequences: int = 256          # device arena: sequence slots
    max_sequence_tokens: int = 32768  # device arena: tokens per slot
    prefix_max_entries: int = 64      # device arena: published prefixes kept
    device_pages: int = 0             # device arena: pages per layer (0: from the budget)


@dataclass
class CacheBundle:
    entries: tuple
    closed: bool = False

    @property
    def nbytes(self):
        return sum(e.nbytes for e in self.entries)

    @property
    def offset(self):
        return max((e.offset for e in self.entries), default=0)


@dataclass
class CacheReservation:
    reservation_id: str
    nbytes: int
    handle_id: str | None = None
    committed: bool = False
    released: bool = False


@dataclass
class CacheHandle:
    handle_id: str
    request_id: str
    sequence_id: str
    bundle: CacheBundle
    backend: str
    key_type: str
    token_count: int = 0
    reserved_bytes: int = 0
    closed: bool = False
    reservation: CacheReservation | None = None
    metadata: dict = field(default_factory=dict)


@dataclass(frozen=True)
class CacheMemoryStats:
    budget_bytes: int
    reserved_bytes: int
    transient_bytes: int
    allocated_bytes: int
    live_handles: int
    arena: dict


class CacheManager:
    def __init__(self, bundle, config: CacheConfig = CacheConfig(), *, device="cuda"):
        if config.backend != "paged":
            raise ValueError("this build serves the paged backend only")
        if config.page_arena not in ("host", "device"):
            raise ValueError("page_arena must be 'host' or 'device'")
        self.bundle, self.config = bundle, config
        self.device = device
        self.device_arenas = {}    # (dtype, bits) -> (DevicePageArena, DevicePrefixIndex)
        self._device_bytes = 0     # page-pool bytes of every device arena, against the budget
        self.block_pool = SegmentedPageArena(config.memory_budget_bytes,
                                             block_tokens=config.block_size_tokens, device=device)
        self.block_prefix = BlockPrefixIndex(config.prefix_cache_budget_bytes,
                                             block_tokens=config.block_size_tokens)
        self.cold_prefix = None
        if config.ssd_cache_directory:
            from pkv.cold_prefix import ColdPrefixStore

            self.cold_prefix = ColdPrefixStore(config.ssd_cache_directory,
                                               budget_bytes=config.ssd_cache_budget_bytes,
                                               staging_bytes=config.ssd_staging_budget_bytes,
                                               max_entries=config.ssd_max_entries)
        self._lock = threading.RLock()
        self._handles = {}
        self._reserved = 0
        self._transient = 0
        self._closed = False

    @property
    def layer_specs(self):
        return self.bundle.spec.layers

    def _ensure_open(self):
        if self._closed:
            raise CacheCorruptionError("cache manager is closed")

    # -- handles -------------------------------------------------------------------
    def create_handle(self, request_id, *, sequence_id=None, key_type="f16", value_type="f16"):
        with self._lock:
            self._ensure_open()
            if key_type != value_type or key_type not in _BITS:
                raise KVQuantizationUnsupported("paged KV requires matched precision")
            bits = _BITS[key_type]
            dtype = "bfloat16" if key_type == "bf16" else "float16"
            if self.config.page_arena == "device":
                entries = self._slot_entries(dtype, bits)
            else:
                entries = tuple(PagedKVCache(self.block_pool, layer_id=s.layer_id, dtype=dtype,
                                             bits=bits, group_size=self.config.group_size)
                                for s in self.layer_specs)
            handle = CacheHandle(f"cache-{uuid.uuid4().hex}", request_id,
                                 sequence_id or request_id, CacheBundle(entries), "paged",
                                 key_type)
            self._handles[handle.handle_id] = handle
            return handle

    # -- device arena ------------------------------------------------------------------
    def _device_arena(self, dtype, bits):
        """The DevicePageArena (and its prefix index) of one precision: every
        layer's pool sized from the byte budget."""
        key = (dtype, bits)
        if key not in self.device_arenas:
            import torch

            from pkv.device_arena import DevicePageArena
            from pkv.device_cache import DevicePrefixIndex
            from pkv.ops import PageFormat

            specs = self.layer_specs
            if len({(s.num_kv_heads, s.key_head_dim, s.value_head_dim) for s in specs}) != 1:
                raise CacheTopologyUnsupported("a device arena holds layers of one shape")
            s0 = specs[0]
            fmt = PageFormat(s0.num_kv_heads, s0.key_head_dim, self.config.block_size_tokens,
                             bits or 16, self.config.group_size if bits else 32,
                             getattr(torch, dtype))
            # Every precision's arena is charged against the one byte budget
            # (the reference's arena enforces one capacity across all its
            # segments, engine/arena.py:71): pools are allocated whole, so an
            # arena takes device_pages pages if set, else what the arenas
            # opened before it left of the budget.
            per_page = fmt.page_bytes * len(specs)
            left = self.config.memory_budget_bytes - self._device_bytes
            capacity = self.config.device_pages or left // per_page
            if capacity < 1 or capacity * per_page > left:
                raise CacheCapacityError(
                    f"device arena for {dtype}/{bits or 16}-bit pages needs "
                    f"{max(capacity, 1) * per_page} bytes; {max(left, 0)} of the cache budget "
                    "are left", retryable=False)
            arena = DevicePageArena(fmt, capacity, num_layers=len(specs),
                                    max_slots=self.config.max_sequences +
                                    self.config.prefix_max_entries,
                                    max_tokens=self.config.max_sequence_tokens,
                                    device=self.device)
            prefix = DevicePrefixIndex(arena, capacity_pages=max(
                self.config.prefix_cache_budget_bytes // per_page, 0),
                max_entries=self.config.prefix_max_entries)
            self.device_arenas[key] = (arena, prefix)
            self._device_bytes += capacity * per_page
        return self.device_arenas[key]

    def _slot_entries(self, dtype, bits):
        from pkv.device_cache import SlotLayerCache
        from pkv.paged import _layout

        arena, _ = self._device_arena(dtype, bits)
        slot = arena.open_slot()
        return tuple(SlotLayerCache(arena, slot, s.layer_id, dtype, bits, self.config.group_size,
                                    _layout(s.layer_id, self.config.block_size_tokens,
                                            s.num_kv_heads, s.key_head_dim, dtype, bits,
                                            self.config.group_size))
                     for s in self.layer_specs)

    @staticmethod
    def _device_slot(handle):
        first = handle.bundle.entries[0] if handle.bundle.entries else None
        return first if first is not None and hasattr(first, "slot") else None

    def _validate_handle(self, handle):
        if handle.closed or self._handles.get(handle.handle_id) is not handle:
            raise CacheCorruptionError("unknown or closed cache handle")

    def estimate_growth(self, handle, prompt_tokens, max_new_tokens=0):
        """Bytes the handle may grow by (``cache_manager.py:217-266``)."""
        self._validate_handle(handle)
        tokens = max(int(prompt_tokens) + int(max_new_tokens) - handle.bundle.offset, 0)
        bits = _BITS[handle.key_type]
        if bits is None:
            amount = self.bundle.spec.bytes_per_token() * tokens
        else:
            g = self.config.group_size
            amount = sum(s.num_kv_heads * tokens * sum(
                ((dim + g - 1) // g) * (g * bits // 8 + 4) for dim in (s.key_head_dim, s.value_head_dim))
                for s in self.layer_specs)
            # page-granular sealing overlap (the reference's tail allowance)
            amount += self.bundle.spec.bytes_per_token() * self.config.block_size_tokens * 16
        handle.metadata["admission_request"] = {"prompt_tokens": prompt_tokens,
                                                "requested_output_tokens": max_new_tokens,
                                                "total_growth_bytes": amount}
        return amount

    # -- shared prefixes ------------------------------------------------------------------
    def fingerprint(self, *, key_type="f16", value_type="f16", context_tokens=None,
                    namespace=None, rendering_options=None, multimodal_identity=None):
        """The reuse key of cached KV for this model and precision (``cache_manager.py:99-130``)."""
        spec = self.bundle.spec
        shape = [(s.layer_id, s.query_heads, s.kv_heads, s.key_dim) for s in spec.layers]
        topology = hashlib.sha256(json.dumps(shape).encode()).hexdigest()
        rope = json.dumps({"rope_theta": spec.rope_theta, "rope_scaling": spec.rope_scaling},
                          sort_keys=True, default=str)
        rendering = json.dumps(rendering_options or {}, sort_keys=True, default=str)
        return CacheFingerprint(
            model_id=str(getattr(self.bundle, "model_id", "pkv-attention-stack")),
            revision=getattr(self.bundle, "revision", None),
            model_identity=str(getattr(self.bundle, "model_identity", topology)),
            adapter_identity=getattr(self.bundle, "adapter_identity", None),
            tokenizer_identity=str(getattr(self.bundle, "tokenizer_identity", "")),
            template_identity=str(getattr(self.bundle, "template_identity", "")),
            topology_digest=topology, key_type=key_type, value_type=value_type,
            context_tokens=int(context_tokens or 0), rope_identity=hashlib.sha256(
                rope.encode()).hexdigest(),
            namespace=namespace or "private",
            rendering_identity=hashlib.sha256(rendering.encode()).hexdigest(),
            multimodal_identity=multimodal_identity)

    def adopt_prefix(self, handle, fingerprint, tokens, *, minimum_tokens=1):
        """Give the handle the longest published prefix of ``tokens``; returns
        the tokens reused (0 when none).  ``cache_manager.py:415-497``, paged branch."""
        with self._lock:
            self._validate_handle(handle)
            handle.metadata["fingerprint"] = fingerprint
            if fingerprint.multimodal_identity is not None:
                raise PrefixReuseUnsupported("multimodal prefix restoration is unavailable")
            if not self.config.prefix_cache_enabled:
                return 0
            view = self._device_slot(handle)
            if view is not None:
                _, prefix = self._device_arena(view.dtype, view.bits)
                entry, pages = prefix.longest(fingerprint, tokens, minimum_tokens)
                if entry is None:
                    return 0
                count = prefix.adopt(view.slot, entry, pages)
                handle.token_count = count
                handle.metadata["shared_blocks"] = pages
                handle.metadata["prefix_tokens_reused"] = count
                return count
            match = self.block_prefix.lookup(fingerprint, tuple(tokens),
                                             minimum_tokens=minimum_tokens)
            if match is None:
                return self._adopt_cold(handle, fingerprint, tokens, minimum_tokens)
            if len(match.layer_references) != len(handle.bundle.entries):
                for layer in match.layer_references:
                    for ref in layer:
                        ref.close()
                raise CacheTopologyUnsupported("prefix layer count does not match cache plan")
            staged = []
            try:
                for cache, refs in zip(handle.bundle.entries, match.layer_references, strict=True):
                    draft = cache.empty()
                    draft.adopt(list(refs))
                    staged.append(draft)
            except BaseException:
                for draft in staged:
                    draft.reset()
                for layer in match.layer_references[len(staged):]:
                    for ref in layer:
                        if not ref.closed:
                            ref.close()
                raise
            old = handle.bundle
            handle.bundle = CacheBundle(tuple(staged))
            for entry in old.entries:
                entry.reset()
            handle.token_count = match.token_count
            handle.metadata["shared_blocks"] = match.block_count
            handle.metadata["prefix_tokens_reused"] = match.token_count
            return match.token_count

    def publish_prefix(self, handle, fingerprint, tokens, *, maximum_entries=None):
        """Index the handle's complete pages under ``tokens`` (the prompt it
        holds); ``cache_manager.py:633-667``, paged branch."""
        with self._lock:
            self._validate_handle(handle)
            if not self.config.prefix_cache_enabled or not tokens:
                return False
            if (handle.metadata.get("cancelled") or fingerprint.multimodal_identity is not None
                    or any(int(c.offset) != len(tokens) for c in handle.bundle.entries)):
                return False
            view = self._device_slot(handle)
            if view is not None:
                _, prefix = self._device_arena(view.dtype, view.bits)
                stored = prefix.publish(view.slot, fingerprint, tokens)
                handle.metadata["prefix_publications"] = (
                    handle.metadata.get("prefix_publications", 0) + int(stored))
                return stored
            layers = tuple(cache.full_block_refs for cache in handle.bundle.entries)
            stored = self.block_prefix.publish(fingerprint, tuple(tokens), layers) > 0
            handle.metadata["prefix_publications"] = (
                handle.metadata.get("prefix_publications", 0) + int(stored))
            return self._publish_cold(handle, fingerprint, tokens) or stored

    def _adopt_cold(self, handle, fingerprint, tokens, minimum):
        """Restore the longest on-disk prefix into fresh pages (``cache_manager.py:499-540``)."""
        if self.cold_prefix is None:
            return 0
        with self.transient_reservation(self.cold_prefix.staging):
            bits = {e.bits for e in handle.bundle.entries}
            match = self.cold_prefix.lookup(fingerprint, tuple(tokens), self.layer_specs,
                                            page_pool=self.block_pool, minimum=minimum,
                                            bits=bits.pop() if len(bits) == 1 else None)
            if match is None:
                return 0
            count, restored = match
            old = handle.bundle
            handle.bundle = restored
            for entry in old.entries:
                entry.reset()
            handle.token_count = count
            handle.metadata["cold_prefix_tokens"] = count
            return count

    def _publish_cold(self, handle, fingerprint, tokens):
        """Keep the handle's caches on disk as well (``cache_manager.py:541-559``).
        Page images are stored, so quantized caches qualify too."""
        if self.cold_prefix is None:
            return False
        return self.cold_prefix.put(fingerprint, tokens, handle.bundle,
                                    page_tokens=self.config.block_size_tokens,
                                    cancelled=lambda: bool(handle.closed or
                                                           handle.metadata.get("cancelled")))

    # -- byte budget -------------------------------------------------------------------
    def reserve(self, handle, nbytes):
        with self._lock:
            self._ensure_open()
            self._validate_handle(handle)
            nbytes = int(nbytes)
            if nbytes < 0:
                raise ValueError("negative reservation")
            if self._reserved + self._transient + nbytes > self.config.memory_budget_bytes:
                raise CacheCapacityError("paged cache budget exhausted", retryable=True)
            self._reserved += nbytes
            reservation = CacheReservation(f"resv-{uuid.uuid4().hex}", nbytes, handle.handle_id)
            handle.reservation = reservation
            handle.reserved_bytes += nbytes
            return reservation

    def commit(self, reservation, allocated_bytes=0):
        with self._lock:
            if reservation.released:
                raise CacheCorruptionError("reservation already released")
            reservation.committed = True

    def release_reservation(self, reservation):
        with self._lock:
            if reservation.released:
                return
            reservation.released = True
            self._reserved -= reservation.nbytes
            handle = self._handles.get(reservation.handle_id)
            if handle is not None:
                handle.reserved_bytes -= reservation.nbytes
                if handle.reservation is reservation:
                    handle.reservation = None

    def reconcile(self, handle):
        """Refresh the handle's token count from its caches."""
        with self._lock:
            self._validate_handle(handle)
            handle.token_count = handle.bundle.offset

    @contextmanager
    def transient_reservation(self, nbytes):
        with self._lock:
            self._ensure_open()
            nbytes = int(nbytes)
            if self._reserved + self._transient + nbytes > self.config.memory_budget_bytes:
                raise CacheCapacityError("transient reservation exceeds the cache budget",
                                         retryable=True)
            self._transient += nbytes
        try:
            yield nbytes
        finally:
            with self._lock:
                self._transient -= nbytes

    def release(self, handle):
        with self._lock:
            if handle.closed:
                raise CacheCorruptionError("cache handle released twice")
            self._validate_handle(handle)
            view = self._device_slot(handle)
            if view is not None:
                view.arena.release([view.slot])
            for entry in handle.bundle.entries:
                entry.reset()
            if handle.reservation is not None:
                self.release_reservation(handle.reservation)
            handle.bundle.closed = handle.closed = True
            del self._handles[handle.handle_id]

    def stats(self):
        with self._lock:
            arena = self.block_pool.stats()
            allocated = self.block_pool.allocated_nbytes
            for (dtype, bits), (dev, prefix) in self.device_arenas.items():
                pages = dev.capacity * len(dev.pools)
                allocated += pages * dev.fmt.page_bytes
                arena[f"device_{dtype}_{bits or 16}"] = {
                    "capacity_pages": dev.capacity, "layers": len(dev.pools),
                    "page_bytes": dev.fmt.page_bytes, "prefix_entries": prefix.entries}
            return CacheMemoryStats(self.config.memory_budget_bytes, self._reserved,
                                    self._transient, allocated, len(self._handles), arena)

    def close(self):
        with self._lock:
            for handle in list(self._handles.values()):
                self.release(handle)
            for _, prefix in self.device_arenas.values():
                prefix.clear()
            self.block_prefix.clear()
            self.block_pool.clear()
            self._closed = True
