"""Device-side page allocation: the paged cache with its bookkeeping on the GPU.

The reference keeps page ownership on the host -- ``BlockPool`` refcounts and
seals (``engine/block_cache.py:121-326``), the arena's staging and per-layer
page tables (``engine/arena.py:27-225``), a clone that copies every mutable
tail (``engine/paged.py:77-101``) -- and ``PagedKVCache.append`` walks it per
sequence and layer.  ``DevicePageArena`` keeps the same ownership in device
memory (libpkv's ``pkv_arena_*``): a free stack and a reference count per page,
a page table and a length per sequence slot, one page id space shared by all
layers.  A step's page reservation is one kernel for the whole batch and every
layer, so a decode step carries no host bookkeeping and can be captured and
replayed as a HIP graph.

Semantics follow the reference's paged cache: ``fork`` is ``clone`` (pages
shared by reference count; a shared, partly filled tail is copied when it is
first written, not at fork time), ``truncate`` is ``trim``/rollback by length,
``release`` is ``reset``.  Errors (no free page, a full table) are recorded on
the device and raised by ``check()`` as ``CacheCapacityError`` /
``CacheCorruptionError``; a call that hits one leaves its slots unchanged.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from pkv import _native as nat
from pkv import ops
from pkv.cache_errors import CacheCapacityError, CacheCorruptionError

OUT_OF_PAGES, TABLE_FULL, BAD_ARGUMENT, CORRUPT = 1, 2, 4, 8
HEADER_WORDS = 16


@dataclass(frozen=True)
class Reservation:
    """One reserve call's device operands for append and attention."""

    slots: torch.Tensor        # [B] int32
    widths: torch.Tensor       # [B] int32 new tokens per slot
    table: torch.Tensor        # [B, max_pages] int32 page ids (entries past a slot's pages unset)
    starts: torch.Tensor       # [B] int32 length before the step (= the first new position)
    lens: torch.Tensor         # [B] int32 length after the step


class DevicePageArena:
    """``capacity_pages`` pages of ``fmt`` in ``num_layers`` device pools, and
    ``max_slots`` sequence slots of at most ``max_tokens`` tokens each (rounded
    up to a whole multiple of four pages)."""

    def __init__(self, fmt, capacity_pages, *, num_layers=1, max_slots=64, max_tokens=8192,
                 device="cuda"):
        if capacity_pages < 1 or num_layers < 1 or max_slots < 1 or max_tokens < 1:
            raise ValueError("arena capacity, layers, slots and tokens must be positive")
        if num_layers > 128:
            raise ValueError("a device arena holds at most 128 layer pools")
        self.fmt = fmt
        self.capacity = int(capacity_pages)
        self.page_tokens = fmt.page_tokens
        # rows of four-entry multiples: the reserve kernel copies them 16 bytes at a time
        self.max_pages = -(-int(max_tokens) // (4 * self.page_tokens)) * 4
        self.max_slots = int(max_slots)
        self.device = torch.device(device)
        lib = nat.load()
        nbytes = int(lib.pkv_arena_state_bytes(self.capacity))
        if nbytes <= 0:
            raise ValueError("arena capacity out of range")
        self.pools = [torch.zeros((self.capacity, fmt.page_bytes), dtype=torch.uint8,
                                  device=self.device) for _ in range(num_layers)]
        self.state = torch.empty(nbytes // 4, dtype=torch.int32, device=self.device)
        self.table = torch.full((self.max_slots, self.max_pages), -1, dtype=torch.int32,
                                device=self.device)
        self.lens = torch.zeros(self.max_slots, dtype=torch.int32, device=self.device)
        self._pool_ptrs = (ctypes.c_void_p * num_layers)(*[p.data_ptr() for p in self.pools])
        self._free_slots = list(range(self.max_slots - 1, -1, -1))
        self.lengths = [0] * self.max_slots     # host mirror (exact: growth is by request)
        nat.check(lib.pkv_arena_init(nat.stream_handle(self.device), nat.ptr(self.state),
                                     self.capacity), "arena init")

    # -- slots ----------------------------------------------------------------------
    def open_slot(self):
        """An empty sequence slot."""
        if not self._free_slots:
            raise CacheCapacityError("no free sequence slot in the device arena", retryable=True)
        return self._free_slots.pop()

    def _slots(self, slots):
        if isinstance(slots, torch.Tensor):
            return slots.to(device=self.device, dtype=torch.int32).contiguous(), None
        host = [int(s) for s in slots]
        if len(set(host)) != len(host) or any(s < 0 or s >= self.max_slots for s in host):
            raise ValueError("slots of one call must be distinct valid slot ids")
        return torch.tensor(host, dtype=torch.int32, device=self.device), host

    def _ints(self, values, count):
        if isinstance(values, torch.Tensor):
            return values.to(device=self.device, dtype=torch.int32).contiguous(), None
        host = [int(v) for v in values]
        if len(host) != count:
            raise ValueError("one value per slot")
        return torch.tensor(host, dtype=torch.int32, device=self.device), host

    def _common(self):
        return (self.capacity, self.page_tokens, nat.ptr(self.table), self.max_slots,
                self.max_pages, nat.ptr(self.lens))

    # -- operations ---------------------------------------------------------------------
    def reserve(self, slots, widths, *, out=None):
        """Grow each slot by its width; returns the batch's ``Reservation``.
        Device tensors are used as given (graph capture); host lists are
        validated and update the host length mirror.  ``out`` reuses the
        tensors of an earlier ``Reservation`` of the same batch size."""
        slots_d, host_slots = self._slots(slots)
        count = int(slots_d.numel())
        widths_d, host_widths = self._ints(widths, count)
        if host_slots is not None and host_widths is not None:
            if any(w < 0 for w in host_widths):
                raise ValueError("negative width")
            for s, w in zip(host_slots, host_widths):
                if self.lengths[s] + w > self.max_pages * self.page_tokens:
                    raise CacheCapacityError("sequence exceeds the arena's max_tokens")
        if out is None:
            table = torch.empty((count, self.max_pages), dtype=torch.int32, device=self.device)
            starts = torch.empty(count, dtype=torch.int32, device=self.device)
            lens = torch.empty(count, dtype=torch.int32, device=self.device)
        else:
            table, starts, lens = out.table, out.starts, out.lens
            if table.shape != (count, self.max_pages):
                raise ValueError("reservation buffers do not match the batch")
        code = nat.load().pkv_arena_reserve(
            nat.stream_handle(self.device), nat.ptr(self.state), *self._common(), nat.ptr(slots_d),
            nat.ptr(widths_d), count, self._pool_ptrs, len(self.pools), self.fmt.page_bytes,
            nat.ptr(table), nat.ptr(starts), nat.ptr(lens))
        nat.check(code, "arena reserve")
        if host_slots is not None and host_widths is not None:
            for s, w in zip(host_slots, host_widths):
                self.lengths[s] += w
        return Reservation(slots_d, widths_d, table, starts, lens)

    def truncate(self, slots, keep_tokens):
        """Cut each slot back to ``keep_tokens`` (rollback by length / ``trim``)."""
        slots_d, host_slots = self._slots(slots)
        count = int(slots_d.numel())
        keep_d, host_keep = self._ints(keep_tokens, count)
        if host_slots is not None and host_keep is not None:
            for s, k in zip(host_slots, host_keep):
                if k < 0 or k > self.lengths[s]:
                    raise ValueError("truncate keeps between 0 and the slot's length")
        code = nat.load().pkv_arena_truncate(nat.stream_handle(self.device), nat.ptr(self.state),
                                             *self._common(), nat.ptr(slots_d), nat.ptr(keep_d),
                                             count)
        nat.check(code, "arena truncate")
        if host_slots is not None and host_keep is not None:
            for s, k in zip(host_slots, host_keep):
                self.lengths[s] = k

    def release(self, slots):
        """Drop every page of the slots and return them to the free slot list."""
        host = [int(s) for s in slots]
        self.truncate(host, [0] * len(host))
        for s in host:
            if s not in self._free_slots:
                self._free_slots.append(s)

    def fork(self, src_slots, dst_slots):
        """Each (empty) destination becomes a copy of its source sharing its pages."""
        src_d, host_src = self._slots(src_slots)
        dst_d, host_dst = self._slots(dst_slots)
        if host_src is not None and host_dst is not None:
            if len(host_src) != len(host_dst) or set(host_src) & set(host_dst):
                raise ValueError("fork sources and destinations must pair up and be disjoint")
            if any(self.lengths[d] for d in host_dst):
                raise ValueError("fork destinations must be empty")
        code = nat.load().pkv_arena_fork(nat.stream_handle(self.device), nat.ptr(self.state),
                                         *self._common(), nat.ptr(src_d), nat.ptr(dst_d),
                                         int(src_d.numel()))
        nat.check(code, "arena fork")
        if host_src is not None and host_dst is not None:
            for s, d in zip(host_src, host_dst):
                self.lengths[d] = self.lengths[s]

    # -- inspection (these synchronise) ---------------------------------------------------
    def sync_lengths(self):
        """Refresh the host length mirror from the device (after graph replays)."""
        self.lengths = [int(x) for x in self.lens.cpu().tolist()]

    def status(self):
        """``(free_pages, error_bits)``."""
        head = self.state[:2].cpu().tolist()
        return head[0], head[1]

    @staticmethod
    def _raise(err):
        if err & (BAD_ARGUMENT | CORRUPT):
            raise CacheCorruptionError(f"device arena error bits {err:#x}")
        raise CacheCapacityError(
            "device arena out of pages" if err & OUT_OF_PAGES else
            "sequence exceeds the arena's table", retryable=bool(err & OUT_OF_PAGES))

    def check(self):
        """Raise the first recorded device error (and clear the record)."""
        free, err = self.status()
        if err:
            self.state[1:2].zero_()
            self._raise(err)
        return free

    def error_probe(self):
        """Enqueue a copy of the error bits (as the stream stands now) into pinned
        host memory; ``probe_failed(probe)`` reads it once that point of the
        stream has run -- usually long before the caller asks.  One probe at a
        time per arena (its calls are ordered on one stream anyway): the pinned
        word and the event are reused."""
        if getattr(self, "_probe", None) is None:
            self._probe = (torch.empty(1, dtype=torch.int32, pin_memory=True), torch.cuda.Event())
        host, event = self._probe
        host.copy_(self.state[1:2], non_blocking=True)
        event.record(torch.cuda.current_stream(self.device))
        return host, event

    def probe_failed(self, probe):
        """The error bits a probe saw (0 if none); a set bit is cleared on the device."""
        host, event = probe
        event.synchronize()
        err = int(host[0])
        if err:
            self.state[1:2].zero_()
        return err

    def refcounts(self):
        return self.state[HEADER_WORDS + self.capacity:HEADER_WORDS + 2 * self.capacity].cpu()

    def free_stack(self):
        free = int(self.state[0].item())
        return self.state[HEADER_WORDS:HEADER_WORDS + free].cpu()

    def pages(self, slot):
        n = -(-int(self.lens[slot].item()) // self.page_tokens)
        return self.table[slot, :n].cpu().tolist()


class DeviceBatchCache:
    """One layer of a reserved batch: ``attend`` appends the step's K/V into the
    layer's pool and runs paged attention, with every operand already on the
    device (``PagedBatchCache.attend``, ``engine/paged.py:245-267``)."""

    def __init__(self, arena, layer, reservation, *, workspace=None, waves=0):
        self.arena, self.layer, self.res = arena, layer, reservation
        # a captured step brings its own workspace (and the waves it was sized
        # for): the shared per-device one may be replaced by a later eager call
        self.workspace, self.waves = workspace, waves

    def attend(self, queries, keys, values, *, scale, position_ids=None):
        """Queries of row b sit at positions ``starts[b] + q`` (taken before the
        append, so the new tokens attend to themselves); ``position_ids`` is not
        read (the reservation fixes the positions on the device)."""
        fmt, pool = self.arena.fmt, self.arena.pools[self.layer]
        dtype = fmt.dtype
        if queries.shape[2] == 1:
            # a decode step (every width 1): the new token at lens - 1, its
            # query there too -- one fused append + attention call
            out = ops.append_paged_attention(fmt, pool, keys.to(dtype), values.to(dtype),
                                             queries.to(dtype), self.res.table, self.res.lens,
                                             scale=scale, waves=self.waves,
                                             workspace=self.workspace)
            return out.to(queries.dtype)
        ops.append_quantize(fmt, pool, keys.to(dtype).contiguous(), values.to(dtype).contiguous(),
                            self.res.table, self.res.starts, self.res.widths)
        out = ops.paged_attention(fmt, pool, queries.to(dtype).contiguous(), self.res.table,
                                  self.res.lens, scale=scale, widths=self.res.widths,
                                  waves=self.waves, workspace=self.workspace)
        return out.to(queries.dtype)


class DeviceRunner:
    """Batch steps of a model over device-arena slots: ``PagedRunner.execute``
    (``engine/paged.py:308-417``) with the page bookkeeping on the device.  One
    reservation covers every layer; a step that raises is rolled back by
    length (``truncate`` to the lengths before it)."""

    def __init__(self, model, arena):
        if len(arena.pools) != model.spec.num_layers:
            raise ValueError("the arena needs one pool per model layer")
        self.model, self.arena = model, arena

    def _forward(self, hidden, res, workspace=None, waves=0):
        batch, width, _ = hidden.shape
        positions = res.starts.view(batch, 1)
        if width > 1:
            positions = positions + torch.arange(width, dtype=torch.int32, device=hidden.device)
        caches = tuple(DeviceBatchCache(self.arena, layer, res, workspace=workspace, waves=waves)
                       for layer in range(len(self.arena.pools)))
        return self.model.forward(hidden, cache=caches, position_ids=positions)

    def execute(self, slots, hidden, widths=None):
        """``hidden [B, T, hidden]`` for ``slots`` (row b's columns past
        ``widths[b]`` are padding); returns the model's ``[B, T, hidden]``."""
        batch, width, _ = hidden.shape
        slots = [int(s) for s in slots]
        widths = [width] * batch if widths is None else [int(w) for w in widths]
        if len(slots) != batch or len(widths) != batch or any(w < 1 or w > width for w in widths):
            raise ValueError("one slot and a width in 1..T per row")
        before = [self.arena.lengths[s] for s in slots]
        res = self.arena.reserve(slots, widths)
        # the reserve kernel's error bits, read after the forward is enqueued:
        # by then the reserve has long run, so the check costs no stall
        probe = self.arena.error_probe()
        try:
            out = self._forward(hidden, res)
        except BaseException:
            self.arena.truncate(slots, before)
            raise
        err = self.arena.probe_failed(probe)
        if err:
            # a failed reserve grew no slot (its append wrote nothing): only
            # the host length mirror moved
            for s, n in zip(slots, before):
                self.arena.lengths[s] = n
            self.arena._raise(err)
        return out

    def capture_decode(self, slots, hidden, *, warm=True):
        """Graphs of one decode step (one token per slot) reading the static
        buffer ``hidden [B, 1, hidden]``: returns a ``CapturedStep`` whose
        ``replay()`` appends a token to every slot and leaves the step's output
        in ``out``.  The step is two graphs, the page reservation and the
        forward, so a caller can read the reservation's error bits between
        them.  ``warm`` runs one step eagerly first (it sizes the buffers and
        warms the libraries; without it the caller must have run a step of
        this shape).  Replays do not advance the host length mirror:
        ``arena.sync_lengths()`` reads the device's."""
        arena = self.arena
        device = arena.device
        slots_d = torch.tensor([int(s) for s in slots], dtype=torch.int32, device=device)
        widths_d = torch.ones_like(slots_d)
        count = int(slots_d.numel())
        # the graph's split-K partials live in a workspace of its own, sized
        # for the waves fixed at capture and held by the CapturedStep
        spec = self.model.spec
        waves = ops.default_waves(arena.fmt, spec.query_heads, 1, count)
        workspace = torch.empty(max(256, ops.workspace_bytes(arena.fmt, spec.query_heads, 1,
                                                             waves)),
                                dtype=torch.uint8, device=device)
        if warm:
            res = arena.reserve(slots_d, widths_d)
            self._forward(hidden, res, workspace, waves)
        else:
            res = Reservation(slots_d, widths_d,
                              torch.empty((count, arena.max_pages), dtype=torch.int32,
                                          device=device),
                              torch.empty(count, dtype=torch.int32, device=device),
                              torch.empty(count, dtype=torch.int32, device=device))
        torch.cuda.synchronize(device)
        reserve_graph, graph = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
        stream = torch.cuda.Stream(device)
        stream.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(stream):
            with torch.cuda.graph(reserve_graph, stream=stream):
                arena.reserve(slots_d, widths_d, out=res)
            with torch.cuda.graph(graph, stream=stream):
                out = self._forward(hidden, res, workspace, waves)
        torch.cuda.current_stream(device).wait_stream(stream)
        if warm:
            arena.sync_lengths()
        return CapturedStep(graph, out, hidden, res, (slots_d, widths_d), workspace, waves,
                            reserve_graph)


@dataclass
class CapturedStep:
    """A captured decode step and every buffer from outside the capture that its
    kernels read or write: they must live as long as the graph."""

    graph: torch.cuda.CUDAGraph
    out: torch.Tensor               # the step's output, rewritten by each replay
    hidden: torch.Tensor            # the static input buffer
    reservation: Reservation        # the batch operands the reserve kernel rewrites
    operands: tuple                 # slot ids and widths read by the reserve kernel
    workspace: torch.Tensor = None  # the attention's split-K partials (every layer's launch)
    waves: int = 0                  # the attention waves the workspace is sized for
    reserve_graph: torch.cuda.CUDAGraph = None   # the page reservation, replayed first

    def replay(self):
        if self.reserve_graph is not None:
            self.reserve_graph.replay()
        self.graph.replay()
