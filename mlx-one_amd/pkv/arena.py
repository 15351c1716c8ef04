"""Page arena and persistent page tables on HBM (the reference's ``engine/arena.py``).

The reference keeps one tuple of MLX tensors per 16-page segment and re-stages
(copies) a whole segment on every write (``src/mlx_one/engine/arena.py:90-113``).
Here each page layout owns one contiguous device pool of fixed-size pages
(``pkv_format.h``); the append kernel writes a token's bytes in place, so a
store is free and the page table holds plain page ids.  The reference's names
and observable accounting are kept: pages group into 16-page "segments"
(``address`` returns ``(segment_id, slot)``), ``lease`` keeps the current pool
buffers alive for a dispatch, ``stats`` reports the same keys.
"""

from __future__ import annotations

import heapq
import weakref
from contextlib import contextmanager

import numpy as np

from pkv.block_cache import BlockPool
from pkv.cache_errors import CacheCapacityError, CacheCorruptionError

ARENA_VERSION = "mi355x-page-pool-v1"
SEGMENT_PAGES = 16


def page_format(layout):
    """``ops.PageFormat`` of a ``BlockLayout``."""
    import torch

    from pkv.ops import PageFormat

    dtype = {"float16": torch.float16, "bfloat16": torch.bfloat16}[layout.key_dtype]
    bits = layout.quantization_bits or 16
    return PageFormat(layout.num_kv_heads, layout.head_dim, layout.page_tokens, bits,
                      layout.quantization_group_size if bits != 16 else 32, dtype)


class DevicePagePool:
    """Pages of one layout in one device buffer ``[capacity, page_bytes]`` (uint8).

    Grows by doubling (copying the live pages, zero-filling the rest), never
    past ``max_pages`` -- the arena's byte budget in pages of this layout -- so
    the buffer stays within the configured bytes; freed pages are reused
    lowest-id first (a heap).
    """

    def __init__(self, fmt, device, ordinal, initial_pages=64, max_pages=None):
        self.fmt, self.device, self.ordinal = fmt, device, ordinal
        self.page_bytes = fmt.page_bytes
        self.buffer = None
        self.capacity = 0
        self.next_page = 0
        self.free = []
        self.initial_pages = initial_pages
        self.max_pages = max_pages

    def _grow(self, need):
        import torch

        capacity = max(self.initial_pages, self.capacity * 2, need)
        if self.max_pages is not None:
            capacity = max(min(capacity, self.max_pages), need)
        buffer = torch.zeros((capacity, self.page_bytes), dtype=torch.uint8, device=self.device)
        if self.buffer is not None:
            buffer[:self.capacity].copy_(self.buffer)
        self.buffer, self.capacity = buffer, capacity

    def take(self):
        if self.free:
            return heapq.heappop(self.free)
        if self.next_page >= self.capacity:
            self._grow(self.next_page + 1)
        self.next_page += 1
        return self.next_page - 1

    def give(self, page):
        heapq.heappush(self.free, page)

    @property
    def live_pages(self):
        return self.next_page - len(self.free)


class SegmentedPageArena(BlockPool):
    """Device page pools behind the reference's arena interface (``arena.py:27-169``)."""

    def __init__(self, capacity_bytes, *, block_tokens=32, retain_free=True, device="cuda"):
        super().__init__(capacity_bytes, block_tokens=block_tokens, retain_free=retain_free)
        self.device = device
        self.pools = {}
        self.table_update_bytes = 0
        self.segment_update_bytes = 0
        self.replacement_peak_bytes = 0
        self._tables = weakref.WeakSet()
        self._leases = []
        self._segment_pages = {}   # occupied segment id -> live pages in it (stats)

    # -- pools ---------------------------------------------------------------
    def pool_for(self, layout) -> DevicePagePool:
        pool = self.pools.get(layout)
        if pool is None:
            fmt = page_format(layout)
            pool = DevicePagePool(fmt, self.device, len(self.pools),
                                  max_pages=max(1, self.capacity_bytes // fmt.page_bytes))
            self.pools[layout] = pool
        return pool

    def _place(self, layout):
        if layout is None:
            raise ValueError("arena allocation requires a valid layout and token count")
        pool = self.pool_for(layout)
        if self.nbytes + pool.page_bytes > self.capacity_bytes:
            raise CacheCapacityError("segmented KV arena is full")
        page = pool.take()
        sid = (pool.ordinal << 32) | (page // SEGMENT_PAGES)
        self._segment_pages[sid] = self._segment_pages.get(sid, 0) + 1
        return page, pool.page_bytes

    def _reclaim_page(self, layout, page):
        pool = self.pools[layout]
        sid = (pool.ordinal << 32) | (page // SEGMENT_PAGES)
        left = self._segment_pages[sid] - 1
        if left:
            self._segment_pages[sid] = left
        else:
            del self._segment_pages[sid]
        pool.give(page)

    def _store_state(self, block, state):
        """Write float K/V page tensors ``[1, HK, P, D]`` (quantizing if the layout says so)."""
        import torch

        from pkv import ops

        keys, values = state[0], state[1]
        layout = block.layout
        pool = self.pool_for(layout)
        count = block.token_count
        table = torch.tensor([[block.page]], dtype=torch.int32, device=pool.buffer.device)
        ops.append_quantize(pool.fmt, pool.buffer, keys[:, :, :count].contiguous(),
                            values[:, :, :count].contiguous(), table,
                            torch.zeros(1, dtype=torch.int32, device=pool.buffer.device))

    # -- reference interface ------------------------------------------------------
    def store(self, block_id):
        """Writes land in the pool in place; nothing to publish (``arena.py:108-113``)."""
        self._require(block_id)

    @property
    def segments(self):
        """Occupied 16-page segments: ``{segment_id: (layout, pages)}``."""
        out = {}
        for block in self._blocks.values():
            pool = self.pools[block.layout]
            sid = (pool.ordinal << 32) | (block.page // SEGMENT_PAGES)
            out.setdefault(sid, (block.layout, set()))[1].add(block.page % SEGMENT_PAGES)
        return out

    def address(self, reference):
        block = reference.block
        if reference.pool is not self or block.block_id not in self._blocks:
            raise CacheCorruptionError("page is not owned by this arena")
        pool = self.pools.get(block.layout)
        if pool is None:
            raise CacheCorruptionError("stale arena address or layout")
        return (pool.ordinal << 32) | (block.page // SEGMENT_PAGES), block.page % SEGMENT_PAGES

    @contextmanager
    def lease(self):
        """Keep the current pool buffers alive while a dispatch uses them."""
        with self._lock:
            held = tuple(p.buffer for p in self.pools.values() if p.buffer is not None)
            self._leases.append(held)
        try:
            yield held
        finally:
            with self._lock:
                self._leases[:] = [x for x in self._leases if x is not held]

    @property
    def allocated_nbytes(self):
        return sum(p.capacity * p.page_bytes for p in self.pools.values())

    def stats(self):
        result = super().stats()
        payload = self.payload_nbytes()
        result.update(arena_version=ARENA_VERSION, segment_count=len(self._segment_pages),
                      segment_capacity_pages=SEGMENT_PAGES, page_payload_bytes=payload,
                      unused_segment_bytes=self.allocated_nbytes - payload,
                      table_bytes=sum(t.table_bytes for t in list(self._tables)),
                      table_update_bytes=self.table_update_bytes,
                      segment_update_bytes=self.segment_update_bytes,
                      replacement_overlap_peak_bytes=self.replacement_peak_bytes,
                      replacement_overlap_bytes=0, pool_count=len(self.pools))
        return result

    def clear(self):
        with self._lock:
            super().clear()
            self.pools.clear()
            self._tables = weakref.WeakSet()
            self._segment_pages = {}


class PersistentPageTable:
    """Logical page index -> page, in 16-entry chunks (``arena.py:172-225``).

    Entries keep the reference's ``(segment_id, slot, start_token,
    token_count)`` tuples; chunks are immutable tuples shared by forks, and
    an edit replaces one chunk (accounted as 256 bytes, as the reference's
    ``[16, 4]`` int32 chunk).  ``pages`` lists the pool page ids in order --
    the row of the device block table, also kept as an int32 array (``row()``)
    so a batch table is assembled by slice copies.  Forks copy ``entries``,
    so edits mutate it in place.
    """

    def __init__(self, arena):
        self.arena, self.chunks, self.entries, self.pages = arena, {}, {}, []
        self._ids = np.full(SEGMENT_PAGES, -1, np.int32)
        arena._tables.add(self)

    @property
    def table_bytes(self):
        return len(self.chunks) * SEGMENT_PAGES * 4 * 4

    def fork(self):
        result = PersistentPageTable(self.arena)
        result.chunks, result.entries, result.pages = dict(self.chunks), dict(self.entries), list(
            self.pages)
        result._ids = self._ids.copy()
        return result

    def row(self):
        """``pages`` as an int32 array view (valid until the next edit)."""
        return self._ids[:len(self.pages)]

    def _rebuild_chunk(self, chunk):
        self.chunks[chunk] = tuple(self.entries.get(i, (-1, -1, 0, 0))
                                   for i in range(chunk * SEGMENT_PAGES, (chunk + 1) * SEGMENT_PAGES))
        self.arena.table_update_bytes += SEGMENT_PAGES * 4 * 4

    def update(self, index, reference):
        sid, slot = self.arena.address(reference)
        block = reference.block
        entry = (sid, slot, index * self.arena.block_tokens, block.token_count)
        if self.entries.get(index) == entry:
            return
        self.entries[index] = entry
        chunk = index // SEGMENT_PAGES
        if chunk in self.chunks:    # edit one slot of the chunk
            row = list(self.chunks[chunk])
            row[index % SEGMENT_PAGES] = entry
            self.chunks[chunk] = tuple(row)
            self.arena.table_update_bytes += SEGMENT_PAGES * 4 * 4
        else:
            self._rebuild_chunk(chunk)
        while len(self.pages) <= index:
            self.pages.append(-1)
        self.pages[index] = block.page
        if index >= len(self._ids):
            grown = np.full(max(2 * len(self._ids), index + 1), -1, np.int32)
            grown[:len(self._ids)] = self._ids
            self._ids = grown
        self._ids[index] = block.page

    def truncate(self, length):
        for index in [i for i in self.entries if i >= length]:
            del self.entries[index]
        del self.pages[length:]
        self._ids[length:] = -1
        for chunk in list(self.chunks):
            if chunk * SEGMENT_PAGES >= length:
                del self.chunks[chunk]
        if length % SEGMENT_PAGES:
            self._rebuild_chunk(length // SEGMENT_PAGES)

    def validate(self, references):
        if len(references) != len(self.entries):
            raise CacheCorruptionError("page table length mismatch")
        for index, ref in enumerate(references):
            sid, slot = self.arena.address(ref)
            if self.entries[index] != (sid, slot, index * self.arena.block_tokens,
                                       ref.block.token_count):
                raise CacheCorruptionError("page table address mismatch")
