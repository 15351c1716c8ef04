"""Reference-counted page ownership (the reference's ``engine/block_cache.py``).

Same identities and rules as ``src/mlx_one/engine/block_cache.py:16-326``:
``BlockId`` packs epoch/slot/generation and is never recycled; a ``BlockRef``
owns exactly one reference and raises on a double close; blocks are sealed only
when full; pins keep a block alive without a reference.  Unlike the reference,
a block's storage is one page of a device pool (``CacheBlock.page``), not a
tuple of tensors: ``state`` is ``None`` and the pool owns the bytes.
"""

from __future__ import annotations

import threading
import uuid
from dataclasses import dataclass, field

from pkv.cache_errors import CacheCapacityError, CacheCorruptionError


class BlockId(int):
    """Opaque epoch/slot/generation identity (``block_cache.py:16-29``)."""

    @property
    def epoch(self) -> int:
        return int(self) >> 96

    @property
    def slot(self) -> int:
        return (int(self) >> 32) & ((1 << 64) - 1)

    @property
    def generation(self) -> int:
        return int(self) & ((1 << 32) - 1)


@dataclass(frozen=True)
class BlockLayout:
    """Page-format descriptor (``block_cache.py:32-43``).

    ``quantization_group_size`` is honoured (the reference only accepts 32).
    """

    version: int = 3
    layer_id: int = 0
    page_tokens: int = 16
    num_kv_heads: int | None = None
    head_dim: int | None = None
    key_dtype: str = "float16"
    value_dtype: str = "float16"
    quantization_bits: int | None = None
    quantization_group_size: int = 32
    kernel_version: str | None = None


@dataclass
class CacheBlock:
    block_id: BlockId
    token_count: int
    page: int = -1                      # page id inside its layout's device pool
    references: int = 1
    pins: int = 0
    immutable: bool = False
    layout: BlockLayout | None = None
    nbytes: int = 0
    state: object = None                # storage lives in the pool, not here
    extra: dict = field(default_factory=dict)


class BlockRef:
    """One deterministic owner of a physical block (``block_cache.py:87-118``)."""

    def __init__(self, pool, block_id, *, acquired=False):
        self.pool = pool
        self.block_id = block_id
        self.closed = False
        if acquired:
            self.pool.acquire(block_id)

    @property
    def block(self) -> CacheBlock:
        if self.closed:
            raise CacheCorruptionError("block reference is closed")
        block = self.pool._blocks.get(self.block_id)   # one atomic dict read
        if block is None:
            raise CacheCorruptionError(f"unknown or freed KV block {self.block_id}")
        return block

    def fork(self) -> "BlockRef":
        if self.closed:
            raise CacheCorruptionError("cannot fork a closed block reference")
        return BlockRef(self.pool, self.block_id, acquired=True)

    def pin(self):
        self.pool.pin(self.block_id)

    def unpin(self):
        self.pool.unpin(self.block_id)

    def close(self):
        if self.closed:
            raise CacheCorruptionError("block reference was released twice")
        self.closed = True
        self.pool.release(self.block_id)


class BlockPool:
    """Identity, refcount, pin and seal bookkeeping (``block_cache.py:121-326``).

    Subclasses provide ``_place(layout) -> (page, nbytes)`` and
    ``_reclaim_page(block)``; this class never touches device memory.
    """

    def __init__(self, capacity_bytes, *, block_tokens=32, retain_free=True):
        if capacity_bytes < 1 or block_tokens < 1:
            raise ValueError("block capacity and token width must be valid")
        self.capacity_bytes = capacity_bytes
        self.block_tokens = block_tokens
        self.retain_free = retain_free
        self._blocks: dict[BlockId, CacheBlock] = {}
        self._next_id = 0
        self._epoch = uuid.uuid4().int
        self._generation = 0
        self._lock = threading.RLock()
        self._live_nbytes = 0      # sum of nbytes over live blocks, kept incrementally
        self._reset_counts()

    # -- running statistics: each block's share, added and taken back around
    # every change of its references, pins or token count, so that stats()
    # costs the same whatever the number of blocks --------------------------------
    def _reset_counts(self):
        self._n_live = self._n_pinned = self._n_shared = 0
        self._b_pinned = self._b_evictable = self._b_shared = self._b_payload = 0

    def _count(self, b, sign):
        if b.references > 0:
            self._n_live += sign
        if b.references > 1:
            self._n_shared += sign
            self._b_shared += sign * b.nbytes * (b.references - 1)
        if b.pins > 0:
            self._n_pinned += sign
            self._b_pinned += sign * b.nbytes
        if b.references == 0 and b.pins == 1:
            self._b_evictable += sign * b.nbytes
        self._b_payload += sign * (b.nbytes * b.token_count // max(self.block_tokens, 1))

    # -- identities --------------------------------------------------------
    def _identity(self, slot):
        self._generation += 1
        return BlockId((self._epoch << 96) | (slot << 32) | self._generation)

    def _require(self, block_id) -> CacheBlock:
        try:
            return self._blocks[BlockId(block_id)]
        except KeyError as exc:
            raise CacheCorruptionError(f"unknown or freed KV block {block_id}") from exc

    # -- allocation ----------------------------------------------------------
    def allocate(self, state, token_count, *, layout=None) -> BlockId:
        if token_count < 1 or token_count > self.block_tokens:
            raise ValueError("block token count exceeds the configured block width")
        with self._lock:
            page, nbytes = self._place(layout)
            block_id = self._identity(page)
            block = CacheBlock(block_id, token_count, page=page, layout=layout, nbytes=nbytes)
            self._blocks[block_id] = block
            self._live_nbytes += nbytes
            self._count(block, 1)
            if state is not None:
                try:
                    self._store_state(block, state)
                except BaseException:
                    del self._blocks[block_id]
                    self._live_nbytes -= nbytes
                    self._count(block, -1)
                    self._reclaim_page(layout, page)
                    raise
            return block_id

    def allocate_ref(self, state, token_count, *, layout=None) -> BlockRef:
        return BlockRef(self, self.allocate(state, token_count, layout=layout))

    def acquire(self, block_id):
        with self._lock:
            block = self._require(block_id)
            self._count(block, -1)
            block.references += 1
            self._count(block, 1)

    def release(self, block_id):
        with self._lock:
            block = self._require(block_id)
            if block.references < 1:
                raise CacheCorruptionError("KV block reference count became negative")
            self._count(block, -1)
            block.references -= 1
            if block.references == 0 and block.pins == 0:
                self._drop(block)
            else:
                self._count(block, 1)

    def pin(self, block_id):
        with self._lock:
            block = self._require(block_id)
            self._count(block, -1)
            block.pins += 1
            self._count(block, 1)

    def unpin(self, block_id):
        with self._lock:
            block = self._require(block_id)
            if block.pins < 1:
                raise CacheCorruptionError("KV block pin count became negative")
            self._count(block, -1)
            block.pins -= 1
            if block.pins == 0 and block.references == 0:
                self._drop(block)
            else:
                self._count(block, 1)

    def set_token_count(self, block, token_count):
        """Change a live block's token count (a tail page filling, or rolled
        back), keeping the running statistics."""
        with self._lock:
            self._count(block, -1)
            block.token_count = token_count
            self._count(block, 1)

    def seal(self, block_id):
        with self._lock:
            block = self._require(block_id)
            if block.token_count != self.block_tokens:
                raise CacheCorruptionError("only complete KV blocks may be sealed")
            block.immutable = True

    def get(self, block_id) -> CacheBlock:
        with self._lock:
            return self._require(block_id)

    def _drop(self, block):
        # its share is already taken back by the caller (release / unpin)
        del self._blocks[block.block_id]
        self._live_nbytes -= block.nbytes
        self._reclaim_page(block.layout, block.page)

    # -- accounting ------------------------------------------------------------
    @property
    def nbytes(self):
        with self._lock:
            return self._live_nbytes

    def stats(self):
        with self._lock:
            return {
                "block_total": len(self._blocks),
                "block_free": 0,
                "block_live": self._n_live,
                "block_prefix": self._n_pinned,
                "block_shared": self._n_shared,
                "block_pinned": self._n_pinned,
                "physical_bytes": self.allocated_nbytes,
                "live_bytes": self._live_nbytes,
                "retained_free_bytes": self.allocated_nbytes - self._live_nbytes,
                "evictable_bytes": self._b_evictable,
                "shared_page_savings_bytes": self._b_shared,
                "pinned_bytes": self._b_pinned,
            }

    def payload_nbytes(self):
        """Bytes of the tokens the live blocks hold (nbytes * tokens / block
        width per block)."""
        with self._lock:
            return self._b_payload

    @property
    def allocated_nbytes(self):
        return self.nbytes

    def clear(self):
        with self._lock:
            self._blocks.clear()
            self._live_nbytes = 0
            self._reset_counts()
            self._next_id = 0
            self._epoch = uuid.uuid4().int

    def discard_free(self):
        """Kept for interface parity; freed pages return to the free list at once."""

    # -- subclass hooks ----------------------------------------------------------
    def _place(self, layout):
        raise NotImplementedError

    def _reclaim_page(self, layout, page):
        raise NotImplementedError

    def _store_state(self, block, state):
        raise NotImplementedError


__all__ = ["BlockId", "BlockLayout", "BlockPool", "BlockRef", "CacheBlock", "CacheCapacityError"]
