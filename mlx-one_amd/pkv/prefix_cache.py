"""Shared prefix pages: the reference's ``BlockPrefixIndex`` (``engine/prefix_cache.py:157-348``).

Each published block of ``block_tokens`` prompt tokens becomes a node keyed by
a hash chained from its parent's key (the first parent is the cache
fingerprint's digest), holding one sealed page per layer; the index pins those
pages, so they outlive the request that computed them.  ``lookup`` walks the
chain for a prompt (never its last token, which must still be computed) and
hands out fresh ``BlockRef``s to the matched pages, which ``PagedKVCache.adopt``
takes.  Over budget, leaves are evicted oldest first (a parent is never
evicted before its children).

Bookkeeping only -- page bytes never move: adopting a prefix is a reference
count, and the attention kernels read the shared pages in place (a shared
prefix is read once per KV head per step whatever the number of sequences
holding it).
"""

from __future__ import annotations

import hashlib
import json
import threading
import time
from collections import OrderedDict
from dataclasses import asdict, dataclass

from pkv.block_cache import BlockRef


@dataclass(frozen=True)
class CacheFingerprint:
    """What must match for cached KV to be reusable (``engine/cache_specs.py:207-230``)."""

    model_id: str
    revision: str | None
    model_identity: str
    adapter_identity: str | None
    tokenizer_identity: str
    template_identity: str
    topology_digest: str
    key_type: str
    value_type: str
    context_tokens: int
    rope_identity: str
    namespace: str = "private"
    special_tokens_identity: str = ""
    rendering_identity: str = ""
    multimodal_identity: str | None = None
    execution_identity: str = ""

    @property
    def digest(self) -> str:
        """sha256 of the fields as canonical JSON (sorted keys, no spaces)."""
        text = json.dumps(asdict(self), sort_keys=True, separators=(",", ":"))
        return hashlib.sha256(text.encode()).hexdigest()


@dataclass(frozen=True)
class BlockLink:
    pool: object
    block_id: int


@dataclass
class BlockPrefixEntry:
    key: str
    parent: str
    fingerprint: CacheFingerprint
    token_count: int                 # tokens from the start of the prompt through this block
    tokens: tuple                    # this block's tokens
    layer_blocks: tuple              # per layer: (BlockLink,)
    last_access: float

    @property
    def metadata_bytes(self) -> int:
        """Bounded host accounting, as the reference charges it."""
        return 512 + 40 * len(self.tokens) + 128 * len(self.layer_blocks)


@dataclass(frozen=True)
class BlockPrefixMatch:
    token_count: int
    layer_references: tuple          # per layer: (BlockRef, ...) one per matched block
    block_count: int


def chain_key(parent: str, tokens) -> str:
    """Key of a block: sha256 over the parent key and the block's tokens (JSON)."""
    payload = json.dumps(list(tokens), separators=(",", ":")).encode("ascii")
    return hashlib.sha256(parent.encode("ascii") + b":" + payload).hexdigest()


class BlockPrefixIndex:
    """Parent-linked index of published prompt blocks (``prefix_cache.py:186-348``)."""

    def __init__(self, capacity_bytes, *, block_tokens, metadata_capacity_bytes=4 << 20):
        if capacity_bytes < 0 or metadata_capacity_bytes < 0:
            raise ValueError("prefix capacity cannot be negative")
        self.capacity_bytes = int(capacity_bytes)
        self.metadata_capacity_bytes = int(metadata_capacity_bytes)
        self.block_tokens = int(block_tokens)
        self._entries = OrderedDict()          # key -> entry, least recently used first
        self._pins = {}                        # (id(pool), block_id) -> owners among entries
        self._lock = threading.RLock()
        self.hits = self.misses = self.evictions = self.tokens_reused = 0

    # -- accounting ---------------------------------------------------------------------
    @property
    def nbytes(self):
        with self._lock:
            pages = {}
            for entry in self._entries.values():
                for layer in entry.layer_blocks:
                    for link in layer:
                        pages[(id(link.pool), int(link.block_id))] = link.pool.get(link.block_id).nbytes
            return sum(pages.values())

    def _metadata_bytes(self):
        return sum(e.metadata_bytes for e in self._entries.values())

    # -- lookup ---------------------------------------------------------------------------
    def _walk(self, fingerprint, tokens):
        """Nodes matching the prompt's leading blocks (the last token never counts)."""
        blocks = (len(tokens) - 1) // self.block_tokens if tokens else 0
        parent, path = fingerprint.digest, []
        for b in range(blocks):
            chunk = tuple(tokens[b * self.block_tokens:(b + 1) * self.block_tokens])
            node = self._entries.get(chain_key(parent, chunk))
            if node is None or node.fingerprint != fingerprint or node.tokens != chunk:
                break
            path.append(node)
            parent = node.key
        return path

    def longest_prefix_tokens(self, fingerprint, tokens, *, minimum_tokens=1):
        with self._lock:
            path = self._walk(fingerprint, tokens)
            count = path[-1].token_count if path else 0
            return count if count >= minimum_tokens else 0

    def lookup(self, fingerprint, tokens, *, minimum_tokens=1):
        """A ``BlockPrefixMatch`` holding new references to the matched pages, or None."""
        with self._lock:
            path = self._walk(fingerprint, tokens)
            if not path or path[-1].token_count < minimum_tokens:
                self.misses += 1
                return None
            taken, layers = [], [[] for _ in path[0].layer_blocks]
            try:
                for node in path:
                    for index, links in enumerate(node.layer_blocks):
                        for link in links:
                            ref = BlockRef(link.pool, link.block_id, acquired=True)
                            taken.append(ref)
                            layers[index].append(ref)
            except BaseException:
                for ref in reversed(taken):
                    ref.close()
                raise
            now = time.monotonic()
            for node in path:
                node.last_access = now
                self._entries.move_to_end(node.key)
            self.hits += 1
            self.tokens_reused += path[-1].token_count
            return BlockPrefixMatch(path[-1].token_count, tuple(tuple(x) for x in layers),
                                    len(taken))

    # -- publication ----------------------------------------------------------------------
    def _pin(self, link):
        key = (id(link.pool), int(link.block_id))
        if not self._pins.get(key):
            link.pool.pin(link.block_id)
        self._pins[key] = self._pins.get(key, 0) + 1

    def _unpin(self, link):
        key = (id(link.pool), int(link.block_id))
        left = self._pins[key] - 1
        if left:
            self._pins[key] = left
        else:
            del self._pins[key]
            link.pool.unpin(link.block_id)

    def _drop(self, entry):
        for layer in entry.layer_blocks:
            for link in layer:
                self._unpin(link)

    def publish(self, fingerprint, tokens, layer_blocks):
        """Index the complete sealed pages of a prompt (per layer, in order);
        returns how many new blocks were added."""
        if not layer_blocks or not self.capacity_bytes:
            return 0
        complete = min(min(len(layer) for layer in layer_blocks), len(tokens) // self.block_tokens)
        for layer in layer_blocks:                       # check everything before pinning
            for ref in layer[:complete]:
                block = ref.block
                if not block.immutable or block.token_count != self.block_tokens:
                    raise ValueError("prefix publication requires sealed complete pages")
        added = []
        parent = fingerprint.digest
        with self._lock:
            try:
                for index in range(complete):
                    chunk = tuple(tokens[index * self.block_tokens:(index + 1) * self.block_tokens])
                    key = chain_key(parent, chunk)
                    if key not in self._entries:
                        links = tuple((BlockLink(layer[index].pool, layer[index].block_id),)
                                      for layer in layer_blocks)
                        pinned = []
                        try:
                            for layer in links:
                                for link in layer:
                                    self._pin(link)
                                    pinned.append(link)
                        except BaseException:
                            for link in reversed(pinned):
                                self._unpin(link)
                            raise
                        self._entries[key] = BlockPrefixEntry(
                            key, parent, fingerprint, (index + 1) * self.block_tokens, chunk,
                            links, time.monotonic())
                        added.append(key)
                    parent = key
            except BaseException:
                for key in reversed(added):
                    self._drop(self._entries.pop(key))
                raise
            self._evict()
            return sum(key in self._entries for key in added)

    def _evict(self):
        """Drop least recently used leaves until both budgets hold."""
        while self._entries and (self.nbytes > self.capacity_bytes
                                 or self._metadata_bytes() > self.metadata_capacity_bytes):
            parents = {entry.parent for entry in self._entries.values()}
            key = next(k for k in self._entries if k not in parents)
            self._drop(self._entries.pop(key))
            self.evictions += 1

    def clear(self):
        with self._lock:
            for entry in self._entries.values():
                self._drop(entry)
            self._entries.clear()

    def stats(self):
        with self._lock:
            return {"entries": len(self._entries), "bytes": self.nbytes,
                    "metadata_bytes": self._metadata_bytes(),
                    "capacity_bytes": self.capacity_bytes, "hits": self.hits,
                    "misses": self.misses, "evictions": self.evictions,
                    "tokens_reused": self.tokens_reused}
