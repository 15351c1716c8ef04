"""Shared prefix pages: ``BlockPrefixIndex`` (reference interface:
``engine/prefix_cache.py:186-348``; ``CacheFingerprint``:
``engine/cache_specs.py:207-230``).

A published prompt is stored as a path in a trie, one trie per cache
fingerprint.  Each edge is one page of prompt tokens (``block_tokens`` of
them) and the node it leads to holds that page of every layer, pinned in its
pool for as long as the node lives, so the pages outlive the request that
computed them.  ``lookup`` follows the trie along a new prompt (never its last
token, which the model must still compute) and hands out fresh ``BlockRef``s
to the pages of the nodes it passed, which ``PagedKVCache.adopt`` takes.

Names kept from the reference (callers use them): ``lookup``,
``longest_prefix_tokens``, ``publish``, ``clear``, ``stats``, the
``BlockPrefixMatch`` result.  Node keys are ``chain_key`` chains from the
fingerprint's digest, the reference's key construction, so a key identifies
the same prefix here and there; the trie itself is walked by token chunks.

Budgets: page bytes (each node is charged its pages, all layers) and host
metadata bytes.  Over either, the least recently used leaf goes first (a
node is never dropped before its children); recency is a logical clock
stamped along every path a lookup or publication touches, and leaves wait in
a heap whose stale items are skipped when popped.

Bookkeeping only -- page bytes never move: adopting a prefix is a reference
count, and the attention kernels read the shared pages in place.
"""

from __future__ import annotations

import hashlib
import heapq
import itertools
import json
import threading
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
class BlockPrefixMatch:
    token_count: int
    layer_references: tuple          # per layer: (BlockRef, ...) one per matched block
    block_count: int


def chain_key(parent: str, tokens) -> str:
    """Key of a block: sha256 over the parent key and the block's tokens (JSON)."""
    payload = json.dumps(list(tokens), separators=(",", ":")).encode("ascii")
    return hashlib.sha256(parent.encode("ascii") + b":" + payload).hexdigest()


# host bytes charged per node: the node itself, its token chunk (8 bytes per
# token id) and one (pool, block id) pair per layer
_NODE_BYTES = 192
_TOKEN_BYTES = 8
_LINK_BYTES = 48


class _Node:
    """One page of a published prompt: the trie edge ``chunk`` from ``parent``
    and the pinned page of each layer (``pages[layer] = (pool, block_id)``)."""

    __slots__ = ("key", "parent", "chunk", "children", "pages", "page_bytes", "meta_bytes",
                 "depth", "stamp", "attached")

    def __init__(self, key, parent, chunk, pages, page_bytes, depth):
        self.key, self.parent, self.chunk = key, parent, chunk
        self.children = {}
        self.pages = pages
        self.page_bytes = page_bytes
        self.meta_bytes = _NODE_BYTES + _TOKEN_BYTES * len(chunk) + _LINK_BYTES * len(pages)
        self.depth = depth              # pages from the start of the prompt through this one
        self.stamp = 0
        self.attached = True


class BlockPrefixIndex:
    """Per-fingerprint tries of published prompt pages."""

    def __init__(self, capacity_bytes, *, block_tokens, metadata_capacity_bytes=4 << 20):
        if capacity_bytes < 0 or metadata_capacity_bytes < 0:
            raise ValueError("prefix capacity cannot be negative")
        self.capacity_bytes = int(capacity_bytes)
        self.metadata_capacity_bytes = int(metadata_capacity_bytes)
        self.block_tokens = int(block_tokens)
        self._roots = {}                # fingerprint -> root node (no pages)
        self._count = 0                 # nodes with pages
        self._page_bytes = 0
        self._meta_bytes = 0
        self._clock = itertools.count(1)
        self._leaves = []               # heap of (stamp, tie, node); stale items skipped
        self._tie = itertools.count()
        self._lock = threading.RLock()
        self.hits = self.misses = self.evictions = self.tokens_reused = 0

    # -- accounting ---------------------------------------------------------------------
    @property
    def nbytes(self):
        """Page bytes the index holds (every node's pages, all layers)."""
        return self._page_bytes

    def _over_budget(self):
        return (self._page_bytes > self.capacity_bytes
                or self._meta_bytes > self.metadata_capacity_bytes)

    # -- trie walks -----------------------------------------------------------------------
    def _chunks(self, tokens, count):
        p = self.block_tokens
        return (tuple(tokens[i * p:(i + 1) * p]) for i in range(count))

    def _follow(self, fingerprint, tokens):
        """Nodes along ``tokens``' leading pages; a prompt's last token is never
        part of a match (``(len - 1) // block_tokens`` pages at most)."""
        node = self._roots.get(fingerprint)
        path = []
        if node is None or not tokens:
            return path
        for chunk in self._chunks(tokens, (len(tokens) - 1) // self.block_tokens):
            node = node.children.get(chunk)
            if node is None:
                break
            path.append(node)
        return path

    def _touch(self, path):
        stamp = next(self._clock)
        for node in path:
            node.stamp = stamp
            if not node.children:
                heapq.heappush(self._leaves, (stamp, next(self._tie), node))
        if len(self._leaves) > 4 * self._count + 64:
            # mostly stale items (leaves touched again): rebuild from the live leaves
            self._leaves = [(n.stamp, next(self._tie), n) for n in self._nodes() if not n.children]
            heapq.heapify(self._leaves)

    def _nodes(self):
        stack = [child for root in self._roots.values() for child in root.children.values()]
        while stack:
            node = stack.pop()
            stack.extend(node.children.values())
            yield node

    # -- lookup ---------------------------------------------------------------------------
    def longest_prefix_tokens(self, fingerprint, tokens, *, minimum_tokens=1):
        with self._lock:
            count = len(self._follow(fingerprint, tuple(tokens))) * self.block_tokens
            return count if count >= minimum_tokens else 0

    def lookup(self, fingerprint, tokens, *, minimum_tokens=1):
        """A ``BlockPrefixMatch`` holding new references to the matched pages
        (per layer, in prompt order), or None."""
        with self._lock:
            path = self._follow(fingerprint, tuple(tokens))
            count = len(path) * self.block_tokens
            if not path or count < minimum_tokens:
                self.misses += 1
                return None
            layers = len(path[0].pages)
            refs = [[] for _ in range(layers)]
            try:
                for node in path:
                    for layer, (pool, block_id) in enumerate(node.pages):
                        refs[layer].append(BlockRef(pool, block_id, acquired=True))
            except BaseException:
                for layer in refs:
                    for ref in layer:
                        ref.close()
                raise
            self._touch(path)
            self.hits += 1
            self.tokens_reused += count
            return BlockPrefixMatch(count, tuple(tuple(layer) for layer in refs),
                                    layers * len(path))

    # -- publication ----------------------------------------------------------------------
    def publish(self, fingerprint, tokens, layer_blocks):
        """Index the complete sealed pages of a prompt (``layer_blocks[layer]``:
        that layer's ``BlockRef``s in prompt order); returns how many new
        pages (trie nodes) the index holds after its budgets are applied."""
        if not layer_blocks or not self.capacity_bytes:
            return 0
        tokens = tuple(tokens)
        count = min(min(len(refs) for refs in layer_blocks), len(tokens) // self.block_tokens)
        # every page is checked before anything is pinned
        for refs in layer_blocks:
            for ref in refs[:count]:
                block = ref.block
                if not block.immutable or block.token_count != self.block_tokens:
                    raise ValueError("prefix publication requires sealed complete pages")
        with self._lock:
            root = self._roots.get(fingerprint)
            if root is None:
                root = self._roots[fingerprint] = _Node(fingerprint.digest, None, (), (), 0, 0)
            node, path, made = root, [], []
            try:
                for index, chunk in enumerate(self._chunks(tokens, count)):
                    child = node.children.get(chunk)
                    if child is None:
                        pages = tuple((refs[index].pool, refs[index].block_id)
                                      for refs in layer_blocks)
                        child = self._attach(node, chunk, pages)
                        made.append(child)
                    path.append(child)
                    node = child
            except BaseException:
                for child in reversed(made):
                    self._detach(child)
                raise
            self._touch(path)
            self._shrink()
            return sum(child.attached for child in made)

    def _attach(self, parent, chunk, pages):
        """A new node under ``parent``: its pages pinned (all or none)."""
        pinned = []
        try:
            for pool, block_id in pages:
                pool.pin(block_id)
                pinned.append((pool, block_id))
        except BaseException:
            for pool, block_id in reversed(pinned):
                pool.unpin(block_id)
            raise
        page_bytes = sum(pool.get(block_id).nbytes for pool, block_id in pages)
        node = _Node(chain_key(parent.key, chunk), parent, chunk, pages, page_bytes,
                     parent.depth + 1)
        parent.children[chunk] = node
        self._count += 1
        self._page_bytes += node.page_bytes
        self._meta_bytes += node.meta_bytes
        return node

    def _detach(self, node):
        """Unlink a leaf and unpin its pages; a parent left childless becomes
        a leaf candidate."""
        parent = node.parent
        del parent.children[node.chunk]
        node.attached = False
        self._count -= 1
        self._page_bytes -= node.page_bytes
        self._meta_bytes -= node.meta_bytes
        for pool, block_id in node.pages:
            pool.unpin(block_id)
        if parent.parent is not None and not parent.children:
            heapq.heappush(self._leaves, (parent.stamp, next(self._tie), parent))

    def _shrink(self):
        """Least recently used leaves go until both budgets hold."""
        while self._count and self._over_budget():
            stamp, _, node = heapq.heappop(self._leaves)
            if node.attached and not node.children and node.stamp == stamp:
                self._detach(node)
                self.evictions += 1

    def clear(self):
        with self._lock:
            for node in list(self._nodes()):
                node.attached = False
                for pool, block_id in node.pages:
                    pool.unpin(block_id)
            self._roots.clear()
            self._leaves.clear()
            self._count = self._page_bytes = self._meta_bytes = 0

    def stats(self):
        with self._lock:
            return {"entries": self._count, "bytes": self._page_bytes,
                    "metadata_bytes": self._meta_bytes, "capacity_bytes": self.capacity_bytes,
                    "hits": self.hits, "misses": self.misses, "evictions": self.evictions,
                    "tokens_reused": self.tokens_reused}
