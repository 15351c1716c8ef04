"""The reference-named cache API over device-side page ownership.

``CacheManager(bundle, CacheConfig(backend="paged", page_arena="device", ...))``
keeps the reference's interface (``engine/cache_manager.py``: ``create_handle``,
``adopt_prefix`` / ``publish_prefix``, ``release``, budgets) but gives each
handle one sequence slot of a ``DevicePageArena``: its per-layer entries are
``SlotLayerCache`` views of that slot, and ``PagedRunner.execute`` runs such a
batch as ``DeviceRunner`` does -- one page reservation kernel for the batch
and every layer, append and attention straight from the reservation's device
operands, rollback by truncation -- so a step carries no host page
bookkeeping (``engine/paged.py:308-417`` is the host-bookkept original).

Per-layer mutation outside the runner (``append``, ``clone``, ``adopt``,
``trim``) is what the device arena cannot do layer by layer: every layer of a
slot grows together.  Those calls raise ``ModelCapabilityUnsupported``; the
slot-wide equivalents are the arena's ``reserve`` / ``fork`` / ``truncate``.

Shared prefixes (``DevicePrefixIndex``): a published prompt is kept as a
forked slot holding its page-aligned prefix (one more reference per page, no
copy); a later request adopts the longest match by forking that slot and
truncating to the matched pages.  Prompt pages are keyed with the host
index's chained block keys (``prefix_cache.chain_key``), never taking a
prompt's last token, and entries leave least recently used first past a page
budget.
"""

from __future__ import annotations

import time
from dataclasses import dataclass

from pkv.modes import ModelCapabilityUnsupported
from pkv.prefix_cache import chain_key


class SlotLayerCache:
    """Layer ``layer_id`` of sequence slot ``slot`` in ``arena``: the names of
    ``PagedKVCache`` that the runner and the manager read."""

    def __init__(self, arena, slot, layer_id, dtype, bits, group_size, layout):
        self.arena, self.slot, self.layer_id = arena, slot, layer_id
        self.dtype, self.bits, self.group_size = dtype, bits, group_size
        self._layout = layout

    @property
    def pool(self):
        return self.arena

    @property
    def block_tokens(self):
        return self.arena.page_tokens

    @property
    def offset(self):
        return self.arena.lengths[self.slot]

    @property
    def layout(self):
        return self._layout

    @property
    def nbytes(self):
        return -(-self.offset // self.block_tokens) * self.arena.fmt.page_bytes

    def reset(self):
        """Slot-wide: the manager's ``release`` returns the slot; a layer alone
        holds nothing to drop."""

    release = reset

    def _unsupported(self, *_a, **_k):
        raise ModelCapabilityUnsupported(
            "device-arena caches advance through PagedRunner.execute (slot-wide reserve, "
            "fork and truncate); per-layer edits are not available")

    append = clone = snapshot = adopt = trim = replace_from = _unsupported

    def update(self, *_):
        raise ModelCapabilityUnsupported("paged cache requires direct attention dispatch")

    def state(self):
        raise ModelCapabilityUnsupported("paged histories cannot be materialized")


@dataclass
class _Prefix:
    fingerprint: str
    keys: tuple          # chained key of each page of the prefix
    slot: int            # the slot holding the prefix pages
    last_access: float


class DevicePrefixIndex:
    """Published prompt prefixes as forked slots of one ``DevicePageArena``."""

    def __init__(self, arena, *, capacity_pages, max_entries):
        self.arena = arena
        self.capacity_pages, self.max_entries = int(capacity_pages), int(max_entries)
        self._entries = []

    def _keys(self, fingerprint, tokens, pages):
        keys, parent = [], fingerprint.digest
        p = self.arena.page_tokens
        for i in range(pages):
            parent = chain_key(parent, tokens[i * p:(i + 1) * p])
            keys.append(parent)
        return tuple(keys)

    def _drop(self, entry):
        self._entries.remove(entry)
        self.arena.release([entry.slot])

    def publish(self, slot, fingerprint, tokens):
        """Keep the page-aligned prefix of ``tokens`` that ``slot`` holds; True
        when a new entry was made."""
        tokens = tuple(int(t) for t in tokens)
        pages = min(len(tokens), self.arena.lengths[slot]) // self.arena.page_tokens
        if pages == 0 or pages > self.capacity_pages:
            return False
        keys = self._keys(fingerprint, tokens, pages)
        for entry in self._entries:
            if entry.fingerprint == fingerprint.digest and entry.keys[:pages] == keys:
                entry.last_access = time.monotonic()
                return False
        # room: least recently used entries leave first
        while self._entries and (len(self._entries) >= self.max_entries or
                                 sum(len(e.keys) for e in self._entries) + pages
                                 > self.capacity_pages):
            self._drop(min(self._entries, key=lambda e: e.last_access))
        holder = self.arena.open_slot()
        try:
            self.arena.fork([slot], [holder])
            if self.arena.lengths[holder] > pages * self.arena.page_tokens:
                self.arena.truncate([holder], [pages * self.arena.page_tokens])
        except BaseException:
            self.arena.release([holder])
            raise
        for entry in list(self._entries):         # entries this one extends
            if entry.fingerprint == fingerprint.digest and keys[:len(entry.keys)] == entry.keys:
                self._drop(entry)
        self._entries.append(_Prefix(fingerprint.digest, keys, holder, time.monotonic()))
        return True

    def longest(self, fingerprint, tokens, minimum=1):
        """(entry, pages) of the longest published prefix of ``tokens`` (never
        its last token), or (None, 0)."""
        tokens = tuple(int(t) for t in tokens)
        usable = max(len(tokens) - 1, 0) // self.arena.page_tokens
        query = self._keys(fingerprint, tokens, usable)
        best, pages = None, 0
        for entry in self._entries:
            if entry.fingerprint != fingerprint.digest:
                continue
            n, top = 0, min(len(query), len(entry.keys))
            while n < top and query[n] == entry.keys[n]:
                n += 1
            if n > pages:
                best, pages = entry, n
        if best is None or pages * self.arena.page_tokens < max(minimum, 1):
            return None, 0
        return best, pages

    def adopt(self, slot, entry, pages):
        """The (empty) ``slot`` takes the entry's first ``pages`` pages by
        reference; returns the tokens adopted."""
        if self.arena.lengths[slot]:
            raise ValueError("prefix adoption requires an empty cache")
        self.arena.fork([entry.slot], [slot])
        tokens = pages * self.arena.page_tokens
        if self.arena.lengths[slot] > tokens:
            self.arena.truncate([slot], [tokens])
        entry.last_access = time.monotonic()
        return tokens

    @property
    def entries(self):
        return len(self._entries)

    def clear(self):
        for entry in list(self._entries):
            self._drop(entry)
