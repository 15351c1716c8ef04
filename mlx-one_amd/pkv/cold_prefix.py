"""Cold tier of the prefix cache: published prefixes kept on disk as page images.

Interface of the reference's ``ColdPrefixStore`` (``engine/cold_prefix.py:93``:
``ColdPrefixStore(directory, budget_bytes=, max_entries=)`` with ``put``,
``lookup``, ``preview``, ``stats``, ``clear``), used by ``CacheManager`` when
the in-memory ``BlockPrefixIndex`` misses.  The storage is this build's own:

* **One file per entry**, ``<name>.pkvc``: the 8-byte magic ``PKVCOLD1``, a
  little-endian u32 header length, a JSON header, then the payload -- every
  layer's page images in order, ``[pages, page_bytes]`` bytes each, exactly as
  the device pools hold them (codes, scales and biases in the kernels' layout,
  or float pages).  A restore is one host-to-device copy into fresh pages,
  lossless for quantized caches.
* **Page-chain keys.**  Page ``i`` of an entry is keyed by a 16-byte BLAKE2b
  digest of the previous key and the page's token ids (int32, little endian),
  starting from the cache fingerprint's digest.  A lookup keys the query's
  full pages the same way (never its last token, which the caller must
  compute) and takes the entry sharing the longest run of leading keys: a
  page-aligned longest common prefix, in memory, with no file read.
* **No shared index file.**  The catalog (fingerprint, keys, size, last use)
  is rebuilt at start-up from the entries' headers; each entry is written to a
  temporary file and renamed into place, so a crash leaves either the whole
  entry or nothing.  The directory carries a marker file and must hold nothing
  else: ``clear`` deletes entries only from a directory this store owns.
* **Integrity.**  The header records the payload's byte count and SHA-256 and
  each layer's page layout; a lookup checks all of them (and this build's page
  size) before it allocates a page, and raises ``ValueError`` on a mismatch.
* **Budget.**  Total entry bytes and entry count are bounded; the least
  recently used entries leave first, an entry that another one extends is
  replaced by it, and an entry larger than the whole budget is not kept.
"""

from __future__ import annotations

import hashlib
import json
import os
import struct
import threading
import time
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

MAGIC = b"PKVCOLD1"
FORMAT = "pkv-cold-pages-v1"
MARKER = ".pkv-cold-prefix"
SUFFIX = ".pkvc"
MAX_HEADER_BYTES = 64 << 20


def page_keys(fingerprint_digest, tokens, page_tokens, pages):
    """The chain keys (hex) of the first ``pages`` full pages of ``tokens``."""
    keys, parent = [], fingerprint_digest.encode()
    ids = np.asarray(tokens[:pages * page_tokens], dtype="<i4")
    for i in range(pages):
        h = hashlib.blake2b(parent, digest_size=16)
        h.update(ids[i * page_tokens:(i + 1) * page_tokens].tobytes())
        parent = h.digest()
        keys.append(parent.hex())
    return keys


@dataclass
class _Entry:
    name: str
    fingerprint: str
    page_tokens: int
    keys: tuple
    nbytes: int
    payload_bytes: int
    last_used: float = field(default=0.0)


class ColdPrefixStore:
    def __init__(self, directory, *, budget_bytes, max_entries=128, staging_bytes=256 << 20):
        if budget_bytes < 1 or max_entries < 1 or staging_bytes < 1:
            raise ValueError("cold prefix budgets must be positive")
        self.root = Path(directory)
        self.budget_bytes, self.max_entries = int(budget_bytes), int(max_entries)
        self.staging = int(staging_bytes)          # host bytes a restore may stage
        self._lock = threading.RLock()
        self._entries = {}
        self._counts = {"hits": 0, "misses": 0, "writes": 0, "evictions": 0}
        self.root.mkdir(parents=True, exist_ok=True)
        marker = self.root / MARKER
        if not marker.exists():
            stray = [p.name for p in self.root.iterdir()]
            if stray:
                raise ValueError("cold prefix directory is not empty and not a cold prefix "
                                 f"store (found {stray[0]!r})")
            marker.write_text(FORMAT + "\n")
        for path in self.root.iterdir():
            if path.name == MARKER:
                continue
            if path.name.endswith(".tmp"):      # an interrupted write
                path.unlink(missing_ok=True)
                continue
            if path.suffix != SUFFIX or path.is_symlink() or not path.is_file():
                raise ValueError(f"cold prefix directory holds a foreign file {path.name!r}")
            try:
                header, _ = self._read_header(path)
            except ValueError:
                continue                        # unreadable entries are never served
            self._entries[path.stem] = _Entry(path.stem, header["fingerprint"],
                                              int(header["page_tokens"]),
                                              tuple(header["keys"]), path.stat().st_size,
                                              int(header["payload_bytes"]),
                                              path.stat().st_mtime)

    # -- file format ---------------------------------------------------------------
    def _path(self, name):
        return self.root / (name + SUFFIX)

    @staticmethod
    def _read_header(path):
        with open(path, "rb") as f:
            head = f.read(12)
            if len(head) != 12 or head[:8] != MAGIC:
                raise ValueError("not a cold prefix entry")
            (length,) = struct.unpack("<I", head[8:])
            if length > MAX_HEADER_BYTES:
                raise ValueError("cold prefix header too large")
            raw = f.read(length)
        if len(raw) != length:
            raise ValueError("truncated cold prefix header")
        header = json.loads(raw.decode())
        if header.get("format") != FORMAT:
            raise ValueError("unsupported cold prefix format")
        return header, 12 + length

    # -- matching -------------------------------------------------------------------
    def _best(self, fingerprint, tokens, minimum):
        """(entry, matched pages) of the longest page-aligned prefix, or (None, 0)."""
        digest = fingerprint.digest
        candidates = [e for e in self._entries.values() if e.fingerprint == digest]
        if not candidates:
            return None, 0
        queries = {}                                # page size -> the query's keys
        best, pages = None, 0
        for entry in candidates:
            page = entry.page_tokens
            if page not in queries:
                usable = max(len(tokens) - 1, 0) // page     # never the last token
                queries[page] = page_keys(digest, tokens, page, usable)
            query = queries[page]
            n, top = 0, min(len(query), len(entry.keys))
            while n < top and query[n] == entry.keys[n]:
                n += 1
            if n * page > pages * (best.page_tokens if best else 1):
                best, pages = entry, n
        if best is None or pages * best.page_tokens < max(minimum, 1):
            return None, 0
        return best, pages

    def preview(self, fingerprint, tokens, *, minimum=1):
        """Tokens a ``lookup`` would restore (from the catalog: no file is read)."""
        with self._lock:
            entry, pages = self._best(fingerprint, tuple(tokens), minimum)
            return 0 if entry is None else pages * entry.page_tokens

    # -- writes ---------------------------------------------------------------------
    def put(self, fingerprint, tokens, bundle, *, page_tokens, cancelled=lambda: False):
        """Store the full pages of ``bundle`` covering ``tokens``; True if written."""
        import torch

        tokens = tuple(int(t) for t in tokens)
        caches = tuple(getattr(bundle, "entries", bundle))
        pages = len(tokens) // page_tokens
        if pages == 0 or not caches or cancelled():
            return False
        if any(c.offset < pages * page_tokens or len(c._blocks) < pages for c in caches):
            return False
        keys = page_keys(fingerprint.digest, tokens, page_tokens, pages)
        with self._lock:
            for entry in self._entries.values():
                if (entry.fingerprint == fingerprint.digest and entry.page_tokens == page_tokens
                        and entry.keys[:pages] == tuple(keys)):
                    entry.last_used = time.time()
                    return False                 # already held (by this or a longer entry)
        layers, images = [], []
        from pkv.snapshot import _layout_record

        for cache in caches:
            layout = cache.layout
            pool = cache.pool.pool_for(layout)
            ids = torch.tensor([r.block.page for r in cache._blocks[:pages]], dtype=torch.int64,
                               device=pool.buffer.device)
            images.append(pool.buffer.index_select(0, ids).cpu().numpy())
            layers.append({"layer_id": cache.layer_id, "pages": pages,
                           "layout": _layout_record(layout, pool.page_bytes)})
        if cancelled():
            return False
        payload = b"".join(np.ascontiguousarray(a).tobytes() for a in images)
        header = {"format": FORMAT, "fingerprint": fingerprint.digest, "page_tokens": page_tokens,
                  "tokens": pages * page_tokens, "keys": keys, "layers": layers,
                  "payload_bytes": len(payload),
                  "payload_sha256": hashlib.sha256(payload).hexdigest(),
                  "written": time.time()}
        raw = json.dumps(header, sort_keys=True).encode()
        size = 12 + len(raw) + len(payload)
        if size > self.budget_bytes or len(payload) > self.staging:
            return False
        name = keys[-1]
        with self._lock:
            self._make_room(size)
            temporary = self.root / f".{name}.tmp"
            with open(temporary, "wb") as f:
                f.write(MAGIC + struct.pack("<I", len(raw)) + raw)
                f.write(payload)
                f.flush()
                os.fsync(f.fileno())
            os.replace(temporary, self._path(name))
            self._entries[name] = _Entry(name, fingerprint.digest, page_tokens, tuple(keys),
                                         size, len(payload), time.time())
            self._counts["writes"] += 1
            # entries this one extends are now redundant
            for other in list(self._entries.values()):
                if (other.name != name and other.fingerprint == fingerprint.digest
                        and other.page_tokens == page_tokens and len(other.keys) < pages
                        and tuple(keys[:len(other.keys)]) == other.keys):
                    self._drop(other)
        return True

    def _drop(self, entry):
        self._entries.pop(entry.name, None)
        self._path(entry.name).unlink(missing_ok=True)

    def _make_room(self, size):
        """Evict least recently used entries until ``size`` more bytes and one
        more entry fit the budgets."""
        while self._entries and (
                sum(e.nbytes for e in self._entries.values()) + size > self.budget_bytes
                or len(self._entries) + 1 > self.max_entries):
            oldest = min(self._entries.values(), key=lambda e: e.last_used)
            self._drop(oldest)
            self._counts["evictions"] += 1

    # -- reads ----------------------------------------------------------------------
    def lookup(self, fingerprint, tokens, specs, *, page_pool, minimum=1, bits=None):
        """Restore the longest stored page-aligned prefix of ``tokens`` into fresh
        pages of ``page_pool``: ``(tokens restored, CacheBundle)`` or None.  The
        entry is checked in full before any page is taken."""
        import torch

        from pkv.cache_manager import CacheBundle
        from pkv.paged import KERNEL_VERSION, PagedKVCache

        tokens = tuple(int(t) for t in tokens)
        specs = tuple(specs)
        with self._lock:
            entry, pages = self._best(fingerprint, tokens, minimum)
            if entry is None:
                self._counts["misses"] += 1
                return None
            path = self._path(entry.name)
            if path.is_symlink():
                raise ValueError("cold prefix entry is a symbolic link")
            header, offset = self._read_header(path)
            if entry.payload_bytes > self.staging:
                self._counts["misses"] += 1
                return None
            with open(path, "rb") as f:
                f.seek(offset)
                payload = f.read()
            if (len(payload) != int(header["payload_bytes"])
                    or hashlib.sha256(payload).hexdigest() != header["payload_sha256"]):
                raise ValueError("cold prefix entry checksum mismatch")
            if (header["fingerprint"] != fingerprint.digest
                    or header["page_tokens"] != page_pool.block_tokens
                    or len(header["layers"]) != len(specs)):
                raise ValueError("cold prefix entry does not match the cache plan")
            plans, cursor = [], 0
            for spec, layer in zip(specs, header["layers"], strict=True):
                rec = layer["layout"]
                if (layer["layer_id"] != spec.layer_id or rec["num_kv_heads"] != spec.num_kv_heads
                        or rec["head_dim"] != spec.key_head_dim
                        or rec["kernel_version"] != KERNEL_VERSION
                        or (bits is not None and rec["bits"] != bits)
                        or int(layer["pages"]) < pages):
                    raise ValueError("cold prefix page layout does not match the cache plan")
                span = int(layer["pages"]) * int(rec["page_bytes"])
                image = np.frombuffer(payload, np.uint8, span, cursor).reshape(
                    int(layer["pages"]), int(rec["page_bytes"]))
                cursor += span
                plans.append((spec, rec, image[:pages]))
            if cursor != len(payload):
                raise ValueError("cold prefix payload size does not match its layers")
            entry.last_used = time.time()
            os.utime(path)
            self._counts["hits"] += 1
        count = pages * header["page_tokens"]
        caches = []
        try:
            for spec, rec, image in plans:
                cache = PagedKVCache(page_pool, layer_id=spec.layer_id, dtype=rec["dtype"],
                                     bits=rec["bits"], group_size=rec["group_size"])
                caches.append(cache)
                layout = cache.layout_for(rec["num_kv_heads"], rec["head_dim"])
                pool = page_pool.pool_for(layout)
                if pool.page_bytes != int(rec["page_bytes"]):
                    raise ValueError("cold prefix page size differs from this build's page format")
                cache._plan_append(count, layout)          # takes and seals the pages
                ids = torch.tensor([r.block.page for r in cache._blocks], dtype=torch.int64,
                                   device=pool.buffer.device)
                pool.buffer.index_copy_(0, ids, torch.from_numpy(image.copy()).to(
                    pool.buffer.device))
        except BaseException:
            for cache in caches:
                cache.reset()
            raise
        return count, CacheBundle(tuple(caches))

    # -- accounting -----------------------------------------------------------------------
    def stats(self):
        with self._lock:
            return {"entries": len(self._entries),
                    "bytes": sum(e.nbytes for e in self._entries.values()),
                    "budget_bytes": self.budget_bytes, "max_entries": self.max_entries,
                    **self._counts}

    def clear(self):
        """Delete every entry (the store's own files only)."""
        with self._lock:
            for entry in list(self._entries.values()):
                self._drop(entry)
            for path in self.root.glob(f"*{SUFFIX}"):
                path.unlink(missing_ok=True)
