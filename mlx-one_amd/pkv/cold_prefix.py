"""Cold (on-disk) prefix tier: the reference's ``ColdPrefixStore`` (``engine/cold_prefix.py:93-240``).

A dedicated directory of generations -- one snapshot (``pkv.snapshot``, page
images) per published prompt -- and ``index.json`` listing them (identity =
the fingerprint digest, prompt tokens, bytes, page size, the manifest's
sha256), itself checksummed.  ``put`` writes a generation and publishes it by
rewriting the index (oldest entries leave first past the entry or byte
budget; obsolete generations are deleted under the exclusive lock);
``lookup`` picks the record sharing the longest page-aligned prefix with the
prompt (never its last token), checks the manifest digest and the byte count
before loading, restores the pages into the caller's arena and trims them to
the match.
"""

from __future__ import annotations

import hashlib
import json
import os
import shutil
import tempfile
import uuid
from pathlib import Path

from pkv.snapshot import _lock, load_snapshot, save_snapshot

COLD_PREFIX_VERSION = "pkv-cold-prefix-v1"


def _digest(value):
    return hashlib.sha256(json.dumps(value, sort_keys=True, separators=(",", ":")).encode()).hexdigest()


def _atomic_json(path, data):
    with tempfile.NamedTemporaryFile("w", dir=path.parent, delete=False) as handle:
        temporary = Path(handle.name)
        handle.write(json.dumps(data, sort_keys=True) + "\n")
        handle.flush()
        os.fsync(handle.fileno())
    os.replace(temporary, path)


class ColdPrefixStore:
    def __init__(self, directory, *, budget_bytes, max_entries=128, staging_bytes=256 << 20):
        if min(budget_bytes, max_entries, staging_bytes) < 1:
            raise ValueError("cold prefix tier requires positive byte and entry limits")
        self.root = Path(directory).expanduser().resolve()
        self.root.mkdir(parents=True, exist_ok=True)
        self.budget, self.max_entries, self.staging = budget_bytes, max_entries, staging_bytes
        self.hits = self.misses = self.rejections = 0

    # -- index ------------------------------------------------------------------------
    def _index(self):
        path = self.root / "index.json"
        if not path.exists():
            if any(p.name != ".state.lock" for p in self.root.iterdir()):
                raise ValueError("SSD cache directory must be dedicated to prefix storage")
            return []
        if path.stat().st_size > 16 << 20:
            raise ValueError("cold index metadata exceeds limit")
        data = json.loads(path.read_text())
        if data.get("schema") != COLD_PREFIX_VERSION or data.get("sha256") != _digest(data["entries"]):
            raise ValueError("cold index checksum/schema mismatch")
        records = data["entries"]
        if not isinstance(records, list) or len(records) > self.max_entries:
            raise ValueError("cold index entry limit mismatch")
        for r in records:
            generation = r.get("generation")
            if (not isinstance(generation, str) or len(generation) != 32
                    or any(c not in "0123456789abcdef" for c in generation)
                    or not isinstance(r.get("bytes"), int) or r["bytes"] < 0
                    or not isinstance(r.get("tokens"), list)
                    or any(type(t) is not int or t < 0 for t in r["tokens"])):
                raise ValueError("invalid cold prefix record")
        return records

    @staticmethod
    def _match(record, identity, tokens, minimum):
        """Tokens of the prompt the record can give back (page-aligned, last token excluded)."""
        if record["identity"] != identity:
            return 0
        count = 0
        for a, b in zip(record["tokens"], tokens[:-1]):
            if a != b:
                break
            count += 1
        page = record["page_tokens"]
        if page:
            count = count // page * page
        return count if count >= minimum else 0

    def preview(self, fingerprint, tokens, *, minimum=1):
        with _lock(self.root, exclusive=False):
            return max((self._match(r, fingerprint.digest, tuple(tokens), minimum)
                        for r in self._index()), default=0)

    # -- publication ---------------------------------------------------------------------
    def put(self, fingerprint, tokens, bundle, *, page_tokens, cancelled=lambda: False):
        """Store ``bundle`` (holding exactly ``tokens``) as a generation."""
        tokens = tuple(int(t) for t in tokens)
        if (not tokens or fingerprint.multimodal_identity is not None
                or bundle.offset != len(tokens) or cancelled()):
            return False
        estimate = bundle.nbytes + 16 * len(tokens) + 65536
        if estimate > self.staging:
            self.rejections += 1
            return False
        generation = uuid.uuid4().hex
        directory = self.root / generation
        identity = {"fingerprint": fingerprint.digest, "prefix_version": COLD_PREFIX_VERSION}
        published = False
        with _lock(self.root, exclusive=True):
            records = self._index()
            try:
                if shutil.disk_usage(self.root).free < estimate:
                    self.rejections += 1
                    return False
                save_snapshot(directory, bundle, identity=identity, tensor_format="safetensors")
                size = sum(p.stat().st_size for p in directory.iterdir() if p.is_file())
                if size > self.budget or cancelled():
                    return False
                record = {"identity": fingerprint.digest, "generation": generation,
                          "tokens": list(tokens), "bytes": size, "page_tokens": int(page_tokens),
                          "state_sha256": hashlib.sha256(
                              (directory / "state.json").read_bytes()).hexdigest()}
                kept = [r for r in records
                        if (r["identity"], r["tokens"]) != (record["identity"], record["tokens"])]
                kept.append(record)
                while len(kept) > self.max_entries or sum(r["bytes"] for r in kept) > self.budget:
                    kept.pop(0)
                _atomic_json(self.root / "index.json", {"schema": COLD_PREFIX_VERSION,
                                                        "entries": kept, "sha256": _digest(kept)})
                published = True
                live = {r["generation"] for r in kept}
                for path in self.root.iterdir():   # obsolete or orphaned generations
                    if path.is_dir() and len(path.name) == 32 and path.name not in live:
                        shutil.rmtree(path)
                return True
            finally:
                if not published:
                    shutil.rmtree(directory, ignore_errors=True)

    # -- restoration ----------------------------------------------------------------------
    def lookup(self, fingerprint, tokens, specs, *, page_pool, minimum=1, bits=None):
        """``(tokens reused, CacheBundle)`` restored into ``page_pool``, or None."""
        tokens = tuple(int(t) for t in tokens)
        with _lock(self.root, exclusive=False):
            scored = [(self._match(r, fingerprint.digest, tokens, minimum), r) for r in self._index()]
            count, record = max(scored, key=lambda pair: pair[0], default=(0, None))
            if not count:
                self.misses += 1
                return None
            directory = self.root / record["generation"]
            if directory.is_symlink() or any(p.is_symlink() for p in directory.iterdir()):
                raise ValueError("cold generation cannot contain symbolic links")
            if record["bytes"] > self.staging or record["bytes"] > self.budget:
                raise ValueError("cold restore exceeds staging/disk policy")
            if hashlib.sha256((directory / "state.json").read_bytes()).hexdigest() != \
                    record["state_sha256"]:
                raise ValueError("cold state manifest checksum mismatch")
            if sum(p.stat().st_size for p in directory.iterdir() if p.is_file()) != record["bytes"]:
                raise ValueError("cold generation byte accounting mismatch")
        identity = {"fingerprint": fingerprint.digest, "prefix_version": COLD_PREFIX_VERSION}
        restored = load_snapshot(directory, identity=identity, expected_specs=specs,
                                 page_pool=page_pool, bits=bits)
        try:
            if restored.offset != len(record["tokens"]):
                raise ValueError("cold committed token identity mismatch")
            for cache in restored.entries:
                if cache.offset != count:
                    cache.trim(cache.offset - count)
            self.hits += 1
            return count, restored
        except BaseException:
            for cache in restored.entries:
                cache.reset()
            raise

    def stats(self):
        with _lock(self.root, exclusive=False):
            records = self._index()
            return {"entries": len(records), "disk_bytes": sum(r["bytes"] for r in records),
                    "budget_bytes": self.budget, "staging_budget_bytes": self.staging,
                    "hits": self.hits, "misses": self.misses, "rejections": self.rejections}

    def clear(self):
        with _lock(self.root, exclusive=True):
            _atomic_json(self.root / "index.json", {"schema": COLD_PREFIX_VERSION, "entries": [],
                                                    "sha256": _digest([])})
            for path in self.root.iterdir():
                if path.is_dir() and len(path.name) == 32:
                    shutil.rmtree(path)
