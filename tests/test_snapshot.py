"""CPU: paged snapshots on disk (``pkv.snapshot``; the reference's
``engine/components.py:317-530`` snapshot protocol with page-image storage).

Round trip of page bytes, token counts and offsets into a fresh arena; the
manifest is the commit point (payload digest, identity, layout and schema are
checked before anything is allocated); an older payload is removed on the
next save.
"""

from __future__ import annotations

import json

import numpy as np
import pytest

from pkv.cache_manager import CacheConfig, CacheManager
from pkv.layer import ModelSpec
from pkv.snapshot import load_snapshot, save_snapshot

torch = pytest.importorskip("torch")


class _Bundle:
    def __init__(self, spec):
        self.spec = spec
        self.activation_dtype = spec.dtype


def _manager():
    spec = ModelSpec(hidden=256, query_heads=8, kv_heads=2, head_dim=64, num_layers=3,
                     dtype="float16")
    return CacheManager(_Bundle(spec), CacheConfig(block_size_tokens=16, group_size=32),
                        device="cpu")


def _filled(cm, tokens, seed=0):
    h = cm.create_handle("r", key_type="q8_0", value_type="q8_0")
    rng = np.random.default_rng(seed)
    for cache in h.bundle.entries:
        layout = cache.layout_for(2, 64)
        cache._plan_append(tokens, layout)
        pool = cache.pool.pool_for(layout)
        for ref in cache._blocks:
            pool.buffer[ref.block.page] = torch.from_numpy(
                rng.integers(0, 256, pool.page_bytes, dtype=np.uint8))
    return h


def _bytes(cache):
    pool = cache.pool.pool_for(cache.layout)
    return [pool.buffer[r.block.page].clone() for r in cache._blocks]


@pytest.mark.parametrize("fmt", ["npz", "safetensors"])
def test_round_trip_restores_pages_counts_and_offsets(tmp_path, fmt):
    cm = _manager()
    h = _filled(cm, 53)
    manifest = save_snapshot(tmp_path, h.bundle, identity="model-a", tensor_format=fmt)
    assert manifest["schema_version"] == "pkv-pages-v1" and len(manifest["layers"]) == 3
    other = _manager()
    restored = load_snapshot(tmp_path, identity="model-a", expected_specs=other.layer_specs,
                             page_pool=other.block_pool, bits=8)
    for mine, theirs in zip(restored.entries, h.bundle.entries, strict=True):
        assert mine.offset == theirs.offset == 53 and mine.bits == 8
        assert [r.block.token_count for r in mine._blocks] == [16, 16, 16, 5]
        assert [r.block.immutable for r in mine._blocks] == [True, True, True, False]
        assert all(torch.equal(a, b) for a, b in zip(_bytes(mine), _bytes(theirs), strict=True))
        assert mine.page_table.pages == [r.block.page for r in mine._blocks]


def test_manifest_is_checked_before_anything_is_allocated(tmp_path):
    cm = _manager()
    h = _filled(cm, 40)
    manifest = save_snapshot(tmp_path, h.bundle, identity="model-a")
    other = _manager()
    with pytest.raises(ValueError, match="identity"):
        load_snapshot(tmp_path, identity="model-b", expected_specs=other.layer_specs,
                      page_pool=other.block_pool)
    with pytest.raises(ValueError, match="layout"):
        load_snapshot(tmp_path, identity="model-a", expected_specs=other.layer_specs,
                      page_pool=other.block_pool, bits=4)
    payload = tmp_path / manifest["payload"]
    data = bytearray(payload.read_bytes())
    data[len(data) // 2] ^= 0xFF
    payload.write_bytes(bytes(data))
    with pytest.raises(ValueError, match="digest"):
        load_snapshot(tmp_path, identity="model-a", expected_specs=other.layer_specs,
                      page_pool=other.block_pool)
    assert other.block_pool.nbytes == 0


def test_a_new_save_replaces_the_payload_and_empty_caches_round_trip(tmp_path):
    cm = _manager()
    first = save_snapshot(tmp_path, _filled(cm, 20).bundle, identity="m")
    empty = cm.create_handle("e", key_type="q8_0", value_type="q8_0")
    second = save_snapshot(tmp_path, empty.bundle, identity="m")
    assert not (tmp_path / first["payload"]).exists() and (tmp_path / second["payload"]).exists()
    assert json.loads((tmp_path / "state.json").read_text())["payload"] == second["payload"]
    other = _manager()
    restored = load_snapshot(tmp_path, identity="m", expected_specs=other.layer_specs,
                             page_pool=other.block_pool, bits=8, dtype="float16")
    assert [c.offset for c in restored.entries] == [0, 0, 0]
    with pytest.raises(ValueError):
        save_snapshot(tmp_path, [], identity="m")


# ---------------------------------------------------------------- cold prefix tier
# ColdPrefixStore and the manager's fallback to it (engine/cold_prefix.py:93-240,
# engine/cache_manager.py:499-559).


def _cold_manager(directory, **kw):
    spec = ModelSpec(hidden=256, query_heads=8, kv_heads=2, head_dim=64, num_layers=3,
                     dtype="float16")
    config = CacheConfig(block_size_tokens=16, group_size=32, prefix_cache_enabled=True,
                         ssd_cache_directory=str(directory), **kw)
    return CacheManager(_Bundle(spec), config, device="cpu")


def test_cold_tier_restores_a_prefix_another_manager_published(tmp_path):
    cm = _cold_manager(tmp_path)
    fp = cm.fingerprint(key_type="q8_0", value_type="q8_0")
    prompt = tuple(range(300, 353))                      # 53 tokens
    h = _filled(cm, 53)
    h.token_count = 53
    assert cm.publish_prefix(h, fp, prompt)
    assert cm.cold_prefix.stats()["entries"] == 1
    fresh = _cold_manager(tmp_path)                     # empty in-memory index: disk only
    g = fresh.create_handle("g", key_type="q8_0", value_type="q8_0")
    assert fresh.adopt_prefix(g, fp, prompt[:40] + (1, 2, 3)) == 32   # page-aligned match
    for mine, theirs in zip(g.bundle.entries, h.bundle.entries, strict=True):
        assert mine.offset == 32
        assert all(torch.equal(a, b) for a, b in zip(_bytes(mine), _bytes(theirs)[:2], strict=True))
    assert fresh.cold_prefix.stats()["hits"] == 1
    other = fresh.fingerprint(key_type="q8_0", value_type="q8_0", namespace="tenant-b")
    assert fresh.adopt_prefix(fresh.create_handle("x", key_type="q8_0", value_type="q8_0"),
                              other, prompt) == 0


def test_cold_tier_budget_and_corruption(tmp_path):
    cm = _cold_manager(tmp_path, ssd_max_entries=2)
    fp = cm.fingerprint(key_type="q8_0", value_type="q8_0")
    for n in range(3):
        h = _filled(cm, 20 + n, seed=n)
        cm.publish_prefix(h, fp, tuple(range(n * 100, n * 100 + 20 + n)))
        cm.release(h)
    store = cm.cold_prefix
    assert store.stats()["entries"] == 2 and store.stats()["evictions"] == 1   # the oldest left
    assert len(list(tmp_path.glob("*.pkvc"))) == 2
    assert store.preview(fp, tuple(range(0, 21)) + (9,)) == 0
    assert store.preview(fp, tuple(range(200, 222)) + (9,)) == 16
    # a flipped payload byte is caught before any page is taken
    newest = max(tmp_path.glob("*.pkvc"), key=lambda p: p.stat().st_mtime)
    raw = bytearray(newest.read_bytes())
    raw[-1] ^= 0xFF
    newest.write_bytes(bytes(raw))
    live = cm.block_pool.stats()["block_live"]
    with pytest.raises(ValueError, match="checksum"):
        store.lookup(fp, tuple(range(200, 222)) + (9,), cm.layer_specs, page_pool=cm.block_pool)
    assert cm.block_pool.stats()["block_live"] == live
    # a reopened store rebuilds its catalog from the entries' headers
    again = _cold_manager(tmp_path, ssd_max_entries=2).cold_prefix
    assert again.stats()["entries"] == 2
    assert again.preview(fp, tuple(range(100, 121)) + (9,)) == 16
    store.clear()
    assert store.stats()["entries"] == 0 and not list(tmp_path.glob("*.pkvc"))


def test_cold_tier_refuses_foreign_directories_and_replaces_extended_entries(tmp_path):
    (tmp_path / "notes.txt").write_text("not a cache")
    with pytest.raises(ValueError, match="not empty"):
        _cold_manager(tmp_path)
    root = tmp_path / "cold"
    cm = _cold_manager(root)
    fp = cm.fingerprint(key_type="q8_0", value_type="q8_0")
    prompt = tuple(range(1000, 1070))
    short = _filled(cm, 33, seed=1)
    assert cm.cold_prefix.put(fp, prompt[:33], short.bundle, page_tokens=16)
    assert not cm.cold_prefix.put(fp, prompt[:33], short.bundle, page_tokens=16)  # held already
    long = _filled(cm, 70, seed=1)
    assert cm.cold_prefix.put(fp, prompt, long.bundle, page_tokens=16)
    assert cm.cold_prefix.stats()["entries"] == 1        # the 2-page entry was extended
    assert cm.cold_prefix.preview(fp, prompt + (5,)) == 64
    assert cm.cold_prefix.preview(fp, prompt[:20] + (5, 6, 7)) == 16
    assert cm.cold_prefix.preview(fp, prompt[:16]) == 0  # never the last token
    cancelled = _filled(cm, 40, seed=2)
    assert not cm.cold_prefix.put(fp, tuple(range(40)), cancelled.bundle, page_tokens=16,
                                  cancelled=lambda: True)
    (root / "stray.bin").write_bytes(b"x")
    with pytest.raises(ValueError, match="foreign"):
        _cold_manager(root)
