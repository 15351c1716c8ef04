"""Snapshots of paged caches on disk (``engine/components.py:317-530``, paged storage).

The reference's snapshot is a directory with an immutable tensor payload
(``npz`` or ``safetensors``) and a JSON manifest written last (``state.json``:
the commit point, with the payload's sha256), taken under a file lock; its
paged storage exports each layer's float keys/values (``paged-fp16-v1``).

This build stores what the device holds: each layer's page images, byte for
byte (``pkv-pages-v1``: codes, scales and biases in the kernels' layout, or
float pages), plus each page's token count, so a restore is one copy into
freshly allocated pages -- lossless for quantized caches, where a float export
would be re-quantized on the way back.  With ``reference_pages=True`` (device
pools) the payload also carries every layer's pages in the reference's
per-page tensor format (``quantize_page`` codes / scale / bias, or float K/V,
from ``gather_pages``) for readers of that format.
"""

from __future__ import annotations

import fcntl
import hashlib
import json
import os
import tempfile
import uuid
from contextlib import contextmanager
from pathlib import Path

import numpy as np

from pkv.cache_manager import CacheBundle
from pkv.paged import KERNEL_VERSION, PagedKVCache

SCHEMA = "pkv-pages-v1"


@contextmanager
def _lock(root, exclusive):
    root.mkdir(parents=True, exist_ok=True)
    with (root / ".state.lock").open("a+b") as handle:
        fcntl.flock(handle, fcntl.LOCK_EX if exclusive else fcntl.LOCK_SH)
        try:
            yield
        finally:
            fcntl.flock(handle, fcntl.LOCK_UN)


def _layout_record(layout, page_bytes):
    return {"layer_id": layout.layer_id, "page_tokens": layout.page_tokens,
            "num_kv_heads": layout.num_kv_heads, "head_dim": layout.head_dim,
            "dtype": layout.key_dtype, "bits": layout.quantization_bits,
            "group_size": layout.quantization_group_size,
            "kernel_version": layout.kernel_version, "page_bytes": int(page_bytes)}


def _write_atomic(root, name, data: bytes):
    with tempfile.NamedTemporaryFile(dir=root, delete=False) as handle:
        temporary = Path(handle.name)
        handle.write(data)
        handle.flush()
        os.fsync(handle.fileno())
    os.replace(temporary, root / name)


def save_snapshot(directory, bundle, *, identity, tensor_format="npz", reference_pages=False):
    """Write the caches of ``bundle`` (a ``CacheBundle`` or a sequence of
    ``PagedKVCache``) under ``directory``; returns the manifest."""
    import torch

    if tensor_format not in {"npz", "safetensors"}:
        raise ValueError("unsupported snapshot tensor format")
    entries = tuple(getattr(bundle, "entries", bundle))
    if not entries or any(not isinstance(c, PagedKVCache) for c in entries):
        raise ValueError("a paged snapshot needs PagedKVCache entries")
    if len({c.offset for c in entries}) > 1:
        raise ValueError("snapshot components are not at one committed boundary")
    root = Path(directory)
    tensors, layers = {}, []
    for index, cache in enumerate(entries):
        layer = {"kind": "full_kv", "storage": SCHEMA, "offset": cache.offset,
                 "layer_id": cache.layer_id, "tensors": {}}
        if cache._blocks:
            layout = cache.layout
            pool = cache.pool.pool_for(layout)
            ids = torch.tensor([r.block.page for r in cache._blocks], dtype=torch.int64,
                               device=pool.buffer.device)
            pages = pool.buffer.index_select(0, ids).cpu().numpy()
            counts = np.array([r.block.token_count for r in cache._blocks], np.int32)
            layer["layout"] = _layout_record(layout, pool.page_bytes)
            for name, value in (("pages", pages), ("token_counts", counts)):
                key = f"layer_{index}_{name}"
                tensors[key] = value
                layer["tensors"][name] = {"key": key, "shape": list(value.shape),
                                          "dtype": str(value.dtype)}
            if reference_pages and pool.buffer.is_cuda:
                from pkv import ops

                exported = ops.gather_pages(pool.fmt, pool.buffer, ids.to(torch.int32))
                names = (("k_codes", "k_scale", "k_bias", "v_codes", "v_scale", "v_bias")
                         if len(exported) == 6 else ("keys", "values"))
                for name, value in zip(names, exported, strict=True):
                    key = f"layer_{index}_reference_{name}"
                    array = value.cpu()
                    if array.dtype == torch.bfloat16:     # lossless widening for npz
                        array = array.float()
                    tensors[key] = array.numpy()
                    layer["tensors"][f"reference_{name}"] = {"key": key,
                                                             "shape": list(array.shape),
                                                             "dtype": str(value.dtype)}
        layers.append(layer)
    with _lock(root, exclusive=True):
        payload = f"tensors-{uuid.uuid4().hex}.{tensor_format}"
        if tensor_format == "npz":
            import io

            buffer = io.BytesIO()
            np.savez(buffer, **tensors)
            data = buffer.getvalue()
        else:
            from safetensors.numpy import save

            data = save({k: np.ascontiguousarray(v) for k, v in tensors.items()})
        _write_atomic(root, payload, data)
        manifest = {"schema_version": SCHEMA, "identity": identity, "layers": layers,
                    "payload": payload, "tensor_format": tensor_format,
                    "kernel_version": KERNEL_VERSION, "sha256": hashlib.sha256(data).hexdigest()}
        try:
            _write_atomic(root, "state.json",
                          (json.dumps(manifest, sort_keys=True, indent=2) + "\n").encode())
        except BaseException:
            (root / payload).unlink(missing_ok=True)
            raise
        for old in (*root.glob("tensors-*.npz"), *root.glob("tensors-*.safetensors")):
            if old.name != payload:
                old.unlink()
    return manifest


def _read_tensors(path, tensor_format):
    if tensor_format == "npz":
        with np.load(path, allow_pickle=False) as data:
            return {k: data[k] for k in data.files}
    if tensor_format == "safetensors":
        from safetensors.numpy import load_file

        return load_file(str(path))
    raise ValueError("unsupported snapshot tensor format")


def load_snapshot(directory, *, identity, expected_specs, page_pool, dtype=None, bits=None,
                  group_size=None):
    """Restore a snapshot into fresh pages of ``page_pool`` (a
    ``SegmentedPageArena``): returns a ``CacheBundle`` of ``PagedKVCache``, one
    per spec of ``expected_specs`` (layer shapes).  Identity, schema, payload
    digest and every page layout are checked first; any mismatch raises
    ``ValueError`` and allocates nothing."""
    import torch

    root = Path(directory)
    with _lock(root, exclusive=False):
        manifest = json.loads((root / "state.json").read_text())
        if manifest.get("schema_version") != SCHEMA:
            raise ValueError("unsupported snapshot schema")
        if manifest.get("identity") != identity:
            raise ValueError("snapshot identity mismatch")
        payload = root / manifest["payload"]
        data = payload.read_bytes()
        if hashlib.sha256(data).hexdigest() != manifest["sha256"]:
            raise ValueError("snapshot payload digest mismatch")
        tensors = _read_tensors(payload, manifest["tensor_format"])
    specs = tuple(expected_specs)
    layers = manifest["layers"]
    if len(layers) != len(specs):
        raise ValueError("snapshot layer count does not match the cache plan")
    plans = []
    for spec, layer in zip(specs, layers, strict=True):
        if layer.get("storage") != SCHEMA or layer.get("kind") != "full_kv" \
                or layer.get("layer_id") != spec.layer_id:
            raise ValueError("snapshot layer does not match the cache plan")
        if not layer["offset"]:
            plans.append((spec, layer, None, None, None))
            continue
        rec = layer["layout"]
        if (rec["page_tokens"] != page_pool.block_tokens or rec["num_kv_heads"] != spec.num_kv_heads
                or rec["head_dim"] != spec.key_head_dim or rec["kernel_version"] != KERNEL_VERSION
                or (dtype is not None and rec["dtype"] != dtype)
                or (bits is not None and rec["bits"] != bits)
                or (group_size is not None and rec["group_size"] != group_size)):
            raise ValueError("snapshot page layout does not match the arena")
        pages = tensors[layer["tensors"]["pages"]["key"]]
        counts = tensors[layer["tensors"]["token_counts"]["key"]]
        if (pages.dtype != np.uint8 or pages.ndim != 2 or pages.shape[1] != rec["page_bytes"]
                or len(counts) != len(pages) or int(counts.sum()) != layer["offset"]
                or any(int(c) != rec["page_tokens"] for c in counts[:-1])
                or not 0 < int(counts[-1]) <= rec["page_tokens"]):
            raise ValueError("snapshot pages are inconsistent")
        plans.append((spec, layer, rec, pages, counts))
    caches = []
    try:
        for spec, layer, rec, pages, counts in plans:
            if rec is None:
                caches.append(PagedKVCache(page_pool, layer_id=spec.layer_id,
                                           dtype=dtype or "float16", bits=bits,
                                           group_size=group_size or 32))
                continue
            cache = PagedKVCache(page_pool, layer_id=spec.layer_id, dtype=rec["dtype"],
                                 bits=rec["bits"], group_size=rec["group_size"])
            caches.append(cache)
            layout = cache.layout_for(rec["num_kv_heads"], rec["head_dim"])
            pool = page_pool.pool_for(layout)
            if pool.page_bytes != rec["page_bytes"]:
                raise ValueError("snapshot page size does not match this build's page format")
            cache._plan_append(int(counts.sum()), layout)   # takes and seals the pages
            ids = torch.tensor([r.block.page for r in cache._blocks], dtype=torch.int64,
                               device=pool.buffer.device)
            pool.buffer.index_copy_(0, ids, torch.from_numpy(pages).to(pool.buffer.device))
    except BaseException:
        for cache in caches:
            cache.reset()
        raise
    return CacheBundle(tuple(caches))
