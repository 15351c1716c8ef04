"""Paged KV cache per layer and batched attend (the reference's ``engine/paged.py``).

Same interface and semantics as ``src/mlx_one/engine/paged.py:24-267``:

* ``quantize_page`` / ``dequantize_page`` -- affine unsigned groups, f16 scale
  and bias (:24-54), on the GPU; ``group_size`` generalises the reference's 32.
* ``PagedKVCache`` -- ``append`` / ``clone`` / ``adopt`` / ``trim`` / ``reset``;
  full pages are sealed (immutable, shareable), a shared mutable tail is an
  error, ``update`` and ``state`` refuse to materialise history (:57-206).
* ``PagedBatchCache.attend`` -- query positions taken before the append, so
  each new token attends to itself (:245-267).

MI355X differences: every appended token is quantized as it is written (one
kernel for the whole batch), so a partly filled page reads quantized values
where the reference reads its float tail page; full pages hold bit-identical
codes, scales and biases.  Clone copies the mutable tail page on the device.
"""

from __future__ import annotations

import functools
import math
import time

import numpy as np

from pkv.arena import PersistentPageTable, SegmentedPageArena
from pkv.block_cache import BlockLayout
from pkv.modes import ModelCapabilityUnsupported

KERNEL_VERSION = "mi355x-paged-mfma-v1"
_DTYPES = {"float16", "bfloat16"}


def _torch_dtype(name):
    import torch

    return {"float16": torch.float16, "bfloat16": torch.bfloat16}[name]


def quantize_page(value, bits, group_size=32):
    """``(codes, scale, bias)`` of ``value [..., D]`` (``paged.py:24-41``), on the GPU."""
    from pkv import ops

    if bits not in {4, 8}:
        raise ValueError("paged quantization supports 4 or 8 bits")
    return ops.quantize_rows(value, bits, group_size)


def dequantize_page(state, bits, dim, group_size=32):
    """float32 ``[..., dim]`` from ``(codes, scale, bias)`` (``paged.py:44-54``)."""
    from pkv import ops

    return ops.dequantize_rows(state, bits, dim, group_size)


@functools.lru_cache(maxsize=256)
def _layout(layer_id, page_tokens, heads, dim, dtype, bits, group_size):
    """One shared ``BlockLayout`` object per distinct page format (identity compares)."""
    return BlockLayout(version=3, layer_id=layer_id, page_tokens=page_tokens,
                       num_kv_heads=heads, head_dim=dim, key_dtype=dtype, value_dtype=dtype,
                       quantization_bits=bits, quantization_group_size=group_size,
                       kernel_version=KERNEL_VERSION)


class PagedKVCache:
    """One layer of one sequence: page refs, offset and a persistent page table."""

    def __init__(self, pool, *, layer_id=0, dtype="float16", bits=None, group_size=32):
        if dtype not in _DTYPES or bits not in {None, 4, 8}:
            raise ModelCapabilityUnsupported("unsupported paged storage precision")
        if not isinstance(pool, SegmentedPageArena):
            raise ValueError("paged storage requires a segmented arena")
        self.pool, self.layer_id, self.dtype, self.bits = pool, layer_id, dtype, bits
        self.group_size = group_size
        self.block_tokens = pool.block_tokens
        self._blocks = []
        self._offset = 0
        self.page_table = PersistentPageTable(pool)

    # -- properties ------------------------------------------------------------
    @property
    def offset(self):
        return self._offset

    @property
    def nbytes(self):
        return sum(ref.block.nbytes * ref.block.token_count // self.block_tokens
                   for ref in self._blocks)

    @property
    def full_block_refs(self):
        return tuple(r for r in self._blocks if r.block.token_count == self.block_tokens)

    def layout_for(self, heads, dim):
        return _layout(self.layer_id, self.block_tokens, int(heads), int(dim), self.dtype,
                       self.bits, self.group_size)

    @property
    def layout(self):
        return self._blocks[0].block.layout if self._blocks else None

    def empty(self):
        return PagedKVCache(self.pool, layer_id=self.layer_id, dtype=self.dtype, bits=self.bits,
                            group_size=self.group_size)

    # -- host page bookkeeping ------------------------------------------------------
    def _plan_append(self, width, layout):
        """Reserve pages and advance counts for ``width`` new tokens; returns start offset."""
        if self._blocks:
            stored = self._blocks[0].block.layout
            if stored is not layout and stored != layout:
                raise ValueError("paged append layout mismatch")
        start = self._offset
        cursor = 0
        while cursor < width:
            tail = self._blocks[-1].block if self._blocks else None
            if tail is None or tail.immutable:
                take = min(self.block_tokens, width - cursor)
                self._blocks.append(self.pool.allocate_ref(None, take, layout=layout))
                tail, fill = self._blocks[-1].block, take
            else:
                if tail.references != 1 or tail.pins:
                    raise ValueError("mutable paged tail is shared")
                fill = min(self.block_tokens - tail.token_count, width - cursor)
                self.pool.set_token_count(tail, tail.token_count + fill)
            cursor += fill
            self._offset += fill
            if tail.token_count == self.block_tokens:
                self.pool.seal(tail.block_id)
            self.page_table.update(len(self._blocks) - 1, self._blocks[-1])
        return start

    def page_row(self, width):
        """Page ids of this sequence, padded with -1 to ``width`` entries."""
        row = np.full(width, -1, np.int32)
        pages = self.page_table.row()
        row[:len(pages)] = pages
        return row

    def append(self, keys, values):
        """Append ``keys/values [1, HK, T, D]`` (device tensors) to this sequence."""
        import torch

        from pkv import ops

        if keys.shape != values.shape or keys.dim() != 4 or keys.shape[0] != 1:
            raise ValueError("paged append requires matching B=1 K/V tensors")
        dtype = _torch_dtype(self.dtype)
        keys, values = keys.to(dtype), values.to(dtype)
        layout = self.layout_for(keys.shape[1], keys.shape[3])
        width = int(keys.shape[2])
        # planning takes pages one by one: a failure part way (or before the
        # launch) must not leave the cache claiming tokens that were never written
        mark = self.checkpoint()
        try:
            start = self._plan_append(width, layout)
            pool = self.pool.pool_for(layout)
            device = pool.buffer.device
            table = torch.from_numpy(self.page_row(len(self.page_table.pages))[None]).to(device)
            ops.append_quantize(pool.fmt, pool.buffer, keys.to(device), values.to(device), table,
                                torch.tensor([start], dtype=torch.int32, device=device))
        except BaseException:
            self.rollback(mark)
            raise

    def clone(self):
        """Branch: sealed pages are shared (refcount), the mutable tail is copied."""
        from pkv import ops

        result = self.empty()
        result.page_table = self.page_table.fork()
        try:
            for ref in self._blocks:
                block = ref.block
                if block.immutable:
                    copied = ref.fork()
                else:
                    copied = self.pool.allocate_ref(None, block.token_count, layout=block.layout)
                    pool = self.pool.pool_for(block.layout)
                    ops.copy_pages(pool.fmt, pool.buffer, [block.page], [copied.block.page])
                result._blocks.append(copied)
                result.page_table.update(len(result._blocks) - 1, copied)
                result._offset += block.token_count
            return result
        except BaseException:
            result.reset()
            raise

    snapshot = clone

    def adopt(self, references):
        """Take sealed prefix pages (``paged.py:174-183``)."""
        if self._blocks or self._offset:
            raise ValueError("prefix adoption requires an empty cache")
        for reference in references:
            layout = reference.block.layout
            if (layout.version != 3 or layout.kernel_version != KERNEL_VERSION
                    or layout.key_dtype != self.dtype or layout.value_dtype != self.dtype
                    or layout.quantization_bits != self.bits
                    or layout.quantization_group_size != self.group_size):
                raise ModelCapabilityUnsupported("prefix page precision or layout mismatch")
            if reference.pool is not self.pool:
                raise ValueError("prefix belongs to another pool")
            if not reference.block.immutable or reference.block.token_count != self.block_tokens:
                raise ValueError("only sealed complete blocks may be adopted")
        self._blocks.extend(references)
        self._offset = len(references) * self.block_tokens
        for index, reference in enumerate(references):
            self.page_table.update(index, reference)

    def replace_from(self, draft):
        old = self._blocks
        self._blocks, self._offset = draft._blocks, draft._offset
        self.page_table = draft.page_table
        draft._blocks, draft._offset = [], 0
        draft.page_table = PersistentPageTable(self.pool)
        for ref in old:
            ref.close()

    def checkpoint(self):
        """State an in-place append can be rolled back to (see ``rollback``)."""
        tail = self._blocks[-1].block if self._blocks else None
        return (len(self._blocks), self._offset, tail,
                tail.token_count if tail is not None else 0,
                tail.immutable if tail is not None else False)

    def rollback(self, mark):
        """Undo appends made since ``checkpoint()``: pages taken since are
        released, the tail page gets back its token count (and its mutability,
        if the undone append filled and sealed it), the page table its length.
        Bytes written past the restored count are never read."""
        count, offset, tail, tail_tokens, sealed = mark
        while len(self._blocks) > count:
            self._blocks.pop().close()
        if tail is not None:
            self.pool.set_token_count(tail, tail_tokens)
            tail.immutable = sealed
        self._offset = offset
        self.page_table.truncate(count)
        if count:
            self.page_table.update(count - 1, self._blocks[-1])

    def reset(self):
        for ref in self._blocks:
            ref.close()
        self._blocks = []
        self._offset = 0
        self.page_table = PersistentPageTable(self.pool)

    release = reset

    def trim(self, count):
        if count < 0:
            raise ValueError("negative trim")
        target = max(self._offset - count, 0)
        if target % self.block_tokens:
            raise ModelCapabilityUnsupported("paged restoration requires complete pages")
        while self._offset > target:
            ref = self._blocks.pop()
            self._offset -= ref.block.token_count
            ref.close()
        self.page_table.truncate(len(self._blocks))
        return True

    def validate(self, spec):
        if (spec.kind != "full_kv" or spec.layer_id != self.layer_id or self.offset < 0
                or spec.key_head_dim != spec.value_head_dim):
            raise ValueError("paged component topology mismatch")
        self.page_table.validate(self._blocks)
        for ref in self._blocks:
            layout = ref.block.layout
            if (layout.num_kv_heads != spec.num_kv_heads or layout.head_dim != spec.key_head_dim
                    or layout.key_dtype != self.dtype or layout.layer_id != self.layer_id
                    or layout.kernel_version != KERNEL_VERSION):
                raise ValueError("paged component layout mismatch")

    def update(self, *_):
        raise ModelCapabilityUnsupported("paged cache requires direct attention dispatch")

    def state(self):
        raise ModelCapabilityUnsupported("paged histories cannot be materialized")


class PagedBatchCache:
    """One layer of a batch of sequences: batched append + attention (``paged.py:240-267``)."""

    def __init__(self, rows, widths, metrics):
        self.rows, self.widths, self.metrics = rows, widths, metrics
        self.offset = max(row.offset for row in rows)

    def attend(self, queries, keys, values, *, scale, position_ids):
        import torch

        batch, _, width, _ = queries.shape
        offsets = np.array([cache.offset for cache in self.rows], np.int64)
        widths = np.array(self.widths, np.int64)
        # logical positions of every query column (padding columns continue the row)
        positions = offsets[:, None] + np.arange(width)[None, :]
        if position_ids is not None:
            if tuple(position_ids.shape) != (len(self.rows), width):
                raise ValueError("paged query position shape mismatch")
            mask = np.arange(width)[None, :] < widths[:, None]
            given = position_ids.to("cpu", torch.int64).numpy()  # free for host tensors
            if not bool((given[mask] == positions[mask]).all()):
                raise ValueError("paged query logical positions mismatch")
        # host: pages for every row, then one append launch for the whole batch.
        # A failure before the launch (no free page part way through a row)
        # rolls every row back: no row claims tokens that were never written.
        layout = self.rows[0].layout_for(keys.shape[1], keys.shape[3])
        marks = [cache.checkpoint() for cache in self.rows]
        try:
            starts = [cache._plan_append(real, layout)
                      for cache, real in zip(self.rows, self.widths, strict=True)]
            return self._launch(queries, keys, values, layout, starts, widths, positions,
                                scale)
        except BaseException:
            for cache, mark in zip(self.rows, marks, strict=True):
                cache.rollback(mark)
            raise

    def _launch(self, queries, keys, values, layout, starts, widths, positions, scale):
        import torch

        from pkv import ops
        from pkv.paged_attention import paged_attention

        batch, _, width, _ = queries.shape
        pool = self.rows[0].pool.pool_for(layout)
        device = pool.buffer.device
        # the step's int32 metadata in one pinned buffer and one host->device copy:
        # block table [B, pages] | start [B] | width [B] | length [B] | q_pos [B, width]
        max_pages = max(len(c.page_table.pages) for c in self.rows)
        sizes = (batch * max_pages, batch, batch, batch, batch * width)
        host = torch.empty(sum(sizes), dtype=torch.int32, pin_memory=device.type == "cuda")
        parts = np.split(host.numpy(), np.cumsum(sizes)[:-1])
        table_h = parts[0].reshape(batch, max_pages)
        table_h.fill(-1)
        for row, cache in enumerate(self.rows):
            ids = cache.page_table.row()
            table_h[row, :len(ids)] = ids
        parts[1][:] = starts
        parts[2][:] = widths
        parts[3][:] = [cache.offset for cache in self.rows]
        parts[4][:] = positions.reshape(-1)
        meta = host.to(device, non_blocking=True)
        table, start_d, width_d, length_d, qpos_d = torch.split(meta, sizes)
        table = table.view(batch, max_pages)
        dtype = _torch_dtype(self.rows[0].dtype)
        ops.append_quantize(pool.fmt, pool.buffer, keys.to(device, dtype).contiguous(),
                            values.to(device, dtype).contiguous(), table, start_d, width_d)
        started = time.perf_counter()
        result = paged_attention(queries, self.rows, positions.tolist(), self.widths,
                                 scale=scale,
                                 _device_meta=(table, length_d, qpos_d.view(batch, width), width_d))
        self.metrics["synchronized_kernel_dispatch_ms"] = self.metrics.get(
            "synchronized_kernel_dispatch_ms", 0.0) + (time.perf_counter() - started) * 1000
        self.metrics["direct_attention_calls"] = self.metrics.get("direct_attention_calls", 0) + 1
        return result
