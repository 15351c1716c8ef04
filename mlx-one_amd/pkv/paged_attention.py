"""Direct paged attention dispatch (the reference's ``engine/paged_attention.py``).

``paged_attention(queries, rows, positions, widths, *, scale)`` keeps the
reference's signature and semantics (``src/mlx_one/engine/paged_attention.py:127-206``):
query ``q`` of row ``b`` at logical position ``positions[b][q]`` attends the
row's tokens ``t <= positions[b][q]``, KV head ``h // (H / HK)``, rows
``q >= widths[b]`` are zero, output in the query dtype.  One libpkv launch
covers the whole batch: no eight-row limit, no 31-binding limit and no host
synchronisation per partition (the reference launches per 16-page chunk and
segment group and evaluates after each merge, :165-203).
"""

from __future__ import annotations

import numpy as np

from pkv.modes import ModelCapabilityUnsupported


def page_bindings(rows):
    """Validate row ownership and layouts; returns the batch's page rows.

    Mirrors the checks of ``paged_attention.py:8-48`` that still apply: the
    committed length matches the page token counts, pages belong to the
    row's arena and layer, quantized pages of a row share one precision.
    """
    from pkv.paged import KERNEL_VERSION

    for cache in rows:
        if sum(r.block.token_count for r in cache._blocks) != cache.offset:
            raise ValueError("paged table committed length mismatch")
        for ref in cache._blocks:
            block = ref.block
            layout = block.layout
            if (ref.pool is not cache.pool or layout is None or layout.version != 3
                    or layout.layer_id != cache.layer_id
                    or layout.page_tokens != cache.block_tokens
                    or layout.key_dtype != cache.dtype or layout.value_dtype != cache.dtype
                    or layout.kernel_version != KERNEL_VERSION
                    or layout.quantization_bits != cache.bits
                    or not 0 < block.token_count <= layout.page_tokens):
                raise ValueError("invalid paged arena ownership or layout")
        cache.page_table.validate(cache._blocks)
    longest = max(len(c.page_table.pages) for c in rows)
    return np.stack([c.page_row(max(longest, 1)) for c in rows])


def paged_attention(queries, rows, positions, widths, *, scale, _device_meta=None):
    """``_device_meta``: ``(block_table, lengths, q_pos, widths)`` already on the
    device, from a caller that has just written them (``PagedBatchCache.attend``)."""
    import torch

    from pkv import ops

    batch, heads, length, dim = queries.shape
    if (len(rows) != batch or len(positions) != batch or len(widths) != batch
            or any(len(p) != length for p in positions)
            or any(w < 1 or w > length for w in widths)
            or any(not c._blocks or c.offset < w for c, w in zip(rows, widths, strict=True))):
        raise ValueError("invalid paged query row mapping")
    layout = rows[0]._blocks[0].block.layout
    if dim < 1 or dim > 256 or heads % layout.num_kv_heads:
        raise ModelCapabilityUnsupported("paged attention supports GQA head dimensions 1..256")
    arena = rows[0].pool
    if any(c.pool is not arena for c in rows):
        raise ValueError("batch spans page arenas")
    if any(c._blocks[0].block.layout != layout for c in rows):
        raise ModelCapabilityUnsupported("incompatible arena page layouts")
    pool = arena.pool_for(layout)
    with arena.lease():
        device = pool.buffer.device
        if _device_meta is None:
            table = torch.from_numpy(page_bindings(rows)).to(device)
            lengths = torch.tensor([c.offset for c in rows], dtype=torch.int32, device=device)
            q_pos = torch.tensor([list(p) for p in positions], dtype=torch.int32, device=device)
            width_d = torch.tensor(list(widths), dtype=torch.int32, device=device)
        else:
            table, lengths, q_pos, width_d = _device_meta
        dtype = queries.dtype
        q = queries.to(device, pool.fmt.dtype)
        out = ops.paged_attention(pool.fmt, pool.buffer, q, table, lengths, scale=scale,
                                  q_pos=q_pos, widths=width_d)
        return out.to(dtype)
