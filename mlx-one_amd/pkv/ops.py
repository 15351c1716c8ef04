"""Functional layer over libpkv: torch device tensors in and out.

These are the primitives the reference-named classes (``pkv.arena``,
``pkv.paged``, ``pkv.paged_attention``) are built on.  Every function enqueues
HIP work on the current torch stream through the C ABI and never falls back to
a CPU implementation.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from pkv import _native as nat

FLOAT_KINDS = {torch.bfloat16: 0, torch.float16: 1}
DTYPES = {0: torch.bfloat16, 1: torch.float16}


@dataclass(frozen=True)
class PageFormat:
    """One layer's page layout; the C ``pkv_layout`` plus derived sizes.

    ``bits`` is 4 or 8 for affine-quantized pages and 16 for float pages
    (the reference's ``BlockLayout.quantization_bits`` None).
    """

    num_kv_heads: int
    head_dim: int
    page_tokens: int
    bits: int = 16
    group_size: int = 32
    dtype: torch.dtype = torch.bfloat16

    def __post_init__(self):
        if self.dtype not in FLOAT_KINDS:
            from pkv.modes import ModelCapabilityUnsupported

            raise ModelCapabilityUnsupported("unsupported paged storage precision")
        if self.page_bytes < 0:
            nat.check(nat.PKV_UNSUPPORTED, "page layout")

    @property
    def c_layout(self):
        return nat.Layout(self.num_kv_heads, self.head_dim, self.page_tokens, self.bits,
                          self.group_size if self.bits != 16 else 32, FLOAT_KINDS[self.dtype])

    @property
    def page_bytes(self):
        return int(nat.load().pkv_page_bytes(self.c_layout))

    @property
    def stored_dim(self):
        return int(nat.load().pkv_stored_dim(self.c_layout))

    @property
    def quantized(self):
        return self.bits != 16

    @property
    def reference_dim(self):
        """Padded head dim of the reference format (``paged.py:31``)."""
        if not self.quantized:
            return self.head_dim
        return (self.head_dim + self.group_size - 1) // self.group_size * self.group_size


def allocate_pool(fmt: PageFormat, num_pages: int, device="cuda"):
    """Device page pool ``[num_pages, page_bytes]`` uint8 (zeroed)."""
    return torch.zeros((num_pages, fmt.page_bytes), dtype=torch.uint8, device=device)


def _i32(x, device):
    if x is None:
        return None
    if isinstance(x, torch.Tensor):
        t = x.to(device=device, dtype=torch.int32)
    else:
        t = torch.as_tensor(x, dtype=torch.int32).to(device)
    return t.contiguous()


def _check_float(t, fmt, name):
    if t.dtype != fmt.dtype:
        raise ValueError(f"{name} dtype {t.dtype} differs from the page dtype {fmt.dtype}")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")


def append_quantize(fmt: PageFormat, pool, keys, values, block_table, start_pos, widths=None,
                    new_lens=None):
    """Write ``keys/values [B, HK, T, D]`` at positions ``start_pos[b] + t``."""
    if keys.shape != values.shape or keys.dim() != 4:
        raise ValueError("paged append requires matching [B, HK, T, D] K/V tensors")
    batch, heads, tokens, dim = keys.shape
    if heads != fmt.num_kv_heads or dim != fmt.head_dim:
        raise ValueError("paged append layout mismatch")
    _check_float(keys, fmt, "keys")
    _check_float(values, fmt, "values")
    device = keys.device
    table = _i32(block_table, device)
    if table.dim() != 2 or table.shape[0] != batch:
        raise ValueError("block table must be [batch, max_pages]")
    start = _i32(start_pos, device)
    width = _i32(widths, device)
    keys, values = keys.contiguous(), values.contiguous()
    code = nat.load().pkv_append_quantize(
        nat.stream_handle(device), fmt.c_layout, nat.ptr(pool), pool.shape[0], nat.ptr(keys),
        nat.ptr(values), batch, tokens, nat.ptr(table), table.shape[1], nat.ptr(start),
        nat.ptr(width), nat.ptr(new_lens))
    nat.check(code, "paged append")


def attention_waves(fmt: PageFormat, num_heads, num_queries):
    """Waves the attention kernel keeps resident for this shape (the default grid)."""
    waves = int(nat.load().pkv_attention_waves(fmt.c_layout, num_heads, num_queries))
    if waves <= 0:
        nat.check(nat.PKV_LAUNCH_FAILED, "attention waves")
    return waves


DECODE_KERNELS = {"mfma": 0, "valu": 1}


def select_decode_kernel(kind):
    """Choose the kernel for decode rows (at most 4 query rows per KV head over
    quantized pages, head_dim <= 128): ``"mfma"`` (the default) or ``"valu"``
    (the same split and merge with vector-ALU dot products).  Process-wide;
    returns the previous choice."""
    if kind not in DECODE_KERNELS:
        raise ValueError(f"decode kernel must be one of {sorted(DECODE_KERNELS)}")
    previous = int(nat.load().pkv_select_decode_kernel(DECODE_KERNELS[kind]))
    if previous < 0:
        nat.check(previous, "select decode kernel")
    return {v: k for k, v in DECODE_KERNELS.items()}[previous]


def default_waves(fmt: PageFormat, num_heads, num_queries, batch):
    """The waves ``paged_attention`` uses by default for this shape and batch."""
    waves = int(nat.load().pkv_attention_default_waves(fmt.c_layout, num_heads, num_queries,
                                                         batch))
    if waves <= 0:
        nat.check(nat.PKV_LAUNCH_FAILED, "attention waves")
    return waves


def decode_queries(fmt: PageFormat, num_heads, num_queries):
    """Queries per sequence of the split-K decode part of a call: all of them
    when the decode kernel serves the call (at most 32 query rows per KV head,
    16 at head_dim > 128), else the most a mixed batch's narrow sequences may
    have there (0 when the GQA ratio leaves none)."""
    gqa = num_heads // fmt.num_kv_heads
    limit = 16 if fmt.stored_dim > 128 else 32
    return num_queries if num_queries * gqa <= limit else limit // max(gqa, 1)


def workspace_bytes(fmt: PageFormat, num_heads, num_queries, waves):
    return int(nat.load().pkv_attention_workspace_bytes(fmt.c_layout, num_heads, num_queries,
                                                          waves))


# One attention workspace per device, grown on demand; calls on one stream
# share it (each call's partials are merged before the next call starts).
_WORKSPACES = {}


def attention_workspace(device, nbytes):
    """A workspace of at least ``nbytes`` on ``device`` (cached, grown on demand)."""
    key = torch.device(device)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=key)
        _WORKSPACES[key] = ws
    return ws


def paged_attention(fmt: PageFormat, pool, queries, block_table, seq_lens, *, scale, q_pos=None,
                    widths=None, waves=0, workspace=None, out=None):
    """Attention of ``queries [B, H, Q, D]`` over the paged cache.

    ``seq_lens`` counts the tokens in each sequence's cache (after the
    append) and stays on the device: the decode kernel shares the tiles of
    all sequences out over ``waves`` waves (default: ``default_waves``);
    query blocks past 32 rows per KV head run on the prefill kernel -- and
    in a mixed batch (``widths`` given), the sequences narrow enough for the
    decode kernel still go to it, in the same call (``waves`` then sizes that
    part).  ``workspace`` (bytes from ``workspace_bytes``) may be given by the
    caller.
    """
    if queries.dim() != 4:
        raise ValueError("queries must be [B, H, Q, D]")
    batch, heads, nq, dim = queries.shape
    if dim != fmt.head_dim:
        raise ValueError("query head dimension differs from the page layout")
    _check_float(queries, fmt, "queries")
    device = queries.device
    table = _i32(block_table, device)
    lens = _i32(seq_lens, device)
    if waves <= 0:
        waves = default_waves(fmt, heads, decode_queries(fmt, heads, nq) or nq, batch)
    need = workspace_bytes(fmt, heads, nq, waves)
    if need < 0:
        nat.check(nat.PKV_INVALID_ARGUMENT, "paged attention workspace")
    if workspace is None:
        workspace = attention_workspace(device, need)
    elif workspace.device != device or workspace.dtype != torch.uint8 or \
            not workspace.is_contiguous():
        raise ValueError("attention workspace must be a contiguous uint8 tensor on the "
                         "queries' device")
    # the kernels read queries and write out as dense [B, H, Q, D]
    queries = queries.contiguous()
    if out is None:
        out = torch.empty(queries.shape, dtype=queries.dtype, device=device)
    elif (tuple(out.shape) != tuple(queries.shape) or out.dtype != queries.dtype
          or out.device != device or not out.is_contiguous()):
        raise ValueError("out must be a contiguous tensor of the queries' shape, dtype and "
                         "device")
    code = nat.load().pkv_paged_attention(
        nat.stream_handle(device), fmt.c_layout, nat.ptr(pool), pool.shape[0], nat.ptr(queries),
        batch, heads, nq, nat.ptr(table), table.shape[1], nat.ptr(lens),
        nat.ptr(_i32(q_pos, device)), nat.ptr(_i32(widths, device)), float(scale),
        int(waves), nat.ptr(workspace), workspace.numel(), nat.ptr(out))
    nat.check(code, "paged attention")
    return out


def append_paged_attention(fmt: PageFormat, pool, keys, values, queries, block_table, seq_lens, *,
                           scale, waves=0, workspace=None, out=None):
    """One single-token step: append ``keys``/``values [B, HK, 1, D]`` at
    position ``seq_lens - 1`` (``seq_lens`` counts the tokens after the
    append) and attend ``queries [B, H, 1, D]`` -- one launch where the decode
    kernel serves the shape (quantized pages, at most 8 query rows per KV
    head), else an append launch and the attention.  Pages and output equal
    ``append_quantize`` followed by ``paged_attention`` bit for bit."""
    if queries.dim() != 4 or queries.shape[2] != 1:
        raise ValueError("queries must be [B, H, 1, D]")
    batch, heads, _, dim = queries.shape
    shape = (batch, fmt.num_kv_heads, 1, dim)
    if dim != fmt.head_dim or tuple(keys.shape) != shape or tuple(values.shape) != shape:
        raise ValueError(f"keys and values must be {shape} and the queries' head dimension "
                         "the page layout's")
    for name, t in (("queries", queries), ("keys", keys), ("values", values)):
        _check_float(t, fmt, name)
    device = queries.device
    table = _i32(block_table, device)
    lens = _i32(seq_lens, device)
    if waves <= 0:
        waves = default_waves(fmt, heads, 1, batch)
    need = workspace_bytes(fmt, heads, 1, waves)
    if need < 0:
        nat.check(nat.PKV_INVALID_ARGUMENT, "paged attention workspace")
    if workspace is None:
        workspace = attention_workspace(device, need)
    elif workspace.device != device or workspace.dtype != torch.uint8 or \
            not workspace.is_contiguous():
        raise ValueError("attention workspace must be a contiguous uint8 tensor on the "
                         "queries' device")
    queries, keys, values = queries.contiguous(), keys.contiguous(), values.contiguous()
    if out is None:
        out = torch.empty(queries.shape, dtype=queries.dtype, device=device)
    elif (tuple(out.shape) != tuple(queries.shape) or out.dtype != queries.dtype
          or out.device != device or not out.is_contiguous()):
        raise ValueError("out must be a contiguous tensor of the queries' shape, dtype and "
                         "device")
    code = nat.load().pkv_append_paged_attention(
        nat.stream_handle(device), fmt.c_layout, nat.ptr(pool), pool.shape[0], nat.ptr(keys),
        nat.ptr(values), nat.ptr(queries), batch, heads, nat.ptr(table), table.shape[1],
        nat.ptr(lens), float(scale), int(waves), nat.ptr(workspace), workspace.numel(),
        nat.ptr(out))
    nat.check(code, "append + paged attention")
    return out


def gather_pages(fmt: PageFormat, pool, page_ids):
    """Pages in the reference's per-page tensor format (``paged_attention.py:31-35``).

    Quantized: ``(k_codes [N,HK,P,Dq] u8, k_scale [N,HK,P,Dp/G] f16, k_bias,
    v_codes, v_scale, v_bias)``; float: ``(k [N,HK,P,D], v)``.
    """
    ids = _i32(page_ids, pool.device)
    n = ids.numel()
    shape = (n, fmt.num_kv_heads, fmt.page_tokens)
    if fmt.quantized:
        dq = fmt.reference_dim * fmt.bits // 8
        ng = fmt.reference_dim // fmt.group_size
        kc = torch.empty(shape + (dq,), dtype=torch.uint8, device=pool.device)
        vc = torch.empty_like(kc)
        ks, kb, vs, vb = (torch.empty(shape + (ng,), dtype=torch.float16, device=pool.device)
                          for _ in range(4))
        outs = (kc, ks, kb, vc, vs, vb)
    else:
        k = torch.empty(shape + (fmt.head_dim,), dtype=fmt.dtype, device=pool.device)
        v = torch.empty_like(k)
        outs = (k, None, None, v, None, None)
    code = nat.load().pkv_gather_pages(nat.stream_handle(pool.device), fmt.c_layout,
                                       nat.ptr(pool), pool.shape[0], nat.ptr(ids), n,
                                       *[nat.ptr(t) for t in outs])
    nat.check(code, "page gather")
    return outs if fmt.quantized else (outs[0], outs[3])


def copy_pages(fmt: PageFormat, pool, src_ids, dst_ids):
    src = _i32(src_ids, pool.device)
    dst = _i32(dst_ids, pool.device)
    if src.numel() != dst.numel():
        raise ValueError("page copy requires matching id lists")
    code = nat.load().pkv_copy_pages(nat.stream_handle(pool.device), fmt.c_layout, nat.ptr(pool),
                                     pool.shape[0], nat.ptr(src), nat.ptr(dst), src.numel())
    nat.check(code, "page copy")


def quantize_rows(values, bits, group_size=32):
    """Reference ``quantize_page`` over the last axis: ``(codes, scale f16, bias f16)``."""
    if values.dtype not in FLOAT_KINDS:
        raise ValueError("quantize expects float16 or bfloat16 values")
    values = values.contiguous()
    dim = values.shape[-1]
    rows = values.numel() // dim if dim else 0
    padded = (dim + group_size - 1) // group_size * group_size
    lead = tuple(values.shape[:-1])
    codes = torch.empty(lead + (padded * bits // 8,), dtype=torch.uint8, device=values.device)
    scale = torch.empty(lead + (padded // group_size,), dtype=torch.float16, device=values.device)
    bias = torch.empty_like(scale)
    code = nat.load().pkv_quantize_rows(nat.stream_handle(values.device), nat.ptr(values), rows,
                                        dim, bits, group_size, FLOAT_KINDS[values.dtype],
                                        nat.ptr(codes), nat.ptr(scale), nat.ptr(bias))
    nat.check(code, "quantize")
    return codes, scale, bias


def dequantize_rows(state, bits, dim, group_size=32):
    """Reference ``dequantize_page``: float32 ``[..., dim]``."""
    codes, scale, bias = (t.contiguous() for t in state)
    rows = scale.numel() // scale.shape[-1] if scale.dim() else 0
    out = torch.empty(tuple(codes.shape[:-1]) + (dim,), dtype=torch.float32, device=codes.device)
    code = nat.load().pkv_dequantize_rows(nat.stream_handle(codes.device), nat.ptr(codes),
                                          nat.ptr(scale), nat.ptr(bias), rows, dim, bits,
                                          group_size, nat.ptr(out))
    nat.check(code, "dequantize")
    return out


_FLOAT_KIND = {torch.bfloat16: 0, torch.float16: 1}


def rope_qkv(qkv, positions, inv_freq, heads, kv_heads):
    """Rotate-half RoPE of a fused projection ``qkv [B, T, (heads + 2*kv_heads) * D]``
    at ``positions [B, T]``: returns ``q [B, heads, T, D]``, ``k, v [B, kv_heads, T, D]``
    (q and k rotated, v copied), contiguous, in ``qkv``'s dtype.  Float32 math as
    the reference's ``apply_rope`` (``models/shared/transformer.py:32-90``)."""
    if qkv.dim() != 3 or qkv.dtype not in _FLOAT_KIND or not qkv.is_cuda:
        raise ValueError("qkv must be a [B, T, width] f16/bf16 device tensor")
    batch, tokens, width = qkv.shape
    if width % (heads + 2 * kv_heads):
        raise ValueError("qkv width is not (heads + 2*kv_heads) * head_dim")
    dim = width // (heads + 2 * kv_heads)
    if dim % 2 or dim > 256 or inv_freq.numel() != dim // 2:
        raise ValueError("RoPE needs an even head dimension <= 256 and dim/2 frequencies")
    if tuple(positions.shape) != (batch, tokens):
        raise ValueError("positions must be [B, T]")
    device = qkv.device
    qkv = qkv.contiguous()
    pos = _i32(positions, device)
    inv = inv_freq.to(device=device, dtype=torch.float32).contiguous()
    q = torch.empty((batch, heads, tokens, dim), dtype=qkv.dtype, device=device)
    k = torch.empty((batch, kv_heads, tokens, dim), dtype=qkv.dtype, device=device)
    v = torch.empty_like(k)
    code = nat.load().pkv_rope_qkv(nat.stream_handle(device), nat.ptr(qkv), batch, tokens, heads,
                                   kv_heads, dim, _FLOAT_KIND[qkv.dtype], nat.ptr(pos),
                                   nat.ptr(inv), nat.ptr(q), nat.ptr(k), nat.ptr(v))
    nat.check(code, "rope")
    return q, k, v

