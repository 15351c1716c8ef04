"""numpy restatement of mlx-one's paged KV algorithm -- TEST INFRASTRUCTURE ONLY.

Imported only by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg; the product path never calls into this module.

Every function cites the reference lines it restates and says what pins it.
Float formats: float16 values are numpy ``float16``; bfloat16 values are held
as float32 arrays whose low 16 bits are zero (``bf16_round`` produces them).
"""

from __future__ import annotations

import numpy as np

# ---------------------------------------------------------------------------
# scalar formats
# ---------------------------------------------------------------------------


def bf16_round(x):
    """float32 -> bfloat16 (round to nearest even), returned as float32 values.

    Pinned by tests against ``torch.Tensor.to(torch.bfloat16)`` on random and
    tie-case bit patterns.  NaN inputs stay NaN.
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    bits = x.view(np.uint32)
    # 32-bit arithmetic: the largest finite pattern plus the increment fits
    rounded = bits + np.uint32(0x7FFF)
    rounded += (bits >> np.uint32(16)) & np.uint32(1)
    rounded &= np.uint32(0xFFFF0000)
    out = rounded.view(np.float32)
    nan = np.isnan(x)
    if nan.any():
        out[nan] = np.float32("nan")
    return out


def padded_dim(dim, group_size):
    """Head dimension padded to whole groups (``paged.py:31`` with 32 -> G)."""
    return (dim + group_size - 1) // group_size * group_size


# ---------------------------------------------------------------------------
# quantizer -- src/mlx_one/engine/paged.py:24-54
# ---------------------------------------------------------------------------


def quantize_page(value, bits, group_size=32):
    """Affine unsigned group quantization, restating ``paged.py:24-41``.

    ``value`` is float16 or bfloat16-as-float32 with the head dim last.  Steps,
    in the reference's order and types:

    1. cast to float32 and zero-pad the last axis to whole groups (:31-32);
    2. ``bias = f16(min(group))`` (:34);
    3. ``scale = f16(max(f32(max(group) - f32(bias)) / (2**bits - 1), 1e-6))``
       -- bias is rounded to f16 *before* it enters the scale (:35-36);
    4. ``code = clip(rint((x - f32(bias)) / f32(scale)), 0, 2**bits - 1)``,
       rint = round half to even (:37-38);
    5. 4-bit packs ``code[2i] | code[2i+1] << 4`` (:39-40).

    ``group_size`` generalises the reference's hard-coded 32 (:25, :31-33).
    Pinned: G=32 bit-exact against golden vectors written by the reference's
    own ``quantize_page`` (``tests/golden``); G=64/128 by the half-copy
    reduction to G=32 and by closed-form invariants (tests/test_oracle.py).
    """
    if bits not in (4, 8):
        raise ValueError("paged quantization supports 4 or 8 bits")
    data = np.asarray(value).astype(np.float32)
    dim = data.shape[-1]
    padded = padded_dim(dim, group_size)
    pad = [(0, 0)] * (data.ndim - 1) + [(0, padded - dim)]
    data = np.pad(data, pad)
    grouped = data.reshape(*data.shape[:-1], padded // group_size, group_size)
    levels = np.float32((1 << bits) - 1)
    bias = grouped.min(axis=-1, keepdims=True).astype(np.float16)
    spread = grouped.max(axis=-1, keepdims=True) - bias.astype(np.float32)
    scale = np.maximum(spread / levels, np.float32(1e-6)).astype(np.float16)
    with np.errstate(invalid="ignore", divide="ignore"):
        ratio = (grouped - bias.astype(np.float32)) / scale.astype(np.float32)
    encoded = np.clip(np.rint(ratio), 0, (1 << bits) - 1)
    encoded = encoded.reshape(data.shape).astype(np.uint8)
    if bits == 4:
        encoded = encoded[..., ::2] | (encoded[..., 1::2] << 4)
    return encoded, scale[..., 0], bias[..., 0]


def dequantize_page(state, bits, dim, group_size=32):
    """``x = f32(code) * f32(scale) + f32(bias)``, restating ``paged.py:44-54``.

    Pinned by golden vectors (G=32) and by the dequantization error bound
    ``|x - dq(q(x))| <= scale/2 + f16 rounding`` (tests/test_oracle.py).
    """
    data, scale, bias = state
    data = np.asarray(data)
    if bits == 4:
        data = np.stack((data & 15, data >> 4), axis=-1).reshape(
            *data.shape[:-1], data.shape[-1] * 2)
    grouped = data.astype(np.float32).reshape(*data.shape[:-1], -1, group_size)
    out = (grouped * np.asarray(scale, np.float32)[..., None]
           + np.asarray(bias, np.float32)[..., None])
    return out.reshape(data.shape)[..., :dim]


# ---------------------------------------------------------------------------
# page store in the reference's format -- arena.py:58-106, paged.py:103-154
# ---------------------------------------------------------------------------


class RefPages:
    """Pages in the reference's per-page tensor format.

    A quantized page holds ``(K codes [HK,P,Dp'], K scale [HK,P,Dp/G], K bias,
    V codes, V scale, V bias)`` (``paged_attention.py:31-35``); a float page
    holds ``(K [HK,P,D], V [HK,P,D])``.  ``Dp' = Dp`` for 8-bit and ``Dp/2`` for
    4-bit.  Pages are addressed by an integer page id and listed per sequence
    in a block table, the role ``PersistentPageTable`` entries play in the
    reference (``arena.py:185-200``).

    ``tail`` selects what the attention reads for the last, partly filled
    page: ``"float"`` keeps the reference's float tail page (``paged.py:113-141``,
    pages quantize when they fill, :142-153); ``"quantized"`` quantizes every
    token as it is appended.  Both give the same codes for every full page,
    because groups run along the head dimension of one (head, token).
    """

    def __init__(self, num_kv_heads, head_dim, page_tokens, *, bits=None,
                 group_size=32, dtype="bfloat16", tail="quantized"):
        self.hk, self.dim, self.page = num_kv_heads, head_dim, page_tokens
        self.bits, self.group, self.dtype, self.tail = bits, group_size, dtype, tail
        self.pages = {}

    def _cast(self, x):
        x = np.asarray(x, np.float32)
        return x.astype(np.float16).astype(np.float32) if self.dtype == "float16" \
            else bf16_round(x)

    def write_sequence(self, table, keys, values):
        """Store ``keys/values [HK, L, D]`` into pages ``table[0..ceil(L/P))``."""
        length = keys.shape[1]
        keys, values = self._cast(keys), self._cast(values)
        for index in range((length + self.page - 1) // self.page):
            lo, hi = index * self.page, min(length, (index + 1) * self.page)
            k = np.zeros((self.hk, self.page, self.dim), np.float32)
            v = np.zeros_like(k)
            k[:, :hi - lo], v[:, :hi - lo] = keys[:, lo:hi], values[:, lo:hi]
            self.pages[int(table[index])] = (k, v, hi - lo)

    def state(self, page_id):
        """Reference-format tensors of one page (quantized pages: 6 tensors)."""
        k, v, count = self.pages[int(page_id)]
        if self.bits is None:
            return k, v
        kq = quantize_page(k, self.bits, self.group)
        vq = quantize_page(v, self.bits, self.group)
        return (*kq, *vq)

    def token_values(self, page_id):
        """Dequantized K, V ``[HK, count, D]`` as the attention reads them."""
        k, v, count = self.pages[int(page_id)]
        if self.bits is None or (self.tail == "float" and count < self.page):
            return k[:, :count], v[:, :count]
        kq = quantize_page(k, self.bits, self.group)
        vq = quantize_page(v, self.bits, self.group)
        kd = dequantize_page(kq, self.bits, self.dim, self.group)
        vd = dequantize_page(vq, self.bits, self.dim, self.group)
        return kd[:, :count], vd[:, :count]

    def gather(self, table, length):
        """Dense ``[HK, length, D]`` K and V for one sequence (block-table gather)."""
        ks, vs = [], []
        for index in range((length + self.page - 1) // self.page):
            k, v = self.token_values(table[index])
            ks.append(k)
            vs.append(v)
        if not ks:
            empty = np.zeros((self.hk, 0, self.dim), np.float32)
            return empty, empty.copy()
        return np.concatenate(ks, 1)[:, :length], np.concatenate(vs, 1)[:, :length]


# ---------------------------------------------------------------------------
# attention -- paged_attention.py:62-113 (kernel), :127-206 (merge), :209-246
# ---------------------------------------------------------------------------


def paged_attention(queries, keys, values, positions, widths, *, scale):
    """Causal GQA attention over gathered K/V, restating ``paged_attention.py:209-246``.

    ``queries [B,H,Q,D]``; ``keys[b], values[b]`` are ``[HK, L_b, D]`` float32
    (already dequantized); ``positions[b][q]`` is the logical position of query
    ``q``; token ``t`` is visible to it when ``t <= positions[b][q]`` (:225).
    Head ``h`` reads KV head ``h // (H // HK)`` (:223).  Query rows ``q >=
    widths[b]`` stay zero (:217, ``test_paged_hybrid.py:630``).  The normalizer
    is floored at 1e-20 (:245).  Computed in float64; returns float64.

    Pinned by brute force against an independent per-token online-softmax loop
    (the reference's own formulation) on tiny shapes, and by closed forms:
    one visible token returns V, identical keys return mean(V).
    """
    q = np.asarray(queries, np.float64)
    batch, heads, width, dim = q.shape
    out = np.zeros((batch, heads, width, dim), np.float64)
    for b in range(batch):
        k = np.asarray(keys[b], np.float64)
        v = np.asarray(values[b], np.float64)
        hk = k.shape[0]
        group = heads // hk
        length = k.shape[1]
        pos = np.asarray(positions[b])
        for h in range(heads):
            kh = h // group
            for qi in range(int(widths[b])):
                visible = np.arange(length) <= pos[qi]
                if not visible.any():
                    continue
                scores = (k[kh, visible] @ q[b, h, qi]) * scale
                top = scores.max()
                weights = np.exp(scores - top)
                out[b, h, qi] = (weights @ v[kh, visible]) / max(weights.sum(), 1e-20)
    return out


def online_softmax_attention(queries, keys, values, positions, widths, *, scale):
    """Per-token online softmax, the reference kernel's own loop (``paged_attention.py:80-97``).

    Used only to cross-check ``paged_attention`` on tiny shapes.
    """
    q = np.asarray(queries, np.float64)
    batch, heads, width, dim = q.shape
    out = np.zeros_like(q)
    for b in range(batch):
        k = np.asarray(keys[b], np.float64)
        v = np.asarray(values[b], np.float64)
        group = heads // k.shape[0]
        for h in range(heads):
            for qi in range(int(widths[b])):
                m, l, acc = -np.inf, 0.0, np.zeros(dim)
                for t in range(k.shape[1]):
                    if t > positions[b][qi]:
                        break
                    s = float(k[h // group, t] @ q[b, h, qi]) * scale
                    nm = max(m, s)
                    a, e = np.exp(m - nm), np.exp(s - nm)
                    acc, l, m = acc * a + v[h // group, t] * e, l * a + e, nm
                out[b, h, qi] = acc / max(l, 1e-20)
    return out


def partition_partials(queries, keys, values, positions, widths, *, scale, split):
    """Per-partition ``(acc, m, l)`` over token ranges of ``split`` tokens.

    The same quantities each reference launch returns for its chunk
    (``paged_attention.py:107-112``): unnormalised accumulator, running max,
    normalizer; ``m = -inf, l = 0`` where a partition has no visible token.
    Returns a list (one per partition index) of ``(acc [B,H,Q,D], m [B,H,Q,1],
    l [B,H,Q,1])`` in float64.
    """
    q = np.asarray(queries, np.float64)
    batch, heads, width, dim = q.shape
    longest = max(np.asarray(k).shape[1] for k in keys)
    parts = []
    for start in range(0, max(longest, 1), split):
        acc = np.zeros((batch, heads, width, dim))
        m = np.full((batch, heads, width, 1), -np.inf)
        l = np.zeros((batch, heads, width, 1))
        for b in range(batch):
            k = np.asarray(keys[b], np.float64)
            v = np.asarray(values[b], np.float64)
            group = heads // k.shape[0]
            stop = min(start + split, k.shape[1])
            for h in range(heads):
                for qi in range(int(widths[b])):
                    tokens = np.arange(start, stop)
                    tokens = tokens[tokens <= positions[b][qi]]
                    if not len(tokens):
                        continue
                    s = (k[h // group, tokens] @ q[b, h, qi]) * scale
                    m[b, h, qi, 0] = s.max()
                    w = np.exp(s - s.max())
                    l[b, h, qi, 0] = w.sum()
                    acc[b, h, qi] = w @ v[h // group, tokens]
        parts.append((acc, m, l))
    return parts


def lse_merge(parts):
    """Log-sum-exp merge of partition partials, restating ``paged_attention.py:191-204``.

    ``M' = max(M, m)``; ``c = M'`` where ``L + l > 0`` else 0;
    ``a = exp((M if L > 0 else -inf) - c)``; ``b = exp((m if l > 0 else -inf) - c)``;
    ``acc = acc*a + pacc*b``; ``L = L*a + l*b``; result ``acc / max(L, 1e-20)``.
    Pinned at atol/rtol .002 against the dense oracle, the bar the reference
    sets for its merger (``test_paged_hybrid.py:574-634``).
    """
    acc, maximum, normalizer = (np.array(x, np.float64) for x in parts[0])
    for pacc, pm, pl in parts[1:]:
        new_max = np.maximum(maximum, pm)
        with np.errstate(invalid="ignore"):
            center = np.where(normalizer + pl > 0, new_max, 0)
            a = np.exp(np.where(normalizer > 0, maximum, -np.inf) - center)
            b = np.exp(np.where(pl > 0, pm, -np.inf) - center)
        acc, normalizer = acc * a + pacc * b, normalizer * a + pl * b
        maximum = new_max
    return acc / np.maximum(normalizer, 1e-20)
