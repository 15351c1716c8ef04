"""Shared helpers of the parity tests: run a workload through libpkv and the oracle."""

from __future__ import annotations

import math

import numpy as np

from oracle import cport, numpy_ref


def to_torch(array, dtype, device="cuda"):
    import torch

    return torch.from_numpy(np.ascontiguousarray(array, np.float32)).to(device=device, dtype=dtype)


def fill_pages(fmt, inst, *, chunk=None, device="cuda"):
    """Append every token of ``inst`` into a fresh pool, ``chunk`` tokens per call.

    Sequences of different lengths use per-sequence widths (ragged appends).
    Returns ``(pool, table, lengths)`` as device tensors.
    """
    import torch

    from pkv import ops

    w = inst.workload
    lengths = np.array([k.shape[1] for k in inst.keys], np.int32)
    pool = ops.allocate_pool(fmt, inst.num_pages, device)
    table = torch.from_numpy(inst.table).to(device)
    longest = int(lengths.max())
    chunk = chunk or longest
    # Shared-prefix pages are written by every sequence that lists them; the
    # tokens there are identical, so the duplicate writes store the same bytes.
    for start in range(0, longest, chunk):
        width = np.clip(lengths - start, 0, chunk).astype(np.int32)
        k = np.zeros((w.batch, w.kv_heads, chunk, w.head_dim), np.float32)
        v = np.zeros_like(k)
        for b in range(w.batch):
            n = int(width[b])
            k[b, :, :n] = inst.keys[b][:, start:start + n]
            v[b, :, :n] = inst.values[b][:, start:start + n]
        starts = torch.full((w.batch,), start, dtype=torch.int32, device=device)
        ops.append_quantize(fmt, pool, to_torch(k, fmt.dtype, device), to_torch(v, fmt.dtype, device),
                            table, starts, torch.from_numpy(width).to(device))
    return pool, table, torch.from_numpy(lengths).to(device)


def oracle_pages(fmt, inst):
    """Reference-format pages of ``inst`` built by the CPU oracle (tail quantized)."""
    w = inst.workload
    ref = numpy_ref.RefPages(w.kv_heads, w.head_dim, w.page_tokens,
                             bits=None if w.bits == 16 else w.bits, group_size=w.group_size,
                             dtype="bfloat16", tail="quantized")
    for b in range(w.batch):
        ref.write_sequence(inst.table[b], inst.keys[b], inst.values[b])
    return ref


def reference_arrays(fmt, ref, num_pages):
    """Dense reference-format arrays indexed by page id (for the C oracle)."""
    w_hk, p = fmt.num_kv_heads, fmt.page_tokens
    if fmt.quantized:
        dq = fmt.reference_dim * fmt.bits // 8
        ng = fmt.reference_dim // fmt.group_size
        kc = np.zeros((num_pages, w_hk, p, dq), np.uint8)
        vc = np.zeros_like(kc)
        ks, kb, vs, vb = (np.zeros((num_pages, w_hk, p, ng), np.float16) for _ in range(4))
        for pid in ref.pages:
            state = ref.state(pid)
            kc[pid], ks[pid], kb[pid], vc[pid], vs[pid], vb[pid] = state
        return (kc, ks, kb, vc, vs, vb)
    k = np.zeros((num_pages, w_hk, p, fmt.head_dim), np.float32)
    v = np.zeros_like(k)
    for pid, (kp, vp, _) in ref.pages.items():
        k[pid], v[pid] = kp, vp
    to_bits = lambda a: (a.view(np.uint32) >> 16).astype(np.uint16)
    return (to_bits(k), to_bits(v))


def oracle_attention(fmt, inst, positions, widths, scale, *, ref=None, use_c=True):
    """Oracle output ``[B, H, Q, D]`` float32 for the instance after the append."""
    w = inst.workload
    ref = ref or oracle_pages(fmt, inst)
    lengths = np.array([k.shape[1] for k in inst.keys], np.int32)
    if use_c:
        arrays = reference_arrays(fmt, ref, inst.num_pages)
        if fmt.quantized:
            return cport.paged_attention(inst.queries, inst.table, lengths, positions, widths,
                                         heads_kv=w.kv_heads, page_tokens=w.page_tokens,
                                         bits=w.bits, group_size=w.group_size, pages=arrays,
                                         scale=scale)
        return cport.paged_attention(inst.queries, inst.table, lengths, positions, widths,
                                     heads_kv=w.kv_heads, page_tokens=w.page_tokens, bits=0,
                                     float_pages=arrays, scale=scale)
    keys, values = [], []
    for b in range(w.batch):
        k, v = ref.gather(inst.table[b], int(lengths[b]))
        keys.append(k)
        values.append(v)
    return numpy_ref.paged_attention(inst.queries, keys, values, positions, widths,
                                     scale=scale).astype(np.float32)


def assert_attention_close(got, want, *, max_abs=2e-2, mean_abs=1e-3):
    """``assert_attention_close_f32`` returning (max abs error, mean abs error);
    elements over ``max_abs`` (allowed only where half a bf16 step is larger)
    are printed."""
    worst, mean, over = assert_attention_close_f32(got, want, max_abs=max_abs,
                                                   mean_abs=mean_abs)
    if over:
        print(f"attention: {over} elements over {max_abs} (|x| >= 8), max abs {worst:.3e}")
    return worst, mean


def assert_attention_close_f32(got, want, *, max_abs=2e-2, mean_abs=1e-3):
    """The north-star bar against the oracle's float32 result.

    ``got`` is the kernel's bf16 output.  Max-abs is taken against the
    unrounded result: every element is within ``max_abs`` except where half a
    bf16 step at |want| is itself larger (|want| >= 8: rounding to bf16 alone
    can move the value that far); there the bound is half a step plus
    2^-9 |want| for the kernel's own arithmetic.  Mean-abs ("in bf16") is taken
    against the result rounded to bf16: outputs of magnitude ~1 carry ~2e-3
    of rounding error on average in bf16 whatever computes them, so against
    the unrounded values the bar would measure the format, not the kernel.
    Returns (max abs error, mean abs error, elements over ``max_abs``).
    """
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    assert got.shape == want.shape
    assert np.isfinite(got).all(), "non-finite attention output"
    err = np.abs(got - want)
    mag = np.maximum(np.abs(want), np.float32(1e-30))
    half = np.exp2(np.floor(np.log2(mag)) - 8).astype(np.float32)   # half a bf16 step
    bound = np.where(half > max_abs, half + mag * np.float32(2.0 ** -9), np.float32(max_abs))
    worst = int(np.argmax(err - bound))
    assert err.flat[worst] <= bound.flat[worst], (
        f"abs error {err.flat[worst]:.3e} > {bound.flat[worst]:.3e} at |x| = {mag.flat[worst]:.3g}"
        f" (max abs error {err.max():.3e})")
    mean = float(np.abs(got - numpy_ref.bf16_round(want)).mean())
    assert mean <= mean_abs, f"mean abs error {mean:.3e} > {mean_abs} (in bf16)"
    return float(err.max()), mean, int((err > max_abs).sum())


def scale_of(dim):
    return 1.0 / math.sqrt(dim)
