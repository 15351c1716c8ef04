"""GPU parity at the configs' stated sizes (C2-C5), through the C ABI.

Inputs come from ``workloads.generate`` (numpy ``default_rng(seed)``, the
configs' draw order: lengths, block-table permutation, queries, keys, values,
outliers).  Each test builds the pool the way a decode step does -- the
cached context first, then the step's own append-and-quantize of the new
tokens -- and checks

* every page's codes, scales and biases bit-exact against the C oracle's
  quantizer (``engine/paged.py:24-41``) on the same tokens, read back with
  ``gather_pages`` (the reference-format block-table gather);
* attention against the C oracle's float32 result (unrounded): within 2e-2
  max-abs except where half a bf16 step is larger, 1e-3 mean-abs
  (``engine/paged_attention.py:209-246`` semantics), with the number of
  elements over 2e-2 reported.

C3 runs with its 512-token partitions (one work wave per partition); C4
builds its 256-token shared prefix through the device arena (one sequence
writes it, fifteen fork it: sixteen references per page) and checks the
reference counts.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import cport
from paged_case import assert_attention_close_f32, to_torch

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from pkv import _native

    _native.load()


def _fmt(w):
    from pkv.ops import PageFormat

    return PageFormat(w.kv_heads, w.head_dim, w.page_tokens, w.bits, w.group_size,
                      torch.bfloat16)


def oracle_arrays(w, keys, values, table, num_pages):
    """Reference-format page arrays indexed by page id, quantized by the C
    oracle; ``counts[p]`` = tokens held by page p."""
    P, HK, D = w.page_tokens, w.kv_heads, w.head_dim
    padded = -(-D // w.group_size) * w.group_size
    dq, ng = padded * w.bits // 8, padded // w.group_size
    arrays = [np.zeros((num_pages, HK, P, dq), np.uint8), np.zeros((num_pages, HK, P, ng),
                                                                   np.float16),
              np.zeros((num_pages, HK, P, ng), np.float16)]
    arrays += [np.zeros_like(a) for a in arrays]
    counts = np.zeros(num_pages, np.int64)
    for b in range(len(keys)):
        L = keys[b].shape[1]
        npg = -(-L // P)
        ids = np.asarray(table[b, :npg])
        for side, src in ((0, keys[b]), (1, values[b])):
            x = np.zeros((HK, npg * P, D), np.float32)
            x[:, :L] = src
            x = np.ascontiguousarray(x.reshape(HK, npg, P, D).transpose(1, 0, 2, 3))
            codes, scale, bias = cport.quantize_rows(x, w.bits, w.group_size)
            arrays[3 * side][ids], arrays[3 * side + 1][ids], arrays[3 * side + 2][ids] = (
                codes, scale, bias)
        counts[ids] = P
        counts[ids[-1]] = L - (npg - 1) * P
    return arrays, counts


def check_pages_bit_exact(fmt, pool, arrays, counts):
    """gather_pages of every written page equals the oracle's tensors up to each
    page's token count."""
    from pkv import ops

    ids = np.nonzero(counts)[0].astype(np.int32)
    got = ops.gather_pages(fmt, pool, torch.from_numpy(ids).cuda())
    torch.cuda.synchronize()
    host = [t.view(torch.int16).cpu().numpy().view(np.uint16) if t.element_size() == 2
            else t.cpu().numpy() for t in got]
    full = counts[ids] == fmt.page_tokens
    for g, want in zip(host, arrays, strict=True):
        w = want[ids]
        if w.dtype == np.float16:
            w = w.view(np.uint16)
        assert np.array_equal(g[full], w[full]), "full pages differ"
        for i in np.nonzero(~full)[0]:
            n = int(counts[ids[i]])
            assert np.array_equal(g[i][:, :n], w[i][:, :n]), f"page {ids[i]} differs"
    return len(ids)


def append(fmt, pool, w, keys, values, table, lo, hi):
    """Append tokens [lo[b], hi[b]) of every sequence (one launch per 256 tokens)."""
    from pkv import ops

    lo, hi = np.asarray(lo), np.asarray(hi)
    t_table = torch.from_numpy(np.ascontiguousarray(table)).cuda()
    for start in range(0, int((hi - lo).max()), 256):
        width = np.clip(hi - lo - start, 0, 256).astype(np.int32)
        n = int(width.max())
        k = np.zeros((len(keys), w.kv_heads, n, w.head_dim), np.float32)
        v = np.zeros_like(k)
        for b in range(len(keys)):
            a, m = int(lo[b]) + start, int(width[b])
            k[b, :, :m], v[b, :, :m] = keys[b][:, a:a + m], values[b][:, a:a + m]
        ops.append_quantize(fmt, pool, to_torch(k, fmt.dtype), to_torch(v, fmt.dtype), t_table,
                            torch.from_numpy((lo + start).astype(np.int32)).cuda(),
                            torch.from_numpy(width).cuda())


def run_config(name, *, waves_of=None):
    """Fill the context, take the step (append + attention), check pages and output."""
    from pkv import ops, workloads

    w = workloads.get(name)
    inst = workloads.generate(w)
    fmt = _fmt(w)
    context = inst.context.astype(np.int64)
    total = inst.total_lengths.astype(np.int64)
    pool = ops.allocate_pool(fmt, inst.num_pages)
    append(fmt, pool, w, inst.keys, inst.values, inst.table, np.zeros_like(context), context)
    if w.append_tokens:                       # the step's own append of its new tokens
        append(fmt, pool, w, inst.keys, inst.values, inst.table, context, total)
    lengths = torch.from_numpy(total.astype(np.int32)).cuda()
    positions = inst.positions
    scale = 1.0 / math.sqrt(w.head_dim)
    waves = waves_of(w, total) if waves_of else 0
    widths = torch.from_numpy(inst.widths).cuda() if w.widths else None
    out = ops.paged_attention(fmt, pool, to_torch(inst.queries, fmt.dtype),
                              torch.from_numpy(inst.table).cuda(), lengths, scale=scale,
                              q_pos=torch.from_numpy(positions).cuda(), widths=widths,
                              waves=waves)
    torch.cuda.synchronize()
    arrays, counts = oracle_arrays(w, inst.keys, inst.values, inst.table, inst.num_pages)
    pages = check_pages_bit_exact(fmt, pool, arrays, counts)
    want = cport.paged_attention(inst.queries, inst.table, total, positions, inst.widths,
                                 heads_kv=w.kv_heads, page_tokens=w.page_tokens, bits=w.bits,
                                 group_size=w.group_size, pages=arrays, scale=scale)
    worst, mean, over = assert_attention_close_f32(out.float().cpu().numpy(), want)
    print(f"{name}: {pages} pages bit-exact, {int(total.sum())} tokens; attention max abs "
          f"{worst:.2e}, mean abs {mean:.2e}, {over} elements over 2e-2")
    assert over == 0
    return out


def test_c2_full_size_decode_step():
    """B32 int8 G64 at the Llama-3-8B shape, L ~ U[1024, 8192], 1% outlier
    channels; the step appends one token per sequence; the library's default
    work split."""
    run_config("c2")


def test_c3_full_size_long_context_512_token_partitions():
    """B8 4-bit G64, 32-token pages, L = 32768: one work wave per 512-token
    partition of every (sequence, KV head), merged by log-sum-exp."""
    import bench

    run_config("c3", waves_of=bench.workload_waves)


def test_c5_full_size_chunked_prefill():
    """B4: a 512-token causal chunk appended over a 4096-token int8 prefix and
    attended by its own 512 queries (the MFMA prefill kernel)."""
    run_config("c5")


def test_mixed_full_size_decode_and_prefill_rows_in_one_call():
    """C2's 32 decode rows and C5's 4 prefill chunks padded into one batch of
    512 query rows: one call serves the decode rows on the split-K kernel and
    the chunks on the prefill kernel; padded rows are zero."""
    out = run_config("mixed")
    assert not out[:32, :, 1:].any()


def test_c4_full_size_verify_over_a_refcounted_shared_prefix():
    """B16 verify, 5 causal drafts, L ~ U[512, 4096]: sequence 0 writes the
    256-token prefix into the device arena, the fifteen others fork it (each
    prefix page then has sixteen references) and append their own tokens; the
    step reserves and appends the 5 drafts of every sequence and attends."""
    from pkv import ops, workloads
    from pkv.device_arena import DevicePageArena

    w = workloads.get("c4")
    inst = workloads.generate(w)
    fmt = _fmt(w)
    context = inst.context.astype(np.int64)
    total = inst.total_lengths.astype(np.int64)
    prefix = w.shared_prefix_pages * w.page_tokens
    distinct = int(sum(-(-int(n) // w.page_tokens) for n in total)) - \
        (w.batch - 1) * w.shared_prefix_pages
    arena = DevicePageArena(fmt, distinct + 8, num_layers=1, max_slots=w.batch,
                            max_tokens=int(total.max()))
    pool = arena.pools[0]
    slots = [arena.open_slot() for _ in range(w.batch)]

    def grow(rows, lo, hi):
        res = arena.reserve([slots[b] for b in rows], [int(hi[b] - lo[b]) for b in rows])
        table = res.table.cpu().numpy()
        append(fmt, pool, w, [inst.keys[b] for b in rows], [inst.values[b] for b in rows], table,
               [lo[b] for b in rows], [hi[b] for b in rows])
        return res

    zeros = np.zeros(w.batch, np.int64)
    grow([0], zeros, np.full(w.batch, prefix))
    for b in range(1, w.batch):
        arena.fork([slots[0]], [slots[b]])
    grow(range(w.batch), np.full(w.batch, prefix), context)
    res = grow(range(w.batch), context, total)          # the step: the drafts
    assert arena.check() >= 0                           # no device error bits
    table = res.table.cpu().numpy()
    assert (table[:, :w.shared_prefix_pages] == table[0, :w.shared_prefix_pages]).all()
    refs = arena.refcounts().numpy()
    assert (refs[table[0, :w.shared_prefix_pages]] == w.batch).all()
    scale = 1.0 / math.sqrt(w.head_dim)
    out = ops.paged_attention(fmt, pool, to_torch(inst.queries, fmt.dtype), res.table, res.lens,
                              scale=scale, q_pos=torch.from_numpy(inst.positions).cuda(),
                              widths=res.widths)
    torch.cuda.synchronize()
    pages = np.maximum(table, 0)
    arrays, counts = oracle_arrays(w, inst.keys, inst.values, pages, arena.capacity)
    checked = check_pages_bit_exact(fmt, pool, arrays, counts)
    assert checked == distinct
    want = cport.paged_attention(inst.queries, pages, total, inst.positions,
                                 np.full(w.batch, w.num_queries, np.int32), heads_kv=w.kv_heads,
                                 page_tokens=w.page_tokens, bits=w.bits, group_size=w.group_size,
                                 pages=arrays, scale=scale)
    worst, mean, over = assert_attention_close_f32(out.float().cpu().numpy(), want)
    print(f"c4: {checked} pages bit-exact ({w.shared_prefix_pages} shared by {w.batch}); "
          f"attention max abs {worst:.2e}, mean abs {mean:.2e}, {over} elements over 2e-2")
    assert over == 0
