"""GPU: the fused single-token step (``pkv_append_paged_attention``) through the C ABI.

One launch appends each sequence's new K/V token and attends its query where
the decode kernel serves the shape (quantized pages, <= 8 query rows per KV
head); other shapes run an append launch and the attention.  Either way the
pages must equal ``pkv_append_quantize`` followed by ``pkv_paged_attention``
bit for bit, and both outputs must meet the oracle's bar
(``engine/paged.py:260-263`` is the reference's append-then-attend pair).
At the case's wave count the outputs are not compared bit for bit: the fused
launch's split charges 16 lead tiles per segment instead of 8, so its pieces
differ, and with them each piece's running maximum, hence the f16 rounding
of its P' operands (outlier channels make that visible at one or two bf16
steps).  With one wave both splits are one piece per segment, and there the
outputs must be equal bit for bit.
"""

from __future__ import annotations

import types

import numpy as np
import pytest

from paged_case import assert_attention_close, fill_pages, oracle_attention, scale_of, to_torch

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from pkv import _native

    _native.load()


def _fmt(w, dtype=None):
    from pkv.ops import PageFormat

    return PageFormat(w.kv_heads, w.head_dim, w.page_tokens, w.bits, w.group_size,
                      dtype or torch.bfloat16)


def _context_pool(fmt, inst):
    """A pool holding every sequence's tokens but the last (the step's new
    one); returns ``(pool, table, lengths after the step)``."""
    from pkv import ops

    lens = np.array([k.shape[1] for k in inst.keys])
    table = torch.from_numpy(inst.table).cuda()
    if (lens > 1).any():
        ctx = types.SimpleNamespace(workload=inst.workload, table=inst.table,
                                    num_pages=inst.num_pages,
                                    keys=[k[:, :-1] for k in inst.keys],
                                    values=[v[:, :-1] for v in inst.values])
        pool, table, _ = fill_pages(fmt, ctx, chunk=64)
    else:
        pool = ops.allocate_pool(fmt, inst.num_pages)
    return pool, table, torch.from_numpy(lens.astype(np.int32)).cuda()


def _new_rows(inst, fmt):
    k = np.stack([kk[:, -1:] for kk in inst.keys])     # [B, HK, 1, D]
    v = np.stack([vv[:, -1:] for vv in inst.values])
    return to_torch(k, fmt.dtype), to_torch(v, fmt.dtype)


CASES = {
    # name: (workload overrides, waves); every case is a single-token step
    "c2_small_default_waves": (dict(name="c2", batch=6, length_range=(1, 700)), 0),
    "c2_small_waves_3": (dict(name="c2", batch=5, length_range=(17, 900)), 3),
    "c2_many_waves_short_pieces": (dict(name="c2", batch=4, lengths=(33, 1, 200, 64)), 500),
    "c2_one_wave": (dict(name="c2", batch=3, lengths=(1500, 16, 31)), 1),
    "every_tile_position": (dict(name="c2", batch=16, lengths=tuple(range(100, 116))), 0),
    "gqa8_slots2_4bit_g32": (dict(name="c3", batch=3, lengths=(300, 47, 1030), group_size=32), 0),
    "int8_d100_p32": (dict(name="c2", batch=4, lengths=(90, 7, 260, 33), head_dim=100,
                           group_size=32, page_tokens=32), 9),
    "int4_d64_p64": (dict(name="c2", batch=3, lengths=(129, 64, 5), bits=4, head_dim=64,
                          group_size=32, page_tokens=64), 0),
    "b80_chunks": (dict(name="c2", batch=80, length_range=(1, 300)), 37),
    "int8_d256_g128": (dict(name="c2", batch=3, lengths=(300, 17, 90), head_dim=256,
                            group_size=128), 0),
    "int8_d256_g32_gqa8": (dict(name="c2", batch=3, lengths=(129, 2, 48), head_dim=256,
                                group_size=32, kv_heads=4), 5),
    "int4_d256_g64_p32": (dict(name="c3", batch=2, lengths=(200, 45), head_dim=256), 0),
    "int8_g128_gqa8_p64": (dict(name="c2", batch=4, lengths=(64, 65, 500, 3), kv_heads=4,
                                group_size=128, page_tokens=64), 0),
    # served by two launches inside the entry point
    "fallback_bf16_pages": (dict(name="c2", batch=3, lengths=(40, 3, 70), bits=16,
                                 group_size=32), 0),
    "fallback_rows16": (dict(name="c2", batch=3, lengths=(50, 18, 200), heads=32, kv_heads=2), 0),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_fused_step_equals_append_then_attend(case):
    overrides, waves = CASES[case]
    _fused_against_separate(overrides, waves)


# head_dim -> quantization groups the page format supports there
_GROUPS = {64: (32, 64), 100: (32,), 128: (32, 64, 128), 256: (32, 64, 128)}


@pytest.mark.parametrize("seed", list(range(24)) + list(range(100, 160)))
def test_fused_step_random_shapes(seed):
    """Seeded random single-token steps over the shapes the fused launch
    serves (4 or 8 bits, head_dim 64/100/128/256 with their groups, pages of
    16-64 tokens, 1-8 query heads per KV head, ragged lengths from 1 token,
    default and odd wave counts), each checked as the fixed cases are."""
    rng = np.random.default_rng(1000 + seed)
    dim = int(rng.choice(list(_GROUPS)))
    kv = int(rng.choice([1, 2, 4, 8]))
    batch = int(rng.integers(1, 13))
    overrides = dict(name="c2", batch=batch, bits=int(rng.choice([4, 8])), head_dim=dim,
                     group_size=int(rng.choice(_GROUPS[dim])),
                     page_tokens=int(rng.choice([16, 32, 64])), kv_heads=kv,
                     heads=kv * int(rng.choice([1, 2, 4, 8])),
                     lengths=tuple(int(x) for x in rng.integers(1, 1500, size=batch)))
    waves = int(rng.choice([0, 0, 1, 3, 17, 64]))
    print(f"seed {seed}: {overrides}, waves {waves}", flush=True)
    _fused_against_separate(overrides, waves)


def _fused_against_separate(overrides, waves):
    from pkv import ops, workloads

    overrides = dict(overrides)
    w = workloads.get(overrides.pop("name"), num_queries=1, append_tokens=1,
                      shared_prefix_pages=0, **overrides)
    inst = workloads.generate(w)
    fmt = _fmt(w)
    k_new, v_new = _new_rows(inst, fmt)
    q = to_torch(inst.queries, fmt.dtype)
    scale = scale_of(w.head_dim)
    # separate: append at L - 1, then attend
    pool_a, table, lens = _context_pool(fmt, inst)
    ops.append_quantize(fmt, pool_a, k_new, v_new, table, lens - 1)
    want_out = ops.paged_attention(fmt, pool_a, q, table, lens, scale=scale, waves=waves)
    # fused
    pool_b, _, _ = _context_pool(fmt, inst)
    got_out = ops.append_paged_attention(fmt, pool_b, k_new, v_new, q, table, lens, scale=scale,
                                         waves=waves)
    torch.cuda.synchronize()
    assert torch.equal(pool_a, pool_b), "pages differ"
    want = oracle_attention(fmt, inst, inst.positions, np.ones(w.batch, np.int32), scale)
    assert_attention_close(want_out.float().cpu().numpy(), want)
    assert_attention_close(got_out.float().cpu().numpy(), want)
    # one wave: the same pieces in both forms.  The fused form runs one wave
    # per run; the separate attention of a two-column-slot shape runs each run
    # on a group of four waves that meet by log-sum-exp, so its sums run in
    # another order (and its P' operands, rounded to f16, see other running
    # maxima): two bf16 steps of the element plus 2^-8 of the row's largest
    # element apart at most (single-wave shapes: equal).  Seeded sweeps of
    # 84 shapes put the largest gap at 4-bit pages, 8 rows per KV head: about
    # 2^-7 of the row's largest element, the two forms' f32 sums rounding to
    # bf16 values two steps apart; both forms meet the oracle's bar above.
    pool_c, _, _ = _context_pool(fmt, inst)
    ops.append_quantize(fmt, pool_c, k_new, v_new, table, lens - 1)
    one_a = ops.paged_attention(fmt, pool_c, q, table, lens, scale=scale, waves=1)
    pool_d, _, _ = _context_pool(fmt, inst)
    one_b = ops.append_paged_attention(fmt, pool_d, k_new, v_new, q, table, lens, scale=scale,
                                       waves=1)
    torch.cuda.synchronize()
    assert torch.equal(pool_c, pool_d), "pages differ (one wave)"
    a32, b32 = one_a.float(), one_b.float()
    big = torch.maximum(a32.abs(), b32.abs())
    bound = big * 2.0 ** -6 + big.amax(dim=-1, keepdim=True) * 2.0 ** -8
    assert bool(((a32 - b32).abs() <= bound).all()), "outputs differ (one wave)"


def test_fused_step_c2_full_size_against_the_oracle():
    """C2 at its stated size: the context filled by appends, then one fused
    step; pages (bit-exact, against the C oracle's quantizer) and attention as
    in the full-size parity test."""
    import math

    from oracle import cport
    from paged_case import assert_attention_close_f32
    from pkv import ops, workloads
    from test_gpu_fullsize import append, check_pages_bit_exact, oracle_arrays

    w = workloads.get("c2")
    inst = workloads.generate(w)
    fmt = _fmt(w)
    context = inst.context.astype(np.int64)
    total = inst.total_lengths.astype(np.int64)
    pool = ops.allocate_pool(fmt, inst.num_pages)
    append(fmt, pool, w, inst.keys, inst.values, inst.table, np.zeros_like(context), context)
    k_new, v_new = _new_rows(inst, fmt)
    lens = torch.from_numpy(total.astype(np.int32)).cuda()
    table = torch.from_numpy(inst.table).cuda()
    scale = 1.0 / math.sqrt(w.head_dim)
    out = ops.append_paged_attention(fmt, pool, k_new, v_new, to_torch(inst.queries, fmt.dtype),
                                     table, lens, scale=scale)
    torch.cuda.synchronize()
    arrays, counts = oracle_arrays(w, inst.keys, inst.values, inst.table, inst.num_pages)
    pages = check_pages_bit_exact(fmt, pool, arrays, counts)
    want = cport.paged_attention(inst.queries, inst.table, total, inst.positions, inst.widths,
                                 heads_kv=w.kv_heads, page_tokens=w.page_tokens, bits=w.bits,
                                 group_size=w.group_size, pages=arrays, scale=scale)
    worst, mean, over = assert_attention_close_f32(out.float().cpu().numpy(), want)
    print(f"fused c2: {pages} pages bit-exact; attention max abs {worst:.2e}, mean abs "
          f"{mean:.2e}, {over} elements over 2e-2")
    assert over == 0


def test_fused_step_rejects_bad_shapes():
    from pkv import ops, workloads

    w = workloads.get("c2", batch=2, lengths=(10, 20), num_queries=1, append_tokens=1)
    inst = workloads.generate(w)
    fmt = _fmt(w)
    pool, table, lens = _context_pool(fmt, inst)
    k_new, v_new = _new_rows(inst, fmt)
    q = to_torch(inst.queries, fmt.dtype)
    with pytest.raises(ValueError):
        ops.append_paged_attention(fmt, pool, k_new[:, :, :0], v_new, q, table, lens, scale=0.1)
    with pytest.raises(ValueError):
        ops.append_paged_attention(fmt, pool, k_new, v_new, q.repeat(1, 1, 2, 1), table, lens,
                                   scale=0.1)
