"""GPU: the VALU decode kernel (``pkv_select_decode_kernel(PKV_DECODE_VALU)``)
against the CPU oracle.

The vector-ALU form of the decode kernel serves calls of at most 4 query rows
per KV head over quantized pages at head_dim <= 128 (single-token decode at
GQA <= 4) with the MFMA kernel's work split, partials and merge; only the
products differ (v_dot2_f32_f16 instead of MFMA), so every case here is one
the MFMA kernel passes too, checked to the same bars: the eligible cases of
the attention parity table, seeded random shapes, stale page bytes, queries
far outside N(0,1), and C2 at its stated size.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import numpy_ref
from paged_case import assert_attention_close, fill_pages, oracle_attention, scale_of, to_torch
from test_gpu_parity import ATTN_CASES, _random_attention_cases

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _valu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from pkv import _native, ops

    _native.load()
    previous = ops.select_decode_kernel("valu")
    yield
    ops.select_decode_kernel(previous)


def _fmt(w, dtype=None):
    from pkv.ops import PageFormat

    return PageFormat(w.kv_heads, w.head_dim, w.page_tokens, w.bits, w.group_size,
                      dtype or torch.bfloat16)


def _eligible(w):
    """Shapes the VALU kernel serves: <= 4 rows per KV head, quantized, D <= 128."""
    rows = w.num_queries * (w.heads // w.kv_heads)
    stored = -(-w.head_dim // w.group_size) * w.group_size if w.bits != 16 else w.head_dim
    return rows <= 4 and w.bits != 16 and stored <= 128


def _attention(w, inst, fmt, waves, *, pool=None):
    from pkv import ops

    if pool is None:
        pool, table, lengths = fill_pages(fmt, inst, chunk=64)
    else:
        pool, table, lengths = pool
    scale = scale_of(w.head_dim)
    out = ops.paged_attention(fmt, pool, to_torch(inst.queries, fmt.dtype), table, lengths,
                              scale=scale, q_pos=torch.from_numpy(inst.positions).cuda(),
                              waves=waves)
    torch.cuda.synchronize()
    widths = np.full(w.batch, w.num_queries, np.int32)
    return out, oracle_attention(fmt, inst, inst.positions, widths, scale)


def _table_cases():
    from pkv import workloads

    names = []
    for name, (overrides, dtype, chunk, waves) in sorted(ATTN_CASES.items()):
        o = dict(overrides)
        if _eligible(workloads.get(o.pop("name"), **o)):
            names.append(name)
    return names


@pytest.mark.parametrize("case", _table_cases())
def test_valu_decode_matches_oracle(case):
    from pkv import ops, workloads

    overrides, dtype, chunk, waves = ATTN_CASES[case]
    overrides = dict(overrides)
    w = workloads.get(overrides.pop("name"), **overrides)
    inst = workloads.generate(w)
    if dtype == "float16":
        inst.keys = [k.astype(np.float16).astype(np.float32) for k in inst.keys]
        inst.values = [v.astype(np.float16).astype(np.float32) for v in inst.values]
        inst.queries = inst.queries.astype(np.float16).astype(np.float32)
    fmt = _fmt(w, getattr(torch, dtype))
    out, want = _attention(w, inst, fmt, waves, pool=fill_pages(fmt, inst, chunk=chunk))
    assert_attention_close(out.float().cpu().numpy(), want)


def _random_valu_cases():
    """Seeded random shapes restricted to what the VALU kernel serves: 4/8-bit
    G32/G64/G128, D 37-128, pages of 16-64 tokens, 1-4 rows per KV head."""
    rng = np.random.default_rng(7)
    cases = []
    for i in range(40):
        bits = int(rng.choice([4, 8]))
        dim = int(rng.choice([37, 64, 100, 128]))
        group = int(rng.choice([32, 64, 128]))
        if -(-dim // group) * group not in (64, 128):
            group = 32
        gqa = int(rng.choice([1, 2, 4]))
        nq = int(rng.integers(1, 4 // gqa + 1))
        kv_heads = int(rng.choice([1, 2, 8]))
        batch = int(rng.integers(1, 12))
        lengths = tuple(int(x) for x in rng.choice([0, 1, 3, 15, 16, 17, 64, 65, 300, 1025],
                                                   size=batch))
        cases.append(dict(bits=bits, head_dim=dim, group_size=group,
                          page_tokens=int(rng.choice([16, 32, 64])), kv_heads=kv_heads,
                          heads=kv_heads * gqa, num_queries=nq, append_tokens=nq, batch=batch,
                          lengths=lengths, waves=int(rng.choice([0, 1, 5, 33, 400])),
                          seed=int(rng.integers(1 << 30)), index=i))
    return cases


@pytest.mark.parametrize("case", _random_valu_cases() + [
    c for c in _random_attention_cases(48, seed=2026)
    if c["bits"] != 16 and c["num_queries"] * (c["heads"] // c["kv_heads"]) <= 4
    and -(-c["head_dim"] // c["group_size"]) * c["group_size"] <= 128],
    ids=lambda c: f"v{c['index']}")
def test_valu_decode_random_shapes_match_oracle(case):
    from pkv import workloads

    case = dict(case)
    waves = case.pop("waves")
    case.pop("index")
    w = workloads.get("c2", shared_prefix_pages=0, outlier_fraction=0.0, length_range=(),
                      **case)
    assert _eligible(w)
    inst = workloads.generate(w)
    out, want = _attention(w, inst, _fmt(w), waves)
    assert_attention_close(out.float().cpu().numpy(), want)


@pytest.mark.parametrize("factor", [30.0, 300.0, 1e6, 3e-6])
def test_valu_decode_large_and_tiny_queries(factor):
    """bf16 queries x1e6 pass the f16 range: the row is scaled by a power of
    two before conversion and the inverse folded into its score scale."""
    from pkv import workloads

    w = workloads.get("c2", batch=4, length_range=(3, 600))
    inst = workloads.generate(w)
    inst.queries = numpy_ref.bf16_round(inst.queries * np.float32(factor))
    fmt = _fmt(w)
    pages = fill_pages(fmt, inst, chunk=64)
    for waves in (0, 7):
        out, want = _attention(w, inst, fmt, waves, pool=pages)
        assert_attention_close(out.float().cpu().numpy(), want)


@pytest.mark.parametrize("bits", [8, 4])
def test_valu_decode_ignores_stale_bytes_of_reused_pages(bits):
    """Every pool byte starts as 0xFF (NaN scales and biases) before the
    sequences' tokens are appended: tokens past each sequence's end must not
    reach the output."""
    from pkv import ops, workloads

    w = workloads.get("c2", batch=5, lengths=(1, 7, 16, 33, 250), heads=16, kv_heads=4,
                      bits=bits, outlier_fraction=0.0)
    inst = workloads.generate(w)
    fmt = _fmt(w)
    clean_pages = fill_pages(fmt, inst, chunk=16)
    pool, table, lengths = clean_pages
    stale = ops.allocate_pool(fmt, pool.shape[0]).fill_(0xFF)
    n = np.array([k.shape[1] for k in inst.keys])
    for start in range(0, int(n.max()), 16):
        width = np.clip(n - start, 0, 16).astype(np.int32)
        k = np.zeros((w.batch, w.kv_heads, 16, w.head_dim), np.float32)
        v = np.zeros_like(k)
        for b in range(w.batch):
            k[b, :, :width[b]] = inst.keys[b][:, start:start + width[b]]
            v[b, :, :width[b]] = inst.values[b][:, start:start + width[b]]
        ops.append_quantize(fmt, stale, to_torch(k, fmt.dtype), to_torch(v, fmt.dtype), table,
                            torch.full((w.batch,), start, dtype=torch.int32, device="cuda"),
                            torch.from_numpy(width).cuda())
    for waves in (0, 3):
        out, want = _attention(w, inst, fmt, waves, pool=(stale, table, lengths))
        clean, _ = _attention(w, inst, fmt, waves, pool=clean_pages)
        assert torch.equal(out, clean), waves
        assert_attention_close(out.float().cpu().numpy(), want)


def test_valu_and_mfma_kernels_agree_and_the_switch_takes_effect():
    """Both kernels on the same inputs: each within the bar of the oracle,
    within f32 rounding of each other, and not bit-identical (different
    summation order) -- so the selection reached the launch."""
    from pkv import ops, workloads

    w = workloads.get("c2", batch=6, length_range=(100, 2000))
    inst = workloads.generate(w)
    fmt = _fmt(w)
    pages = fill_pages(fmt, inst, chunk=64)
    valu, want = _attention(w, inst, fmt, 0, pool=pages)
    ops.select_decode_kernel("mfma")
    try:
        mfma, _ = _attention(w, inst, fmt, 0, pool=pages)
    finally:
        ops.select_decode_kernel("valu")
    assert_attention_close(valu.float().cpu().numpy(), want)
    assert_attention_close(mfma.float().cpu().numpy(), want)
    diff = (valu.float() - mfma.float()).abs()
    assert float(diff.max()) < 2e-2
    assert not torch.equal(valu, mfma)


def test_valu_decode_c2_full_size():
    """C2 at its stated size (B32, L ~ U[1024, 8192], int8 G64, the step's own
    append) on the VALU kernel: pages bit-exact, attention within the bar."""
    from test_gpu_fullsize import run_config

    run_config("c2")


def test_select_decode_kernel_rejects_unknown_kinds():
    from pkv import _native, ops

    with pytest.raises(ValueError):
        ops.select_decode_kernel("simd")
    lib = _native.load()
    assert lib.pkv_select_decode_kernel(7) == _native.PKV_INVALID_ARGUMENT
    assert ops.select_decode_kernel("valu") == "valu"
