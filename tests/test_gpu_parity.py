"""GPU parity: libpkv (through the C ABI) against the CPU oracle on seeded inputs.

Bars (north star): bit-exact quantized codes, scales, biases and block-table
gathers; attention within 2e-2 max-abs and 1e-3 mean-abs in bf16.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import cport, numpy_ref
from paged_case import (assert_attention_close, fill_pages, oracle_attention, oracle_pages,
                        scale_of, to_torch)

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from pkv import _native

    _native.load()  # fails loudly when libpkv.so is missing


def _fmt(w, dtype=None):
    from pkv.ops import PageFormat

    return PageFormat(w.kv_heads, w.head_dim, w.page_tokens, w.bits, w.group_size,
                      dtype or torch.bfloat16)


# ---------------------------------------------------------------- quantizer


GOLDEN = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "quantize_page_g32.npz")
CASES = sorted({k.split("/")[0] for k in GOLDEN.files})


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("bits", [4, 8])
def test_quantize_rows_matches_reference_golden(case, bits):
    from pkv import ops

    x = GOLDEN[f"{case}/input"]
    dtype = torch.float16 if x.dtype == np.float16 else torch.bfloat16
    t = torch.from_numpy(x.astype(np.float32)).to("cuda", dtype)
    codes, scale, bias = ops.quantize_rows(t, bits, 32)
    torch.cuda.synchronize()
    assert np.array_equal(codes.cpu().numpy(), GOLDEN[f"{case}/b{bits}/codes"])
    assert np.array_equal(scale.cpu().numpy().view(np.uint16),
                          GOLDEN[f"{case}/b{bits}/scale"].view(np.uint16))
    assert np.array_equal(bias.cpu().numpy().view(np.uint16),
                          GOLDEN[f"{case}/b{bits}/bias"].view(np.uint16))
    restored = ops.dequantize_rows((codes, scale, bias), bits, x.shape[-1], 32)
    assert np.array_equal(restored.cpu().numpy(), GOLDEN[f"{case}/b{bits}/dequant"])


@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_quantize_rows_matches_c_oracle(group, bits, dtype):
    from pkv import ops

    rng = np.random.default_rng(7 + group + bits)
    x = rng.standard_normal((2048, 128)).astype(np.float32)
    x[:, rng.choice(128, 2, replace=False)] *= 8
    x[::97] *= 300.0           # wide groups
    x[5::113] = 0.25           # constant groups
    x = x.astype(np.float16).astype(np.float32) if dtype == "float16" else numpy_ref.bf16_round(x)
    t = torch.from_numpy(x).to("cuda", getattr(torch, dtype))
    codes, scale, bias = ops.quantize_rows(t, bits, group)
    want = cport.quantize_rows(x, bits, group)
    assert np.array_equal(codes.cpu().numpy(), want[0])
    assert np.array_equal(scale.cpu().numpy().view(np.uint16), want[1].view(np.uint16))
    assert np.array_equal(bias.cpu().numpy().view(np.uint16), want[2].view(np.uint16))


# ------------------------------------------------------- append + gather


LAYOUTS = [
    # bits, head_dim, group, page, dtype, chunk
    (8, 128, 64, 16, "bfloat16", 1),
    (8, 128, 64, 16, "bfloat16", 37),
    (8, 128, 32, 32, "float16", 5),
    (8, 128, 128, 16, "bfloat16", 64),
    (4, 128, 64, 32, "bfloat16", 7),
    (4, 128, 32, 16, "float16", 16),
    (8, 64, 32, 16, "bfloat16", 9),
    (4, 64, 64, 64, "bfloat16", 33),
    (8, 37, 32, 16, "float16", 11),
    (4, 256, 64, 16, "bfloat16", 3),
    (16, 64, 32, 16, "bfloat16", 13),
    (16, 128, 32, 32, "float16", 5),
    (16, 100, 32, 16, "bfloat16", 17),
]


def _small(bits, dim, group, page, batch=3, lengths=(1, 40, 77), seed=11):
    from pkv import workloads

    return workloads.Workload("t", batch=batch, heads=4 * 2, kv_heads=2, head_dim=dim,
                              page_tokens=page, bits=bits, group_size=group,
                              lengths=tuple(lengths), seed=seed)


@pytest.mark.parametrize("bits,dim,group,page,dtype,chunk", LAYOUTS)
def test_append_then_gather_is_bit_exact(bits, dim, group, page, dtype, chunk):
    from pkv import ops, workloads

    w = _small(bits, dim, group, page)
    inst = workloads.generate(w)
    if dtype == "float16":
        inst.keys = [k.astype(np.float16).astype(np.float32) for k in inst.keys]
        inst.values = [v.astype(np.float16).astype(np.float32) for v in inst.values]
    fmt = _fmt(w, getattr(torch, dtype))
    pool, table, lengths = fill_pages(fmt, inst, chunk=chunk)
    ref = numpy_ref.RefPages(w.kv_heads, dim, page, bits=None if bits == 16 else bits,
                             group_size=group, dtype=dtype, tail="quantized")
    for b in range(w.batch):
        ref.write_sequence(inst.table[b], inst.keys[b], inst.values[b])
    ids = sorted(ref.pages)
    raw = lambda t: (t.view(torch.int16).cpu().numpy().view(np.uint16) if t.element_size() == 2
                     else t.cpu().numpy())
    got = [raw(t) for t in ops.gather_pages(fmt, pool, ids)]
    for i, pid in enumerate(ids):
        count = ref.pages[pid][2]
        for g_arr, w_arr in zip(got, ref.state(pid)):
            w_page = np.asarray(w_arr)[:, :count]
            if w_page.dtype == np.float16:
                w_bits = w_page.view(np.uint16)
            elif w_page.dtype == np.float32:   # float pages, values already in page dtype
                w_bits = (w_page.astype(np.float16).view(np.uint16) if dtype == "float16" else
                          (w_page.view(np.uint32) >> 16).astype(np.uint16))
            else:
                w_bits = w_page
            assert np.array_equal(g_arr[i][:, :count], w_bits), f"page {pid}"


def test_copy_pages_duplicates_page_bytes():
    from pkv import ops

    w = _small(8, 128, 64, 16)
    fmt = _fmt(w)
    pool = torch.randint(0, 256, (8, fmt.page_bytes), dtype=torch.uint8, device="cuda")
    ops.copy_pages(fmt, pool, [1, 3], [6, 7])
    torch.cuda.synchronize()
    assert torch.equal(pool[6], pool[1]) and torch.equal(pool[7], pool[3])


# ------------------------------------------------------------- attention


ATTN_CASES = {
    # name: (workload overrides, dtype, chunk, waves); waves 0 = the device's
    # resident capacity, small counts split most (sequence, KV head) pairs
    # into pieces merged in-kernel, 1 runs everything through one wave
    "c1_bf16": (dict(name="c1"), "bfloat16", 64, 0),
    "c1_bf16_waves5": (dict(name="c1"), "bfloat16", 128, 5),
    "c2_small": (dict(name="c2", batch=4, length_range=(1, 900)), "bfloat16", 100, 0),
    "c2_small_waves13": (dict(name="c2", batch=5, length_range=(17, 700)), "bfloat16", 50, 13),
    "c2_g32_f16": (dict(name="c2", batch=3, length_range=(100, 400), group_size=32), "float16",
                   64, 3),
    "c2_one_wave_long": (dict(name="c2", batch=2, lengths=(2100, 1500)), "bfloat16", 256, 1),
    # one piece of 313 pages: the 64-page window slides four times
    "c2_one_wave_two_slides": (dict(name="c2", batch=1, lengths=(5000,)), "bfloat16", 512, 1),
    "c3_small": (dict(name="c3", batch=2, lengths=(1500, 2048)), "bfloat16", 512, 0),
    "c3_partitions512": (dict(name="c3", batch=2, lengths=(2048, 2048)), "bfloat16", 512, 32),
    "c3_one_wave_long": (dict(name="c3", batch=1, lengths=(4100,)), "bfloat16", 512, 1),
    "c4_small": (dict(name="c4", batch=4, length_range=(300, 700)), "bfloat16", 128, 0),
    "c4_waves9": (dict(name="c4", batch=3, length_range=(260, 520)), "bfloat16", 64, 9),
    "d37_int8": (dict(name="c2", batch=3, length_range=(20, 200), head_dim=37, group_size=32),
                 "bfloat16", 40, 2),
    "f16_pages": (dict(name="c1", bits=16), "float16", 64, 1),
    "more_waves_than_tiles": (dict(name="c2", batch=2, lengths=(40, 3)), "bfloat16", 16, 10000),
    # the split's lead tiles ahead of each segment: runs that end inside a
    # lead (no piece), one-tile segments, pieces starting inside a lead
    "lead_short_segments_waves7": (dict(name="c2", batch=6, lengths=(1, 16, 17, 300, 2, 33)),
                                   "bfloat16", 16, 7),
    "lead_short_segments_waves61": (dict(name="c2", batch=6, lengths=(1, 16, 17, 300, 2, 33)),
                                    "bfloat16", 16, 61),
    "lead_c4_waves50": (dict(name="c4", batch=3, lengths=(5, 49, 700)), "bfloat16", 64, 50),
    # more than 64 sequences: the split walks the lengths in 64-sequence
    # chunks (segment lookup, lead alignment test, merge)
    "b80_short_default_waves": (dict(name="c2", batch=80, length_range=(1, 300)), "bfloat16",
                                32, 0),
    "b80_short_waves37": (dict(name="c2", batch=80, length_range=(1, 300)), "bfloat16", 32, 37),
    "b130_c4_waves500": (dict(name="c4", batch=130, length_range=(5, 90),
                              shared_prefix_pages=0), "bfloat16", 32, 500),
    # 17-32 rows per KV head (two row blocks): one metadata group per head
    # (G128), 4-bit at 32-token pages, head_dim 64, short pieces, one wave
    # sliding the page-id window
    "rows17to32_c4_g128": (dict(name="c4", batch=3, length_range=(200, 700), group_size=128),
                       "bfloat16", 64, 0),
    "rows17to32_4bit_rows24_p32": (dict(name="c3", batch=2, lengths=(700, 1500), num_queries=3,
                                    append_tokens=3), "bfloat16", 128, 0),
    "rows17to32_d64_g32_waves13": (dict(name="c4", batch=3, length_range=(100, 600), head_dim=64,
                                    group_size=32), "bfloat16", 64, 13),
    "rows17to32_short_pieces_waves90": (dict(name="c4", batch=4, lengths=(5, 20, 37, 300)),
                                    "bfloat16", 64, 90),
    "rows17to32_one_wave_long": (dict(name="c4", batch=1, lengths=(2100,)), "bfloat16", 256, 1),
    # few waves per (sequence, KV head): one long sequence is cut into ~40
    # pieces, the rest stay whole
    "fused_skewed_many_pieces": (dict(name="c2", batch=8, heads=4, kv_heads=1,
                                      lengths=(8000,) + (16,) * 7), "bfloat16", 256, 40),
    "fused_gqa8_rows8": (dict(name="c3", batch=3, lengths=(900, 2048, 33)), "bfloat16", 128, 20),
    # wide query blocks (> 32 rows per KV head, or > 16 at head_dim 256) run
    # on the chunked-prefill kernel: 128-row blocks, causal over the chunk
    "prefill_c5_small": (dict(name="c5", batch=2, lengths=(300, 170), num_queries=128,
                              append_tokens=128), "bfloat16", 64, 0),
    "prefill_partial_block": (dict(name="c5", batch=2, lengths=(33, 0), num_queries=37,
                                   append_tokens=37), "bfloat16", 16, 0),
    "prefill_g32_f16": (dict(name="c5", batch=2, lengths=(90, 260), num_queries=64,
                             append_tokens=64, group_size=32), "float16", 100, 0),
    "prefill_g128": (dict(name="c5", batch=1, lengths=(200,), num_queries=40, append_tokens=40,
                          group_size=128), "bfloat16", 80, 0),
    "prefill_4bit_p32": (dict(name="c5", batch=2, lengths=(500, 77), num_queries=96,
                              append_tokens=96, bits=4, page_tokens=32), "bfloat16", 128, 0),
    "prefill_4bit_d64_p64": (dict(name="c5", batch=2, lengths=(129, 64), num_queries=48,
                                  append_tokens=48, bits=4, head_dim=64, group_size=32,
                                  page_tokens=64), "bfloat16", 64, 0),
    "prefill_d37": (dict(name="c5", batch=2, lengths=(60, 150), num_queries=33, append_tokens=33,
                         head_dim=37, group_size=32), "bfloat16", 40, 0),
    "prefill_d256_rows20": (dict(name="c5", batch=3, lengths=(100, 260, 31), num_queries=5,
                                 append_tokens=5, head_dim=256, group_size=128), "bfloat16",
                            64, 0),
    "prefill_d256_4bit": (dict(name="c5", batch=2, lengths=(140, 50), num_queries=20,
                               append_tokens=20, head_dim=256, bits=4, group_size=32),
                          "bfloat16", 64, 0),
    "prefill_bf16_pages": (dict(name="c5", batch=2, lengths=(180, 20), num_queries=64,
                                append_tokens=64, bits=16), "bfloat16", 64, 0),
    "prefill_f16_pages_d64": (dict(name="c5", batch=2, lengths=(70, 130), num_queries=40,
                                   append_tokens=40, bits=16, head_dim=64), "float16", 32, 0),
    "prefill_bf16_pages_d100": (dict(name="c5", batch=1, lengths=(150,), num_queries=36,
                                     append_tokens=36, bits=16, head_dim=100), "bfloat16",
                                50, 0),
}


@pytest.mark.parametrize("case", sorted(ATTN_CASES))
def test_attention_matches_oracle(case):
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
    pool, table, lengths = fill_pages(fmt, inst, chunk=chunk)
    positions = inst.positions
    widths = np.full(w.batch, w.num_queries, np.int32)
    scale = scale_of(w.head_dim)
    q = to_torch(inst.queries, fmt.dtype)
    out = ops.paged_attention(fmt, pool, q, table, lengths, scale=scale,
                              q_pos=torch.from_numpy(positions).cuda(), waves=waves)
    torch.cuda.synchronize()
    want = oracle_attention(fmt, inst, positions, widths, scale)
    assert_attention_close(out.float().cpu().numpy(), want)


@pytest.mark.parametrize("nq", [5, 64])
def test_attention_takes_transposed_query_views(nq):
    """Queries laid out [B, Q, H, D] and passed as their [B, H, Q, D] transpose
    (a strided view) give the oracle's result; a wrong-shaped or strided
    ``out`` is rejected."""
    from pkv import ops, workloads

    w = workloads.get("c4", batch=3, length_range=(100, 400), num_queries=nq,
                      append_tokens=nq, shared_prefix_pages=0)
    inst = workloads.generate(w)
    fmt = _fmt(w)
    pool, table, lengths = fill_pages(fmt, inst, chunk=64)
    scale = scale_of(w.head_dim)
    bqhd = to_torch(inst.queries.transpose(0, 2, 1, 3), fmt.dtype)      # [B, Q, H, D]
    q = bqhd.transpose(1, 2)
    assert not q.is_contiguous()
    q_pos = torch.from_numpy(inst.positions).cuda()
    out = ops.paged_attention(fmt, pool, q, table, lengths, scale=scale, q_pos=q_pos)
    torch.cuda.synchronize()
    assert out.is_contiguous() and tuple(out.shape) == tuple(q.shape)
    want = oracle_attention(fmt, inst, inst.positions, np.full(w.batch, nq, np.int32), scale)
    assert_attention_close(out.float().cpu().numpy(), want)
    for bad in (torch.empty_like(bqhd).transpose(1, 2),                  # strided
                torch.empty(q.shape, dtype=torch.float16, device="cuda"),  # dtype
                torch.empty((w.batch, w.heads, nq + 1, w.head_dim), dtype=fmt.dtype,
                            device="cuda")):                             # shape
        with pytest.raises(ValueError, match="out must be"):
            ops.paged_attention(fmt, pool, q, table, lengths, scale=scale, q_pos=q_pos, out=bad)


@pytest.mark.parametrize("bits,nq,dtype", [(16, 1, "bfloat16"), (16, 5, "bfloat16"),
                                           (16, 2, "float16"), (8, 1, "bfloat16"),
                                           (4, 3, "bfloat16"),
                                           # two row blocks: V dequantized in registers
                                           (8, 5, "bfloat16"), (4, 6, "bfloat16")])
def test_attention_ignores_stale_bytes_of_reused_pages(bits, nq, dtype):
    """Pages handed out again still hold their last owner's bytes past the new
    sequence's end; here every byte starts as 0xFF (NaN for float pages,
    NaN/-inf-like scales and biases for quantized ones).  Tokens past each
    sequence's end must not reach the output."""
    from pkv import workloads

    w = workloads.get("c2", batch=5, lengths=(1, 7, 16, 33, 250), heads=16, kv_heads=4,
                      bits=bits, num_queries=nq, append_tokens=nq, outlier_fraction=0.0,
                      group_size=64 if bits != 16 else 32)
    inst = workloads.generate(w)
    if dtype == "float16":
        inst.keys = [k.astype(np.float16).astype(np.float32) for k in inst.keys]
        inst.values = [v.astype(np.float16).astype(np.float32) for v in inst.values]
        inst.queries = inst.queries.astype(np.float16).astype(np.float32)
    fmt = _fmt(w, getattr(torch, dtype))
    from pkv import ops

    stale = ops.allocate_pool(fmt, inst.num_pages).fill_(0xFF)
    pool, table, lengths = fill_pages(fmt, inst, chunk=16)
    # move the written tokens onto the stale pool: copy only what fill_pages wrote
    # by appending again into the 0xFF pool
    lengths_h = np.array([k.shape[1] for k in inst.keys])
    for start in range(0, int(lengths_h.max()), 16):
        width = np.clip(lengths_h - start, 0, 16).astype(np.int32)
        k = np.zeros((w.batch, w.kv_heads, 16, w.head_dim), np.float32)
        v = np.zeros_like(k)
        for b in range(w.batch):
            n = int(width[b])
            k[b, :, :n] = inst.keys[b][:, start:start + n]
            v[b, :, :n] = inst.values[b][:, start:start + n]
        ops.append_quantize(fmt, stale, to_torch(k, fmt.dtype), to_torch(v, fmt.dtype), table,
                            torch.full((w.batch,), start, dtype=torch.int32, device="cuda"),
                            torch.from_numpy(width).cuda())
    scale = scale_of(w.head_dim)
    q = to_torch(inst.queries, fmt.dtype)
    q_pos = torch.from_numpy(inst.positions).cuda()
    want = oracle_attention(fmt, inst, inst.positions, np.full(w.batch, nq, np.int32), scale)
    for waves in (0, 3):
        out = ops.paged_attention(fmt, stale, q, table, lengths, scale=scale, q_pos=q_pos,
                                  waves=waves)
        clean = ops.paged_attention(fmt, pool, q, table, lengths, scale=scale, q_pos=q_pos,
                                    waves=waves)
        torch.cuda.synchronize()
        assert torch.equal(out, clean), waves
        assert_attention_close(out.float().cpu().numpy(), want)


MIXED_CASES = {
    # name: (workload overrides); widths per sequence, Q = their maximum
    "c2_c5_int8": dict(name="c5", batch=6, lengths=(300, 40, 1000, 90, 2, 700), num_queries=64,
                       append_tokens=64, widths=(1, 64, 1, 3, 1, 17)),
    "verify_rows_gqa4": dict(name="c5", batch=5, lengths=(130, 500, 64, 9, 333), num_queries=40,
                             append_tokens=40, widths=(5, 40, 8, 1, 9)),
    "gqa8_4bit_p32": dict(name="c5", batch=4, heads=64, lengths=(200, 1000, 50, 77),
                          num_queries=36, append_tokens=36, bits=4, page_tokens=32,
                          widths=(4, 36, 1, 2)),
    "d256_four_queries": dict(name="c5", batch=4, lengths=(90, 300, 17, 128), head_dim=256,
                              group_size=128, num_queries=20, append_tokens=20,
                              widths=(4, 20, 1, 5)),
    "bf16_pages_many_decode": dict(name="c5", batch=70, lengths=(), length_range=(1, 600),
                                   num_queries=48, append_tokens=48, bits=16,
                                   widths=(48, 1, 2, 3, 7) * 14),
    # head_dim 100: the prefill blocks write the decode rows' zeros row by row
    # (rows of 200 bytes are not 16-byte multiples)
    "d100_zero_rows_by_row": dict(name="c5", batch=5, lengths=(60, 400, 20, 9, 250), head_dim=100,
                                  group_size=32, num_queries=40, append_tokens=40,
                                  widths=(1, 40, 2, 1, 33)),
    # every sequence narrow: no prefill row is live, each block zeroes its own rows
    "all_rows_decode_padded": dict(name="c5", batch=4, lengths=(70, 300, 15, 128), num_queries=40,
                                   append_tokens=40, widths=(1, 2, 8, 3)),
}


@pytest.mark.parametrize("case", sorted(MIXED_CASES))
def test_mixed_batch_routes_rows_per_sequence(case):
    """One call over sequences of different widths: the ones the decode kernel
    serves (at most 32 query rows per KV head) go to it, the others to the
    prefill kernel; both against the oracle, padded rows zero.  With no room
    for the decode part's partials, the prefill kernel serves every sequence
    (same result within the bar)."""
    _check_mixed(MIXED_CASES[case])


_MIXED_GROUPS = {64: (32, 64), 128: (32, 64, 128), 256: (32, 64, 128)}


@pytest.mark.parametrize("seed", list(range(16)) + list(range(500, 530)))
def test_mixed_batch_random(seed):
    """Seeded random mixed batches: 4-bit, int8 or bf16 pages, head_dim
    64/128/256, pages of 16-64 tokens, 1-8 query heads per KV head, and per
    sequence a width from 1 token up to a prefill chunk (at least one chunk
    wide enough for the prefill kernel), each checked as the fixed cases are."""
    rng = np.random.default_rng(2000 + seed)
    dim = int(rng.choice(list(_MIXED_GROUPS)))
    bits = int(rng.choice([4, 8, 16]))
    kv = int(rng.choice([1, 2, 4, 8]))
    gqa = int(rng.choice([1, 2, 4, 8]))
    batch = int(rng.integers(2, 9))
    q = int(rng.integers(33 // gqa + 1, 97))
    widths = [int(x) for x in rng.choice([1, 1, 2, 3, 5, 8, 17, q], size=batch)]
    widths[int(rng.integers(0, batch))] = q
    overrides = dict(name="c5", batch=batch, bits=bits, head_dim=dim,
                     group_size=32 if bits == 16 else int(rng.choice(_MIXED_GROUPS[dim])),
                     page_tokens=int(rng.choice([16, 32, 64])), kv_heads=kv, heads=kv * gqa,
                     lengths=tuple(int(x) for x in rng.integers(1, 800, size=batch)),
                     num_queries=q, append_tokens=q, widths=tuple(widths))
    print(f"seed {seed}: {overrides}", flush=True)
    _check_mixed(overrides)


def _check_mixed(overrides):
    from pkv import ops, workloads

    overrides = dict(overrides)
    w = workloads.get(overrides.pop("name"), **overrides)
    inst = workloads.generate(w)
    fmt = _fmt(w)
    pool, table, lengths = fill_pages(fmt, inst, chunk=64)
    scale = scale_of(w.head_dim)
    q = to_torch(inst.queries, fmt.dtype)
    widths = torch.from_numpy(inst.widths).cuda()
    want = oracle_attention(fmt, inst, inst.positions, inst.widths, scale)
    outs = []
    for q_pos in (torch.from_numpy(inst.positions).cuda(), None):
        for waves in (0, 5):
            out = ops.paged_attention(fmt, pool, q, table, lengths, scale=scale, q_pos=q_pos,
                                      widths=widths, waves=waves)
            torch.cuda.synchronize()
            assert_attention_close(out.float().cpu().numpy(), want)
            outs.append(out)
    tiny = torch.empty(256, dtype=torch.uint8, device="cuda")    # no decode part
    alone = ops.paged_attention(fmt, pool, q, table, lengths, scale=scale, widths=widths,
                                workspace=tiny, waves=5)
    torch.cuda.synchronize()
    assert_attention_close(alone.float().cpu().numpy(), want)
    got = outs[0].float().cpu().numpy()
    for b, n in enumerate(inst.widths):
        assert not got[b, :, n:].any(), b


QUERY_SCALE_CASES = {
    # name: workload overrides (quantized pages take the queries as f16 MFMA operands)
    "decode_int8": dict(name="c2", batch=4, length_range=(3, 600)),
    "decode_int4_g32": dict(name="c3", batch=2, lengths=(700, 40), group_size=32),
    "verify_int8_rows20": dict(name="c4", batch=3, length_range=(10, 400), shared_prefix_pages=0),
    "prefill_int8": dict(name="c5", batch=2, lengths=(200, 70), num_queries=64, append_tokens=64),
    # four and eight quantization groups per row (bias parts: 3 and 2 per group)
    "prefill_int4_g32": dict(name="c5", batch=2, lengths=(150, 40), num_queries=48,
                             append_tokens=48, bits=4, group_size=32),
    "prefill_int8_d256_g32": dict(name="c5", batch=2, lengths=(120, 33), num_queries=40,
                                  append_tokens=40, head_dim=256, group_size=32),
}


def _scale_params():
    params = []
    for case in sorted(QUERY_SCALE_CASES):
        for factor in (10.0, 30.0, 300.0, 1e6, 3e-6):
            if factor == 10.0 and not case.startswith("prefill"):
                continue
            params.append(pytest.param(case, factor, id=f"{case}-{factor:g}"))
    return params


@pytest.mark.parametrize("case,factor", _scale_params())
def test_attention_with_large_and_tiny_queries(case, factor):
    """Queries scaled by 30 and 300 (sharp softmax), by 1e6 (bf16 values past the
    f16 range the quantized-page kernels take queries in) and by 3e-6 (f16
    subnormals): the reference dots float queries in f32
    (``engine/paged_attention.py:82-83, 239-240``) and so must this build --
    a row whose largest element passes 2^15 is scaled by a power of two before
    the f16 conversion and the inverse folded into its softmax scale."""
    from pkv import ops, workloads

    overrides = dict(QUERY_SCALE_CASES[case])
    w = workloads.get(overrides.pop("name"), **overrides)
    inst = workloads.generate(w)
    inst.queries = numpy_ref.bf16_round(inst.queries * np.float32(factor))
    assert np.isfinite(inst.queries).all()
    fmt = _fmt(w)
    pool, table, lengths = fill_pages(fmt, inst, chunk=64)
    scale = scale_of(w.head_dim)
    widths = np.full(w.batch, w.num_queries, np.int32)
    q_pos = torch.from_numpy(inst.positions).cuda()
    want = oracle_attention(fmt, inst, inst.positions, widths, scale)
    for waves in (0, 7):
        out = ops.paged_attention(fmt, pool, to_torch(inst.queries, fmt.dtype), table, lengths,
                                  scale=scale, q_pos=q_pos, waves=waves)
        torch.cuda.synchronize()
        assert_attention_close(out.float().cpu().numpy(), want)


def test_attention_padded_query_rows_are_zero():
    from pkv import ops, workloads

    w = workloads.get("c4", batch=3, length_range=(200, 300))
    inst = workloads.generate(w)
    fmt = _fmt(w)
    pool, table, lengths = fill_pages(fmt, inst, chunk=64)
    widths = np.array([5, 2, 1], np.int32)
    positions = inst.positions
    scale = scale_of(w.head_dim)
    out = ops.paged_attention(fmt, pool, to_torch(inst.queries, fmt.dtype), table, lengths,
                              scale=scale, q_pos=torch.from_numpy(positions).cuda(),
                              widths=torch.from_numpy(widths).cuda(), waves=11)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    want = oracle_attention(fmt, inst, positions, widths, scale)
    assert_attention_close(got, want)
    assert np.all(got[1, :, 2:] == 0) and np.all(got[2, :, 1:] == 0)


@pytest.mark.parametrize("positions_given", [True, False])
def test_prefill_ragged_widths(positions_given):
    """Chunks of different widths in one call: rows past a sequence's width are 0.

    Without ``q_pos`` query q of a width-w chunk sits at position L - w + q.
    """
    from pkv import ops, workloads

    w = workloads.get("c5", batch=3, lengths=(120, 40, 300), num_queries=48, append_tokens=48)
    inst = workloads.generate(w)
    fmt = _fmt(w)
    pool, table, lengths = fill_pages(fmt, inst, chunk=64)
    widths = np.array([48, 17, 1], np.int32)
    total = inst.total_lengths
    positions = np.stack([total[b] - widths[b] + np.arange(w.num_queries) for b in range(w.batch)])
    positions = positions.astype(np.int32)
    scale = scale_of(w.head_dim)
    q_pos = torch.from_numpy(positions).cuda() if positions_given else None
    out = ops.paged_attention(fmt, pool, to_torch(inst.queries, fmt.dtype), table, lengths,
                              scale=scale, q_pos=q_pos, widths=torch.from_numpy(widths).cuda())
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    want = oracle_attention(fmt, inst, positions, widths, scale)
    assert_attention_close(got, want)
    assert np.all(got[1, :, 17:] == 0) and np.all(got[2, :, 1:] == 0)


@pytest.mark.parametrize("shape", [dict(), dict(num_queries=5, append_tokens=5), dict(heads=64)],
                         ids=["rows4", "rows20_grouped", "rows8_grouped"])
def test_split_segment_merge_is_deterministic_across_calls_and_graph_replays(shape):
    """Split segments merged by log-sum-exp in a fixed piece order: back-to-back
    calls on one workspace, and replays of a captured graph (attention + merge
    kernels, eager work between replays), each give the eager result bit for bit
    -- also for the grouped runs (LDS combine, barriers) of 8 and 20 rows."""
    from pkv import ops, workloads

    w = workloads.get("c2", batch=6, length_range=(300, 2000), **shape)
    inst = workloads.generate(w)
    fmt = _fmt(w)
    pool, table, lengths = fill_pages(fmt, inst, chunk=128)
    scale = scale_of(w.head_dim)
    q = to_torch(inst.queries, fmt.dtype)
    q_pos = torch.from_numpy(inst.positions).cuda()
    waves = 3 * w.batch * w.kv_heads       # ~3 pieces per segment
    first = ops.paged_attention(fmt, pool, q, table, lengths, scale=scale, q_pos=q_pos, waves=waves)
    second = ops.paged_attention(fmt, pool, q, table, lengths, scale=scale, q_pos=q_pos,
                                 waves=waves)
    torch.cuda.synchronize()
    want = oracle_attention(fmt, inst, inst.positions, np.full(w.batch, w.num_queries, np.int32),
                            scale)
    assert_attention_close(first.float().cpu().numpy(), want)
    assert torch.equal(first, second)

    out = torch.empty_like(first)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        ops.paged_attention(fmt, pool, q, table, lengths, scale=scale, q_pos=q_pos, waves=waves,
                            out=out)                      # warm-up outside the capture
        stream.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            ops.paged_attention(fmt, pool, q, table, lengths, scale=scale, q_pos=q_pos,
                                waves=waves, out=out)
    torch.cuda.current_stream().wait_stream(stream)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, first)
        eager = ops.paged_attention(fmt, pool, q, table, lengths, scale=scale, q_pos=q_pos,
                                    waves=waves)       # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(eager, first)



def _random_attention_cases(count, seed, dims=(64, 128, 128, 100), groups=(32, 64), prefix=""):
    """Seeded random decode/verify cases across the decode kernel's shapes."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        bits = int(rng.choice([4, 8, 8, 16]))
        dim = int(rng.choice(dims))
        group = int(rng.choice(groups)) if bits != 16 else 32
        if bits != 16 and group > dim:
            group = 32
        if bits != 16 and -(-dim // group) * group not in (64, 128, 256):
            group = 32
        page = int(rng.choice([16, 32, 64]))
        kv_heads = int(rng.choice([1, 2, 8]))
        gqa = int(rng.choice([1, 2, 4, 8]))
        nq = int(rng.integers(1, 5))
        while nq * gqa > 32:
            nq -= 1
        batch = int(rng.integers(1, 12))
        lengths = tuple(int(x) for x in rng.choice([1, 2, 15, 16, 17, 31, 64, 65, 129, 300, 777],
                                                   size=batch))
        waves = int(rng.choice([0, 1, 3, 7, 16, 50, 200, 1000]))
        cases.append(dict(bits=bits, head_dim=dim, group_size=group, page_tokens=page,
                          kv_heads=kv_heads, heads=kv_heads * gqa, num_queries=nq,
                          append_tokens=nq, batch=batch, lengths=lengths, waves=waves,
                          seed=int(rng.integers(1 << 30)), index=f"{prefix}{i}"))
    return cases


# A case that once failed by one sequence (4-bit D128 G32 at 16-token pages,
# 4 rows per KV head, sequences of 3 tokens next to longer ones) when masked
# probabilities were taken as exp2(-inf) instead of through selects.
_RANDOM_REGRESSIONS = [
    dict(bits=4, head_dim=128, group_size=32, page_tokens=16, kv_heads=8, heads=16, num_queries=2,
         append_tokens=2, batch=11, lengths=(1, 1, 129, 64, 1, 65, 17, 65, 16, 64, 17), waves=200,
         seed=765951576, index="reg0"),
]


# a second set with head_dim 256 and G128 (head_dim 256 past 16 rows per KV
# head runs on the prefill kernel)
@pytest.mark.parametrize("case", _random_attention_cases(48, seed=2026) + _RANDOM_REGRESSIONS
                         + _random_attention_cases(32, seed=2027, dims=(64, 128, 256, 256),
                                                   groups=(32, 64, 128), prefix="w")
                         + _random_attention_cases(60, seed=4001, prefix="x"),
                         ids=lambda c: f"r{c['index']}")
def test_attention_random_shapes_match_oracle(case):
    """Random layouts (4/8-bit G32/G64 and bf16 pages, D 64-128, pages of
    16-64 tokens), 1-32 rows per KV head, ragged batches of 1-777 tokens and
    1-1000 waves: the split's lead tiles, runs inside a lead, column slots,
    two row blocks and every merge width, against the oracle."""
    from pkv import ops, workloads

    case = dict(case)
    waves = case.pop("waves")
    case.pop("index")
    w = workloads.get("c2", shared_prefix_pages=0, outlier_fraction=0.0, length_range=(),
                      **case)
    inst = workloads.generate(w)
    fmt = _fmt(w)
    pool, table, lengths = fill_pages(fmt, inst, chunk=64)
    widths = np.full(w.batch, w.num_queries, np.int32)
    scale = scale_of(w.head_dim)
    out = ops.paged_attention(fmt, pool, to_torch(inst.queries, fmt.dtype), table, lengths,
                              scale=scale, q_pos=torch.from_numpy(inst.positions).cuda(),
                              waves=waves)
    torch.cuda.synchronize()
    want = oracle_attention(fmt, inst, inst.positions, widths, scale)
    assert_attention_close(out.float().cpu().numpy(), want)


# Grouped runs (5-8 and 17-32 rows per KV head: four waves per run, iterations
# dealt round robin, states combined in LDS at each piece's end): pieces with
# fewer iterations than the group (sequences of 1-40 tokens, many runs), one
# run for everything (waves <= 4), runs ending inside a lead, and long pieces
# next to short ones, at 4/8 bits and on bf16 pages.
_GROUPED = [
    dict(bits=8, head_dim=128, group_size=64, page_tokens=16, kv_heads=8, heads=64, num_queries=1,
         batch=9, lengths=(1, 2, 3, 17, 33, 40, 5, 16, 31), waves=4000),
    dict(bits=4, head_dim=128, group_size=64, page_tokens=32, kv_heads=4, heads=32, num_queries=1,
         batch=3, lengths=(4096, 7, 1500), waves=3),
    dict(bits=8, head_dim=128, group_size=64, page_tokens=16, kv_heads=8, heads=32, num_queries=5,
         batch=6, lengths=(300, 1, 2, 900, 45, 64), waves=64),
    dict(bits=8, head_dim=64, group_size=32, page_tokens=64, kv_heads=2, heads=16, num_queries=4,
         batch=4, lengths=(1, 130, 2049, 16), waves=1),
    dict(bits=4, head_dim=128, group_size=32, page_tokens=16, kv_heads=8, heads=32, num_queries=2,
         batch=5, lengths=(3, 700, 64, 65, 1), waves=37),
    dict(bits=16, head_dim=128, group_size=32, page_tokens=16, kv_heads=8, heads=32, num_queries=7,
         batch=4, lengths=(20, 5, 333, 1024), waves=120),
]


@pytest.mark.parametrize("case", range(len(_GROUPED)))
def test_grouped_runs_match_oracle(case):
    from pkv import ops, workloads

    case = dict(_GROUPED[case])
    waves = case.pop("waves")
    w = workloads.get("c2", shared_prefix_pages=0, outlier_fraction=0.0, length_range=(),
                      append_tokens=case["num_queries"], seed=101 + len(case["lengths"]), **case)
    inst = workloads.generate(w)
    fmt = _fmt(w)
    pool, table, lengths = fill_pages(fmt, inst, chunk=64)
    widths = np.full(w.batch, w.num_queries, np.int32)
    scale = scale_of(w.head_dim)
    out = ops.paged_attention(fmt, pool, to_torch(inst.queries, fmt.dtype), table, lengths,
                              scale=scale, q_pos=torch.from_numpy(inst.positions).cuda(),
                              waves=waves)
    again = ops.paged_attention(fmt, pool, to_torch(inst.queries, fmt.dtype), table, lengths,
                                scale=scale, q_pos=torch.from_numpy(inst.positions).cuda(),
                                waves=waves)
    torch.cuda.synchronize()
    assert torch.equal(out, again), "grouped runs are not deterministic"
    want = oracle_attention(fmt, inst, inst.positions, widths, scale)
    assert_attention_close(out.float().cpu().numpy(), want)
