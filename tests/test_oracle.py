"""CPU: pin the oracle before trusting it.

Every oracle function is checked against something that does not restate it:
golden vectors written by the reference's own ``quantize_page``, numpy's IEEE
float16 cast, torch's bfloat16 cast, closed forms (one visible token returns
V, identical keys return mean(V)), an independent per-token online-softmax
loop (the reference kernel's own formulation), and the reference's own
partition-merge test (``tests/test_paged_hybrid.py:574-634``).
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest

from oracle import cport, numpy_ref

GOLDEN_PATH = Path(__file__).parent / "golden" / "quantize_page_g32.npz"
GOLDEN = np.load(GOLDEN_PATH)
CASES = sorted({k.split("/")[0] for k in GOLDEN.files})


def _bits16(a):
    return np.asarray(a, np.float16).view(np.uint16)


# ------------------------------------------------------------ formats


def test_f16_conversion_is_ieee_round_to_nearest_even():
    """pkvo_f32_to_f16 against numpy's float16 cast on boundary and tie patterns."""
    lib = cport.load()
    halves = np.arange(0, 0x7C00, dtype=np.uint32)      # every finite positive f16
    f = halves.astype(np.uint16).view(np.float16).astype(np.float32)
    nxt = (halves + 1).astype(np.uint16).view(np.float16).astype(np.float32)
    mid = ((f.astype(np.float64) + nxt.astype(np.float64)) / 2).astype(np.float32)  # exact ties
    rng = np.random.default_rng(3)
    samples = np.concatenate([f, mid, np.nextafter(mid, np.float32(np.inf)),
                              np.nextafter(mid, np.float32(0)),
                              rng.uniform(-70000, 70000, 20000).astype(np.float32),
                              (rng.standard_normal(20000) * 1e-6).astype(np.float32),
                              np.float32([65504, 65519.996, 65520, 1e9, 5.96e-8, 2.98e-8, 1e-6])])
    samples = samples[::7] if samples.size > 120000 else samples
    samples = np.concatenate([samples, -samples])
    with np.errstate(over="ignore"):
        want = samples.astype(np.float16).view(np.uint16)
    got = np.array([lib.pkvo_f32_to_f16(float(x)) for x in samples], np.uint16)
    assert np.array_equal(got, want)
    back = np.array([lib.pkvo_f16_to_f32(int(h)) for h in want[::13]], np.float32)
    assert np.array_equal(back, want[::13].view(np.float16).astype(np.float32))


def test_bf16_round_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(4)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 100,
                        # exact ties: low half 0x8000 with even and odd kept bits
                        (np.arange(5000, dtype=np.uint32) << 16 | 0x8000).view(np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(numpy_ref.bf16_round(x), want)


# ------------------------------------------------------------ quantizer


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("bits", [4, 8])
def test_quantizer_matches_reference_golden(case, bits):
    """numpy and C restatements vs vectors the reference's quantize_page wrote."""
    x = GOLDEN[f"{case}/input"]
    for codes, scale, bias in (numpy_ref.quantize_page(x, bits, 32),
                               cport.quantize_rows(x.astype(np.float32), bits, 32)):
        assert np.array_equal(codes, GOLDEN[f"{case}/b{bits}/codes"])
        assert np.array_equal(_bits16(scale), _bits16(GOLDEN[f"{case}/b{bits}/scale"]))
        assert np.array_equal(_bits16(bias), _bits16(GOLDEN[f"{case}/b{bits}/bias"]))
    restored = numpy_ref.dequantize_page(numpy_ref.quantize_page(x, bits, 32), bits, x.shape[-1])
    assert np.array_equal(restored, GOLDEN[f"{case}/b{bits}/dequant"])


def test_golden_inputs_are_the_generator_inputs():
    """The committed fixture still holds what tests/golden/make_golden.py draws."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden",
                                                  Path(__file__).parent / "golden" / "make_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    for name, value in mod.cases().items():
        assert np.array_equal(np.asarray(GOLDEN[f"{name}/input"]), value), name


@pytest.mark.parametrize("bits", [4, 8])
def test_quantizer_reference_round_trip_tolerance(bits):
    """The reference's own bar (test_paged_hybrid.py:191-199): atol .02 (8-bit) / .24 (4-bit)."""
    values = np.random.default_rng(12).normal(size=(1, 2, 16, 37)).astype(np.float16)
    packed = numpy_ref.quantize_page(values, bits)
    restored = numpy_ref.dequantize_page(packed, bits, 37)
    np.testing.assert_allclose(restored, values, atol=.24 if bits == 4 else .02, rtol=.02)
    assert sum(v.nbytes for v in packed) < values.nbytes


@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("bits", [4, 8])
def test_quantizer_invariants(group, bits):
    rng = np.random.default_rng(group * bits)
    x = numpy_ref.bf16_round(rng.standard_normal((64, 256)).astype(np.float32) * 3)
    codes, scale, bias = numpy_ref.quantize_page(x, bits, group)
    if bits == 4:
        unpacked = np.stack((codes & 15, codes >> 4), -1).reshape(64, 256)
    else:
        unpacked = codes
    assert unpacked.max() <= (1 << bits) - 1
    restored = numpy_ref.dequantize_page((codes, scale, bias), bits, 256, group)
    s = np.repeat(scale.astype(np.float32), group, -1)
    # half a step, plus the f16 rounding of bias and the scale's rounding over 2^b - 1 steps
    bound = s / 2 + np.abs(x) * 2e-3 + np.repeat(np.abs(bias.astype(np.float32)), group, -1) * 1e-3
    assert np.all(np.abs(restored - x) <= bound)
    # the minimum of every group maps near code 0
    assert np.all(unpacked.reshape(64, -1, group).min(-1) <= 1)


def test_quantizer_special_cases():
    # constant group: code 0, bias = f16(x), scale clamps to f16(1e-6) (a subnormal)
    x = np.full((1, 32), 3.25, np.float32)
    codes, scale, bias = numpy_ref.quantize_page(x, 8, 32)
    assert np.all(codes == 0) and bias[0, 0] == np.float16(3.25)
    assert _bits16(scale)[0, 0] == _bits16(np.float16(1e-6))
    # exact .5 ties round half to even
    row = np.zeros((1, 32), np.float32)
    row[0, :6] = [0, 255, 0.5, 1.5, 2.5, 3.5]
    codes, scale, _ = numpy_ref.quantize_page(row, 8, 32)
    assert scale[0, 0] == 1 and list(codes[0, :6]) == [0, 255, 0, 2, 2, 4]
    # 4-bit packs the even element in the low nibble
    row = np.zeros((1, 32), np.float32)
    row[0, :2] = [15, 0]
    row[0, 2] = 15
    codes, _, _ = numpy_ref.quantize_page(row, 4, 32)
    assert codes[0, 0] == 15 and codes[0, 1] == 15


@pytest.mark.parametrize("group", [64, 128])
@pytest.mark.parametrize("bits", [4, 8])
def test_wide_groups_reduce_to_golden_g32(group, bits):
    """Groups of G built from copies of one 32-wide golden group quantize like it.

    min/max of the copies equal the original's, so codes repeat the G=32
    codes and the scale and bias equal the G=32 ones: G in {64, 128} is pinned
    to the reference's own group-32 output.
    """
    x = GOLDEN["bf16_d128_outliers/input"].reshape(-1, 128)[:, :32]   # rows of one group
    wide = np.tile(x, (1, group // 32))
    codes, scale, bias = numpy_ref.quantize_page(wide, bits, group)
    ref_codes = GOLDEN[f"bf16_d128_outliers/b{bits}/codes"].reshape(x.shape[0], -1)
    per_group = 32 * bits // 8
    assert np.array_equal(codes, np.tile(ref_codes[:, :per_group], (1, group // 32)))
    assert np.array_equal(_bits16(scale[:, 0]),
                          _bits16(GOLDEN[f"bf16_d128_outliers/b{bits}/scale"].reshape(x.shape[0], -1)[:, 0]))
    assert np.array_equal(_bits16(bias[:, 0]),
                          _bits16(GOLDEN[f"bf16_d128_outliers/b{bits}/bias"].reshape(x.shape[0], -1)[:, 0]))
    c_codes, c_scale, c_bias = cport.quantize_rows(wide, bits, group)
    assert np.array_equal(c_codes, codes) and np.array_equal(_bits16(c_scale), _bits16(scale))


# ------------------------------------------------------------ attention


def _random_case(rng, batch=2, heads=4, hk=2, q=3, dim=8, lengths=(9, 23)):
    queries = rng.standard_normal((batch, heads, q, dim)).astype(np.float32)
    keys = [rng.standard_normal((hk, n, dim)).astype(np.float32) for n in lengths]
    values = [rng.standard_normal((hk, n, dim)).astype(np.float32) for n in lengths]
    positions = np.stack([np.arange(n - q, n) for n in lengths])
    return queries, keys, values, positions


def test_attention_matches_online_softmax_loop():
    rng = np.random.default_rng(5)
    q, k, v, pos = _random_case(rng)
    widths = (3, 2)
    a = numpy_ref.paged_attention(q, k, v, pos, widths, scale=.4)
    b = numpy_ref.online_softmax_attention(q, k, v, pos, widths, scale=.4)
    np.testing.assert_allclose(a, b, atol=1e-12)
    assert np.all(a[1, :, 2:] == 0)


def test_attention_closed_forms():
    rng = np.random.default_rng(6)
    q, k, v, pos = _random_case(rng, batch=1, lengths=(12,))
    # one visible token: output is that token's V
    out = numpy_ref.paged_attention(q, k, v, np.array([[0, 0, 0]]), (3,), scale=.7)
    for h in range(4):
        np.testing.assert_allclose(out[0, h], np.repeat(v[0][h // 2, :1], 3, 0), atol=1e-6)
    # identical keys: uniform weights, output is the mean of the visible values
    same = [np.repeat(k[0][:, :1], 12, 1)]
    out = numpy_ref.paged_attention(q, same, v, pos, (3,), scale=.7)
    for qi, p in enumerate(pos[0]):
        np.testing.assert_allclose(out[0, 0, qi], v[0][0, :p + 1].mean(0), atol=1e-6)


def test_c_oracle_attention_matches_numpy_oracle():
    from pkv import workloads
    from paged_case import oracle_attention

    class Fmt:
        def __init__(self, w):
            self.num_kv_heads, self.page_tokens, self.head_dim = w.kv_heads, w.page_tokens, w.head_dim
            self.bits, self.group_size, self.quantized = w.bits, w.group_size, w.bits != 16

        @property
        def reference_dim(self):
            return numpy_ref.padded_dim(self.head_dim, self.group_size) if self.quantized \
                else self.head_dim

    for name, over in (("c1", {}), ("c2", dict(batch=3, length_range=(1, 200))),
                       ("c3", dict(batch=2, lengths=(100, 300))),
                       ("c4", dict(batch=3, length_range=(260, 330))),
                       ("c2", dict(batch=2, length_range=(20, 50), head_dim=37, group_size=32))):
        w = workloads.get(name, **over)
        inst = workloads.generate(w)
        f = Fmt(w)
        pos = inst.positions
        wid = np.full(w.batch, w.num_queries, np.int32)
        a = oracle_attention(f, inst, pos, wid, .1, use_c=True)
        b = oracle_attention(f, inst, pos, wid, .1, use_c=False)
        np.testing.assert_allclose(a, b, atol=2e-5)


def test_partition_merge_matches_dense_reference_test_shape():
    """The reference's merger test (test_paged_hybrid.py:574-634) on the LSE restatement.

    Lengths (259, 37), P=16, 16-page launch chunks (256 tokens), H=2, HK=1,
    D=4, Q=3 with widths (3, 1), positions ((256,257,258), (36,37,38)),
    scale .5, atol/rtol .002; padded query rows are zero.
    """
    rng = np.random.default_rng(12)
    keys, values = [], []
    for length in (259, 37):
        keys.append(rng.normal(size=(1, length, 4)).astype(np.float16).astype(np.float32))
        values.append(rng.normal(size=(1, length, 4)).astype(np.float16).astype(np.float32))
    query = rng.normal(size=(2, 2, 3, 4)).astype(np.float16).astype(np.float32)
    positions = ((256, 257, 258), (36, 37, 38))
    widths = (3, 1)
    parts = numpy_ref.partition_partials(query, keys, values, positions, widths, scale=.5,
                                         split=256)
    assert len(parts) == 2
    merged = numpy_ref.lse_merge(parts)
    dense = numpy_ref.paged_attention(query, keys, values, positions, widths, scale=.5)
    np.testing.assert_allclose(merged, dense, atol=.002, rtol=.002)
    assert np.all(merged[1, :, 1:] == 0)


@pytest.mark.parametrize("split", [1, 5, 16, 64])
def test_partition_merge_any_split(split):
    rng = np.random.default_rng(split)
    q, k, v, pos = _random_case(rng, lengths=(70, 33))
    widths = (3, 3)
    merged = numpy_ref.lse_merge(numpy_ref.partition_partials(q, k, v, pos, widths, scale=.3,
                                                              split=split))
    dense = numpy_ref.paged_attention(q, k, v, pos, widths, scale=.3)
    np.testing.assert_allclose(merged, dense, atol=1e-10)


def test_ref_pages_tail_modes_differ_only_in_the_tail():
    """Float-tail (reference) and quantize-on-append pages hold the same full pages."""
    rng = np.random.default_rng(8)
    k = numpy_ref.bf16_round(rng.standard_normal((2, 37, 64)).astype(np.float32))
    v = numpy_ref.bf16_round(rng.standard_normal((2, 37, 64)).astype(np.float32))
    a = numpy_ref.RefPages(2, 64, 16, bits=8, group_size=64, tail="float")
    b = numpy_ref.RefPages(2, 64, 16, bits=8, group_size=64, tail="quantized")
    for p in (a, b):
        p.write_sequence([4, 1, 7], k, v)
    ka, _ = a.gather([4, 1, 7], 37)
    kb, _ = b.gather([4, 1, 7], 37)
    assert np.array_equal(ka[:, :32], kb[:, :32])
    assert np.array_equal(ka[:, 32:], k[:, 32:])          # float tail is the input
    assert not np.array_equal(kb[:, 32:], k[:, 32:])      # quantized tail is not
    assert np.abs(kb[:, 32:] - k[:, 32:]).max() < 0.05
