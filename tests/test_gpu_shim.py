"""GPU: the reference-named classes end to end (PagedKVCache, PagedBatchCache, arena).

Restates the reference's direct-page test (``tests/test_paged_hybrid.py:141-167``:
page widths 16/32/64/128, ragged prompts, three decode steps) and its
clone / shared-page tests (:214-225) against the CPU oracle, through libpkv.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import numpy_ref
from paged_case import assert_attention_close

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from pkv import _native

    _native.load()


def _bf16(rng, shape):
    return numpy_ref.bf16_round(rng.standard_normal(shape).astype(np.float32))


def _seen(history, bits, group):
    """What the attention reads for a token history: quantize-on-append values."""
    if bits is None:
        return history
    return numpy_ref.dequantize_page(numpy_ref.quantize_page(history, bits, group), bits,
                                     history.shape[-1], group)


class Mirror:
    """Host copy of every appended token, to build the oracle's inputs."""

    def __init__(self, batch, hk, dim):
        self.k = [np.zeros((hk, 0, dim), np.float32) for _ in range(batch)]
        self.v = [np.zeros((hk, 0, dim), np.float32) for _ in range(batch)]

    def add(self, b, k, v):
        self.k[b] = np.concatenate([self.k[b], k], 1)
        self.v[b] = np.concatenate([self.v[b], v], 1)


@pytest.mark.parametrize("page", [16, 32, 64, 128])
@pytest.mark.parametrize("bits", [None, 8, 4])
def test_ragged_prefill_then_decode_matches_oracle(page, bits):
    from pkv.arena import SegmentedPageArena
    from pkv.paged import PagedBatchCache, PagedKVCache

    rng = np.random.default_rng(page + (bits or 0))
    H, HK, D, G = 8, 2, 128, 64
    arena = SegmentedPageArena(2**40, block_tokens=page)
    rows = [PagedKVCache(arena, dtype="bfloat16", bits=bits, group_size=G) for _ in range(3)]
    mirror = Mirror(3, HK, D)
    metrics = {}
    schedule = [(page + 1, 3, 37)] + [(1, 1, 1)] * 3        # ragged prefill, then decode
    for widths in schedule:
        q_len = max(widths)
        q = _bf16(rng, (3, H, q_len, D))
        k = _bf16(rng, (3, HK, q_len, D))
        v = _bf16(rng, (3, HK, q_len, D))
        before = [r.offset for r in rows]
        out = PagedBatchCache(rows, widths, metrics).attend(
            torch.from_numpy(q).cuda().bfloat16(), torch.from_numpy(k).cuda().bfloat16(),
            torch.from_numpy(v).cuda().bfloat16(), scale=D ** -0.5, position_ids=None)
        torch.cuda.synchronize()
        for b, w in enumerate(widths):
            mirror.add(b, k[b, :, :w], v[b, :, :w])
        positions = [list(range(o, o + q_len)) for o in before]
        keys = [_seen(x, bits, G) for x in mirror.k]
        values = [_seen(x, bits, G) for x in mirror.v]
        want = numpy_ref.paged_attention(q, keys, values, positions, widths, scale=D ** -0.5)
        assert_attention_close(out.float().cpu().numpy(), want)
        assert [r.offset for r in rows] == [o + w for o, w in zip(before, widths)]
    assert metrics["direct_attention_calls"] == len(schedule)
    for r in rows:
        r.page_table.validate(r._blocks)
        r.reset()
    assert arena.stats()["block_live"] == 0


def test_clone_copies_the_tail_and_shares_sealed_pages():
    from pkv.arena import SegmentedPageArena
    from pkv.paged import PagedKVCache
    from pkv.paged_attention import paged_attention

    rng = np.random.default_rng(1)
    arena = SegmentedPageArena(2**40, block_tokens=16)
    cache = PagedKVCache(arena, dtype="bfloat16", bits=8, group_size=64)
    k, v = _bf16(rng, (1, 2, 21, 128)), _bf16(rng, (1, 2, 21, 128))
    cache.append(torch.from_numpy(k).cuda().bfloat16(), torch.from_numpy(v).cuda().bfloat16())
    branch = cache.clone()
    assert branch._blocks[0].block_id == cache._blocks[0].block_id           # shared sealed page
    assert branch._blocks[-1].block_id != cache._blocks[-1].block_id         # copied tail
    k2, v2 = _bf16(rng, (1, 2, 3, 128)), _bf16(rng, (1, 2, 3, 128))
    branch.append(torch.from_numpy(k2).cuda().bfloat16(), torch.from_numpy(v2).cuda().bfloat16())
    q = _bf16(rng, (1, 8, 1, 128))
    qt = torch.from_numpy(q).cuda().bfloat16()
    for c, keys, values in ((cache, k[0], v[0]),
                            (branch, np.concatenate([k[0], k2[0]], 1), np.concatenate([v[0], v2[0]], 1))):
        n = keys.shape[1]
        out = paged_attention(qt, [c], [(n - 1,)], (1,), scale=0.1)
        torch.cuda.synchronize()
        want = numpy_ref.paged_attention(q, [_seen(keys, 8, 64)], [_seen(values, 8, 64)],
                                         [[n - 1]], [1], scale=0.1)
        assert_attention_close(out.float().cpu().numpy(), want)
    branch.reset()
    cache.reset()


def test_shared_prefix_pages_adopted_by_many_sequences():
    from pkv.arena import SegmentedPageArena
    from pkv.paged import PagedBatchCache, PagedKVCache

    rng = np.random.default_rng(2)
    arena = SegmentedPageArena(2**40, block_tokens=16)
    prefix = PagedKVCache(arena, dtype="bfloat16", bits=8, group_size=64)
    pk, pv = _bf16(rng, (1, 2, 64, 128)), _bf16(rng, (1, 2, 64, 128))
    prefix.append(torch.from_numpy(pk).cuda().bfloat16(), torch.from_numpy(pv).cuda().bfloat16())
    rows = []
    for _ in range(4):
        row = PagedKVCache(arena, dtype="bfloat16", bits=8, group_size=64)
        row.adopt([r.fork() for r in prefix._blocks])
        rows.append(row)
    assert prefix._blocks[0].block.references == 5
    mirror = Mirror(4, 2, 128)
    for b in range(4):
        mirror.add(b, pk[0], pv[0])
    widths = (5, 5, 2, 1)                                     # verify-style drafts
    q, k, v = _bf16(rng, (4, 8, 5, 128)), _bf16(rng, (4, 2, 5, 128)), _bf16(rng, (4, 2, 5, 128))
    out = PagedBatchCache(rows, widths, {}).attend(
        torch.from_numpy(q).cuda().bfloat16(), torch.from_numpy(k).cuda().bfloat16(),
        torch.from_numpy(v).cuda().bfloat16(), scale=0.09, position_ids=None)
    torch.cuda.synchronize()
    for b, w in enumerate(widths):
        mirror.add(b, k[b, :, :w], v[b, :, :w])
    want = numpy_ref.paged_attention(q, [_seen(x, 8, 64) for x in mirror.k],
                                     [_seen(x, 8, 64) for x in mirror.v],
                                     [list(range(64, 69))] * 4, widths, scale=0.09)
    got = out.float().cpu().numpy()
    assert_attention_close(got, want)
    assert np.all(got[2, :, 2:] == 0) and np.all(got[3, :, 1:] == 0)
    for r in rows + [prefix]:
        r.reset()


def test_position_ids_are_checked():
    from pkv.arena import SegmentedPageArena
    from pkv.paged import PagedBatchCache, PagedKVCache

    arena = SegmentedPageArena(2**40, block_tokens=16)
    rows = [PagedKVCache(arena, dtype="bfloat16", bits=8, group_size=64)]
    z = torch.zeros((1, 8, 2, 128), dtype=torch.bfloat16, device="cuda")
    kv = torch.zeros((1, 2, 2, 128), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="positions"):
        PagedBatchCache(rows, (2,), {}).attend(z, kv, kv, scale=.1,
                                               position_ids=torch.tensor([[1, 2]]))


@pytest.mark.parametrize("bits", [4, 8])
def test_quantize_page_matches_oracle(bits):
    from pkv.paged import dequantize_page, quantize_page

    rng = np.random.default_rng(bits)
    x = numpy_ref.bf16_round(rng.standard_normal((1, 8, 16, 128)).astype(np.float32) * 3)
    codes, scale, bias = quantize_page(torch.from_numpy(x).cuda().bfloat16(), bits, 64)
    want = numpy_ref.quantize_page(x, bits, 64)
    assert np.array_equal(codes.cpu().numpy(), want[0])
    assert np.array_equal(scale.cpu().numpy().view(np.uint16), want[1].view(np.uint16))
    assert np.array_equal(bias.cpu().numpy().view(np.uint16), want[2].view(np.uint16))
    back = dequantize_page((codes, scale, bias), bits, 128, 64)
    assert np.array_equal(back.cpu().numpy(), numpy_ref.dequantize_page(want, bits, 128, 64))
