"""GPU: ``pkv_paged_attention_noalloc`` (split-K partials in the library's fixed
device array, no workspace argument) against ``pkv_paged_attention`` (caller
workspace), both called through the C ABI.

With the same wave count both make the same split and the same merge, so the
outputs must agree bit for bit; two calls in a row, the second on a smaller
batch (the array keeps the first call's partials, which the second must not
read).  The library default (waves <= 0) is checked against the oracle, an
explicit wave count whose partials exceed the array is refused.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest

from paged_case import assert_attention_close, fill_pages, oracle_attention, to_torch

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from pkv import _native

    _native.load()


def _case(name, **kw):
    from pkv import ops, workloads

    w = workloads.get(name, **kw)
    inst = workloads.generate(w)
    fmt = ops.PageFormat(w.kv_heads, w.head_dim, w.page_tokens, w.bits, w.group_size,
                         torch.bfloat16)
    pool, table, lengths = fill_pages(fmt, inst, chunk=128)
    q = to_torch(inst.queries, fmt.dtype)
    q_pos = torch.from_numpy(inst.positions).cuda()
    return w, inst, fmt, pool, table, lengths, q, q_pos


def _call(noalloc, w, fmt, pool, table, lengths, q, q_pos, waves):
    from pkv import _native as nat
    from pkv import ops

    lib = nat.load()
    out = torch.empty_like(q)
    stream = nat.stream_handle(q.device)
    scale = 1.0 / math.sqrt(w.head_dim)
    common = (stream, ctypes.byref(fmt.c_layout), nat.ptr(pool), pool.shape[0], nat.ptr(q),
              w.batch, w.heads, w.num_queries, nat.ptr(table), table.shape[1], nat.ptr(lengths),
              nat.ptr(q_pos), None, scale, waves)
    if noalloc:
        code = lib.pkv_paged_attention_noalloc(*common, nat.ptr(out))
    else:
        ws = torch.empty(max(256, ops.workspace_bytes(fmt, w.heads, w.num_queries, waves)),
                         dtype=torch.uint8, device=q.device)
        code = lib.pkv_paged_attention(*common, nat.ptr(ws), ws.numel(), nat.ptr(out))
    return code, out


@pytest.mark.parametrize("name,big,small,waves", [
    ("c2", dict(batch=12, length_range=(200, 3000)), dict(batch=3, length_range=(20, 400)), 96),
    ("c4", dict(batch=6, length_range=(300, 1500), shared_prefix_pages=0),
     dict(batch=2, length_range=(40, 300), shared_prefix_pages=0), 40),
    ("c3", dict(batch=2, lengths=(3000, 1700)), dict(batch=1, lengths=(600,)), 64),
])
def test_noalloc_equals_the_workspace_entry_point_twice_in_a_row(name, big, small, waves):
    for kw in (big, small):                      # the second call is smaller
        w, inst, fmt, pool, table, lengths, q, q_pos = _case(name, **kw)
        code_a, a = _call(True, w, fmt, pool, table, lengths, q, q_pos, waves)
        code_b, b = _call(False, w, fmt, pool, table, lengths, q, q_pos, waves)
        torch.cuda.synchronize()
        assert code_a == 0 and code_b == 0
        assert torch.equal(a, b), (name, kw)
        want = oracle_attention(fmt, inst, inst.positions,
                                np.full(w.batch, w.num_queries, np.int32),
                                1.0 / math.sqrt(w.head_dim))
        assert_attention_close(a.float().cpu().numpy(), want)


def test_noalloc_default_waves_and_refused_sizes():
    from pkv import _native as nat

    w, inst, fmt, pool, table, lengths, q, q_pos = _case("c2", batch=5,
                                                         length_range=(100, 2000))
    code, out = _call(True, w, fmt, pool, table, lengths, q, q_pos, 0)     # library default
    torch.cuda.synchronize()
    assert code == 0
    want = oracle_attention(fmt, inst, inst.positions, np.ones(w.batch, np.int32),
                            1.0 / math.sqrt(w.head_dim))
    assert_attention_close(out.float().cpu().numpy(), want)
    # 2 partial slots x waves x 4 rows x (128 + 2) floats: 9000 waves need ~37 MB
    code, _ = _call(True, w, fmt, pool, table, lengths, q, q_pos, 9000)
    assert code == nat.PKV_OUT_OF_MEMORY
    assert "noalloc" in nat.last_error() and "scratch" in nat.last_error()
    code, again = _call(True, w, fmt, pool, table, lengths, q, q_pos, 0)   # still usable
    torch.cuda.synchronize()
    assert code == 0 and torch.equal(again, out)


def test_noalloc_plain_prefill_needs_no_scratch_at_any_wave_count():
    """A wide call without per-sequence widths runs the prefill kernel alone,
    which takes no split-K scratch: an explicit wave count whose decode
    partials would pass the fixed array is not refused, and the output equals
    the workspace entry point's (given a 256-byte workspace it never uses)."""
    from pkv import _native as nat

    w, inst, fmt, pool, table, lengths, q, q_pos = _case("c5", batch=2, lengths=(300, 90),
                                                         num_queries=48, append_tokens=48)
    waves = 100000                     # decode partials for these rows: ~3 GB
    lib = nat.load()
    stream = nat.stream_handle(q.device)
    scale = 1.0 / math.sqrt(w.head_dim)
    common = (stream, ctypes.byref(fmt.c_layout), nat.ptr(pool), pool.shape[0], nat.ptr(q),
              w.batch, w.heads, w.num_queries, nat.ptr(table), table.shape[1], nat.ptr(lengths),
              nat.ptr(q_pos), None, scale, waves)
    a, b = torch.empty_like(q), torch.empty_like(q)
    assert lib.pkv_paged_attention_noalloc(*common, nat.ptr(a)) == 0, nat.last_error()
    ws = torch.empty(256, dtype=torch.uint8, device=q.device)
    assert lib.pkv_paged_attention(*common, nat.ptr(ws), ws.numel(), nat.ptr(b)) == 0
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    want = oracle_attention(fmt, inst, inst.positions, np.full(w.batch, w.num_queries, np.int32),
                            scale)
    assert_attention_close(a.float().cpu().numpy(), want)
