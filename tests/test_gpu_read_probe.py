"""GPU: ``pkv_read_probe``, the streaming-read bandwidth reference of the bench.

Its result is a fold of every byte it was given to read: lane l of wave w XORs
the 16-byte units u = l (mod 64) of the pages of its run, and the four words of
each unit, so the output pins which bytes were read (every byte of each listed
page, no other) whatever the wave count.
"""

from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _fold(pool, ids, waves):
    pages = pool.reshape(pool.shape[0], -1, 4)               # [pages, units, 4] uint32
    words = np.bitwise_xor.reduce(pages, axis=2)               # [pages, units]
    out = np.zeros((waves, 64), np.uint32)
    n = len(ids)
    for w in range(waves):
        for p in ids[w * n // waves:(w + 1) * n // waves]:
            if 0 <= p < pool.shape[0]:
                for lane in range(64):
                    out[w, lane] ^= np.bitwise_xor.reduce(words[p, lane::64])
    return out.reshape(-1)


@pytest.mark.parametrize("waves,count", [(1, 5), (7, 30), (64, 40)])
def test_read_probe_reads_every_listed_byte(waves, count):
    from pkv import _native, ops

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    lib = _native.load()
    fmt = ops.PageFormat(8, 128, 16, 8, 64, torch.bfloat16)
    rng = np.random.default_rng(waves)
    pool = torch.from_numpy(rng.integers(0, 256, (24, fmt.page_bytes), dtype=np.uint8)).cuda()
    ids = rng.integers(-2, 26, count).astype(np.int32)        # a few ids outside the pool
    ids_dev = torch.from_numpy(ids).cuda()
    out = torch.zeros(waves * 64, dtype=torch.int32, device="cuda")
    code = lib.pkv_read_probe(_native.stream_handle(pool.device), fmt.c_layout, pool.data_ptr(),
                              pool.shape[0], ids_dev.data_ptr(), count, waves, out.data_ptr())
    assert code == 0
    torch.cuda.synchronize()
    want = _fold(pool.cpu().numpy().view(np.uint32), ids, waves)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want)
