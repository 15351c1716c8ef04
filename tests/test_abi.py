"""CPU: libpkv.so loads, exports every symbol include/pkv.h declares, validates inputs.

Only host-side paths run here (layout arithmetic and argument validation return
before any HIP call); the kernels are exercised by the ``gpu`` tests.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from pkv import _native as nat

HEADER = Path(__file__).resolve().parents[1] / "include" / "pkv.h"
FAKE = ctypes.c_void_p(4096)   # never dereferenced: validation fails or returns first


def declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pkv_[a-z_]+)\s*\(", text)))


def test_header_declarations_are_exported_and_bound():
    lib = nat.load()
    names = declared()
    assert len(names) >= 11
    for name in names:
        assert hasattr(lib, name), f"{name} declared in pkv.h but not exported"
    assert set(names) == set(nat.SIGNATURES), "ctypes bindings differ from the header"


def test_version_and_error_text():
    lib = nat.load()
    assert lib.pkv_version() >= 1
    assert isinstance(nat.last_error(), str)


def _layout(**kw):
    base = dict(num_kv_heads=8, head_dim=128, page_tokens=16, bits=8, group_size=64, float_kind=0)
    base.update(kw)
    return nat.Layout(*base.values())


@pytest.mark.parametrize("kw,page_bytes,dim", [
    ({}, 8 * (2 * 16 * 128 + 2 * 16 * 2 * 4), 128),                          # C2 page: 34 KiB
    (dict(num_kv_heads=4, page_tokens=32, bits=4), 4 * (2 * 32 * 64 + 2 * 32 * 2 * 4), 128),  # C3
    (dict(num_kv_heads=2, head_dim=64, bits=16, group_size=32), 2 * 2 * 16 * 64 * 2, 64),      # C1
    (dict(head_dim=37, group_size=32), 8 * (2 * 16 * 64 + 2 * 16 * 2 * 4), 64),  # padded head dim
    (dict(head_dim=256, group_size=128), 8 * (2 * 16 * 256 + 2 * 16 * 2 * 4), 256),
])
def test_page_geometry(kw, page_bytes, dim):
    lib = nat.load()
    layout = _layout(**kw)
    assert lib.pkv_page_bytes(layout) == page_bytes
    assert lib.pkv_stored_dim(layout) == dim


@pytest.mark.parametrize("kw", [dict(bits=5), dict(head_dim=0), dict(head_dim=300),
                                dict(page_tokens=24), dict(page_tokens=8), dict(group_size=16),
                                dict(float_kind=2), dict(num_kv_heads=0)])
def test_invalid_layouts_are_rejected(kw):
    lib = nat.load()
    assert lib.pkv_page_bytes(_layout(**kw)) < 0
    assert lib.pkv_stored_dim(_layout(**kw)) < 0


def test_workspace_size():
    lib = nat.load()
    # 2 slots per wave x 100 waves x 4 rows x (128 + 2) floats
    need = lib.pkv_attention_workspace_bytes(_layout(), 32, 1, 100)
    assert need >= 2 * 100 * 4 * (128 + 2) * 4
    assert lib.pkv_attention_workspace_bytes(_layout(), 32, 1, 0) < 0     # no waves
    assert lib.pkv_attention_workspace_bytes(_layout(), 30, 1, 10) < 0    # not GQA groups
    # query blocks past the decode kernel's 32 rows per KV head run on the
    # prefill kernel, except a mixed batch's sequences of at most 8 queries
    # (32 rows at GQA 4): partials for those only
    assert lib.pkv_attention_workspace_bytes(_layout(), 32, 9, 10) == \
        lib.pkv_attention_workspace_bytes(_layout(), 32, 8, 10)
    assert lib.pkv_attention_workspace_bytes(_layout(), 32, 512, 10) == \
        lib.pkv_attention_workspace_bytes(_layout(), 32, 8, 10)
    # head_dim 256: 16 rows, 4 queries at GQA 4; none at GQA 32
    assert lib.pkv_attention_workspace_bytes(_layout(head_dim=256, group_size=128), 32, 64, 10) \
        == lib.pkv_attention_workspace_bytes(_layout(head_dim=256, group_size=128), 32, 4, 10)
    assert lib.pkv_attention_workspace_bytes(_layout(head_dim=256, group_size=128), 256, 1,
                                             10) == 0
    assert lib.pkv_attention_waves(_layout(), 32, 512) == 1
    assert lib.pkv_attention_waves(_layout(head_dim=256), 32, 5) == 1     # 20 rows at D=256
    assert lib.pkv_attention_workspace_bytes(_layout(), 32, 1 << 23, 10) < 0


def _parts(runs, rows, dp=128):
    slots = 2 * runs
    return -(-(slots * rows * 2 * 4) // 256) * 256 + slots * rows * dp * 4


def test_workspace_size_of_grouped_runs():
    """17-32 rows per KV head (two row blocks) and 5-8 (two column slots) run
    each run of the split on four waves: a launch of W waves has W / 4 runs,
    two partial slots each.  A shape whose fused single-token form runs one
    wave per run (quantized pages, at most 8 rows) is sized for that form."""
    lib = nat.load()
    # 20 rows (5 queries at GQA 4): 100 waves = 25 runs
    assert lib.pkv_attention_workspace_bytes(_layout(), 32, 5, 100) == _parts(25, 20)
    assert lib.pkv_attention_workspace_bytes(_layout(), 32, 5, 3) == _parts(1, 20)  # at least one
    # bf16 pages, 28 rows: grouped, no fused form
    bf = _layout(bits=16, group_size=32)
    assert lib.pkv_attention_workspace_bytes(bf, 32, 7, 100) == _parts(25, 28)
    # 8 rows (GQA 8): grouped when separate, one wave per run when fused
    assert lib.pkv_attention_workspace_bytes(_layout(), 64, 1, 100) == _parts(100, 8)
    # ... and on bf16 pages (no fused form): grouped
    assert lib.pkv_attention_workspace_bytes(bf, 64, 1, 100) == _parts(25, 8)
    # 4 rows: one wave per run
    assert lib.pkv_attention_workspace_bytes(_layout(), 32, 1, 100) == _parts(100, 4)


def _attention(lib, layout, **kw):
    args = dict(stream=None, pool=FAKE, num_pages=10, q=FAKE, batch=2, heads=32, nq=1, table=FAKE,
                max_pages=4, lens=FAKE, q_pos=None, widths=None, scale=0.1, waves=3,
                ws=None, ws_bytes=0, out=FAKE)
    args.update(kw)
    return lib.pkv_paged_attention(args["stream"], layout, args["pool"], args["num_pages"],
                                   args["q"], args["batch"], args["heads"], args["nq"],
                                   args["table"], args["max_pages"], args["lens"], args["q_pos"],
                                   args["widths"], args["scale"], args["waves"],
                                   args["ws"], args["ws_bytes"], args["out"])


@pytest.mark.parametrize("kw,code", [
    (dict(heads=30), nat.PKV_UNSUPPORTED),                      # not a GQA multiple of HK=8
    (dict(nq=1 << 23), nat.PKV_UNSUPPORTED),                    # 2^25 rows per KV head
    (dict(nq=9, pool=None), nat.PKV_INVALID_ARGUMENT),          # prefill route validates too
    (dict(pool=None), nat.PKV_INVALID_ARGUMENT),
    (dict(num_pages=0), nat.PKV_INVALID_ARGUMENT),
    (dict(waves=3), nat.PKV_OUT_OF_MEMORY),                     # the merge needs a workspace
    (dict(waves=3, ws=FAKE, ws_bytes=64), nat.PKV_OUT_OF_MEMORY),
    (dict(waves=1 << 25, ws=FAKE, ws_bytes=1 << 40), nat.PKV_INVALID_ARGUMENT),
    (dict(scale=float("inf")), nat.PKV_INVALID_ARGUMENT),
    (dict(batch=-1), nat.PKV_INVALID_ARGUMENT),
    (dict(batch=0), nat.PKV_OK),
])
def test_attention_argument_validation(kw, code):
    lib = nat.load()
    assert _attention(lib, _layout(), **kw) == code
    if code != nat.PKV_OK:
        assert nat.last_error()


def test_append_argument_validation():
    lib = nat.load()
    layout = _layout()
    call = lambda **kw: lib.pkv_append_quantize(
        None, layout, kw.get("pool", FAKE), 10, FAKE, FAKE, kw.get("batch", 2), 1, FAKE, 4,
        kw.get("start", FAKE), None, kw.get("new_lens", None))
    assert call(pool=None) == nat.PKV_INVALID_ARGUMENT
    assert call(start=None) == nat.PKV_INVALID_ARGUMENT
    assert call(new_lens=FAKE) == nat.PKV_INVALID_ARGUMENT    # aliases start_pos
    assert call(batch=0) == nat.PKV_OK
    assert lib.pkv_append_quantize(None, _layout(bits=3), FAKE, 10, FAKE, FAKE, 1, 1, FAKE, 4,
                                   FAKE, None, None) == nat.PKV_UNSUPPORTED


def test_quantize_rows_argument_validation():
    lib = nat.load()
    assert lib.pkv_quantize_rows(None, FAKE, 4, 128, 3, 32, 0, FAKE, FAKE, FAKE) == nat.PKV_UNSUPPORTED
    assert lib.pkv_quantize_rows(None, FAKE, 4, 128, 8, 48, 0, FAKE, FAKE, FAKE) == nat.PKV_UNSUPPORTED
    assert lib.pkv_quantize_rows(None, FAKE, 0, 128, 8, 32, 0, FAKE, FAKE, FAKE) == nat.PKV_OK
    assert lib.pkv_dequantize_rows(None, FAKE, FAKE, FAKE, 4, 0, 8, 32, FAKE) == nat.PKV_INVALID_ARGUMENT


def test_read_probe_argument_validation():
    lib = nat.load()
    layout = _layout()
    call = lambda **kw: lib.pkv_read_probe(None, kw.get("layout", layout), kw.get("pool", FAKE), 10,
                                           kw.get("ids", FAKE), kw.get("count", 4),
                                           kw.get("waves", 8), kw.get("out", FAKE))
    assert call(waves=0) == nat.PKV_INVALID_ARGUMENT
    assert call(count=-1) == nat.PKV_INVALID_ARGUMENT
    assert call(out=None) == nat.PKV_INVALID_ARGUMENT
    assert call(pool=None) == nat.PKV_INVALID_ARGUMENT
    assert call(ids=None) == nat.PKV_INVALID_ARGUMENT
    assert call(count=0) == nat.PKV_OK
    assert call(layout=_layout(bits=3)) == nat.PKV_UNSUPPORTED


def test_status_codes_map_to_reference_exceptions():
    from pkv.cache_errors import CacheCapacityError
    from pkv.modes import ModelCapabilityUnsupported

    lib = nat.load()
    _attention(lib, _layout(), heads=30)
    with pytest.raises(ModelCapabilityUnsupported):
        nat.check(nat.PKV_UNSUPPORTED, "attention")
    with pytest.raises(ValueError):
        nat.check(nat.PKV_INVALID_ARGUMENT, "attention")
    with pytest.raises(CacheCapacityError):
        nat.check(nat.PKV_OUT_OF_MEMORY, "attention")


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(nat.NativeLibraryMissing):
        nat.load(tmp_path / "libpkv.so")


@pytest.mark.parametrize("args", [
    (1, 1, 8, 2, 127, 1),      # odd head dimension
    (1, 1, 8, 2, 258, 1),      # head dimension above 256
    (1, 1, 0, 2, 128, 1),      # no query heads
    (1, 1, 8, 0, 128, 1),      # no KV heads
    (1, 1, 8, 2, 128, 2),      # unknown float kind
    (-1, 1, 8, 2, 128, 1),     # negative batch
])
def test_rope_rejects_bad_shapes(args):
    lib = nat.load()
    b, t, h, hk, d, kind = args
    code = lib.pkv_rope_qkv(None, FAKE, b, t, h, hk, d, kind, FAKE, FAKE, FAKE, FAKE, FAKE)
    assert code == nat.PKV_INVALID_ARGUMENT


def test_rope_empty_batch_and_null_tensors():
    lib = nat.load()
    assert lib.pkv_rope_qkv(None, None, 0, 5, 8, 2, 128, 1, None, None, None, None, None) == nat.PKV_OK
    assert lib.pkv_rope_qkv(None, None, 1, 1, 8, 2, 128, 1, FAKE, FAKE, FAKE, FAKE,
                            FAKE) == nat.PKV_INVALID_ARGUMENT


def test_arena_state_size_and_argument_checks():
    lib = nat.load()
    assert lib.pkv_arena_state_bytes(100) == (16 + 200) * 4
    assert lib.pkv_arena_state_bytes(0) < 0
    assert lib.pkv_arena_init(None, None, 10) == nat.PKV_INVALID_ARGUMENT
    assert lib.pkv_arena_init(None, FAKE, 0) == nat.PKV_INVALID_ARGUMENT
    common = (None, FAKE, 64, 16, FAKE, 8, 32, FAKE)
    pools = (ctypes.c_void_p * 1)(4096)
    # nothing to do: returns before any HIP call
    assert lib.pkv_arena_reserve(*common, None, None, 0, None, 0, 0, None, None, None) == nat.PKV_OK
    assert lib.pkv_arena_truncate(*common, None, None, 0) == nat.PKV_OK
    assert lib.pkv_arena_fork(*common, None, None, 0) == nat.PKV_OK
    bad = [
        (None, FAKE, 64, 24, FAKE, 8, 32, FAKE),   # page_tokens
        (None, FAKE, 0, 16, FAKE, 8, 32, FAKE),    # capacity
        (None, FAKE, 64, 16, FAKE, 0, 32, FAKE),   # slots
        (None, None, 64, 16, FAKE, 8, 32, FAKE),   # state
    ]
    for args in bad:
        assert lib.pkv_arena_truncate(*args, FAKE, FAKE, 1) == nat.PKV_INVALID_ARGUMENT
    assert lib.pkv_arena_truncate(*common, FAKE, FAKE, -1) == nat.PKV_INVALID_ARGUMENT
    assert lib.pkv_arena_reserve(*common, FAKE, FAKE, 1, pools, 200, 4096, FAKE, FAKE,
                                 FAKE) == nat.PKV_INVALID_ARGUMENT      # pools
    assert lib.pkv_arena_reserve(*common, FAKE, FAKE, 1, pools, 1, 10, FAKE, FAKE,
                                 FAKE) == nat.PKV_INVALID_ARGUMENT      # page bytes
    assert lib.pkv_arena_reserve(*common, FAKE, FAKE, 1, pools, 1, 4096, None, FAKE,
                                 FAKE) == nat.PKV_INVALID_ARGUMENT      # outputs
