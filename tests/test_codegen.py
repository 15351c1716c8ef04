"""Generated-code checks on the built library's gfx950 code (no GPU).

Two kernel variants have returned wrong results on the GPU while their
arithmetic reads correctly, and in both the compiler had emitted an MFMA whose
accumulator input is the inline constant 0 and whose destination registers
partly overlap its A or B operand registers (e.g.
``v_mfma_f32_16x16x16_bf16 v[150:153], v[152:153], v[168:169], 0``): a decode
kernel running every slot's MFMAs unguarded, and a prefill kernel whose bias
MFMA began the score chain.  Identical overlap (``v[4:7], v[4:7], ..., 0``) and
overlap with a register accumulator occur throughout kernels that pass, so
only the partial form with a zero accumulator is refused here, in every kernel
of the library.

The device code objects are read from the library's offload bundles and
disassembled with the ROCm ``llvm-objdump`` (this build's own code).
"""

from __future__ import annotations

import re
import struct
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
LIBRARY = ROOT / "mlx-one_amd" / "pkv" / "libpkv.so"
LLVM = Path("/opt/rocm/llvm/bin")
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def _code_objects(tmp_path):
    """The gfx950 code objects of the library's .hip_fatbin section, one per
    bundle (one bundle per compiled source)."""
    fatbin = tmp_path / "fatbin.bin"
    subprocess.run([str(LLVM / "llvm-objcopy"), f"--dump-section=.hip_fatbin={fatbin}",
                    str(LIBRARY), str(tmp_path / "lib.tmp")], check=True, capture_output=True)
    data = fatbin.read_bytes()
    objects = []
    at = data.find(MAGIC)
    while at >= 0:
        (entries,) = struct.unpack_from("<Q", data, at + len(MAGIC))
        q = at + len(MAGIC) + 8
        for _ in range(entries):
            offset, size, tlen = struct.unpack_from("<QQQ", data, q)
            q += 24
            triple = data[q:q + tlen].decode()
            q += tlen
            if "gfx950" in triple and size:
                path = tmp_path / f"co{len(objects)}.o"
                path.write_bytes(data[at + offset:at + offset + size])
                objects.append(path)
        at = data.find(MAGIC, at + 1)
    return objects


def _regs(operand):
    m = re.fullmatch(r"[va]\[(\d+):(\d+)\]", operand)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"[va](\d+)", operand)
    return {int(m.group(1))} if m else set()


def zero_accumulator_overlaps(listing):
    """(function, instruction) for each MFMA with an inline 0 accumulator whose
    destination partly overlaps its A or B registers."""
    found, func = [], "?"
    for line in listing.splitlines():
        head = re.match(r"^[0-9a-f]+ <(\S+)>:", line)
        if head:
            func = head.group(1)
            continue
        text = line.split("//")[0].strip()
        if not text.startswith("v_mfma"):
            continue
        ops = [o.strip() for o in text.split(None, 1)[1].split(",")]
        if len(ops) < 4 or ops[3] != "0":
            continue
        dst = _regs(ops[0])
        for src in (_regs(ops[1]), _regs(ops[2])):
            if dst & src and dst != src:
                found.append((func, text))
    return found


def test_overlap_scan_flags_the_pattern():
    listing = ("0000000000001000 <k>:\n"
               "\tv_mfma_f32_16x16x16_bf16 v[150:153], v[152:153], v[168:169], 0 // 1000: 0\n"
               "\tv_mfma_f32_16x16x32_f16 v[4:7], v[4:7], v[8:11], 0 // 1008: 0\n"
               "\tv_mfma_f32_16x16x32_f16 v[2:5], v[4:7], v[8:11], v[2:5] // 1010: 0\n")
    assert zero_accumulator_overlaps(listing) == [
        ("k", "v_mfma_f32_16x16x16_bf16 v[150:153], v[152:153], v[168:169], 0")]


@pytest.mark.skipif(not LIBRARY.exists(), reason="libpkv.so not built")
@pytest.mark.skipif(not (LLVM / "llvm-objdump").exists(), reason="ROCm llvm tools not installed")
def test_no_zero_accumulator_mfma_overlaps_its_operands(tmp_path):
    objects = _code_objects(tmp_path)
    assert objects, "no gfx950 code object in the library"
    bad, mfmas = [], 0
    for obj in objects:
        listing = subprocess.run([str(LLVM / "llvm-objdump"), "-d", "--mcpu=gfx950", str(obj)],
                                 check=True, capture_output=True, text=True).stdout
        mfmas += listing.count("v_mfma")
        bad += zero_accumulator_overlaps(listing)
    assert mfmas > 1000
    assert not bad, "\n".join(f"{f}: {t}" for f, t in bad[:20])
