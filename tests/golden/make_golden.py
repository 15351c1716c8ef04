"""Write golden vectors for the page quantizer from the reference's own code.

Runs in the build container only (the reference tree is not present on GPU
boxes) and writes ``quantize_page_g32.npz`` next to this file, which the tests
read.  It imports ``quantize_page`` / ``dequantize_page`` from
``src/mlx_one/engine/paged.py:24-54`` of the reference with a numpy stand-in
for ``mlx.core``, the way the reference's backend-free tests run that code
(``tests/test_dense_batching.py:26-37``, ``tests/test_paged_hybrid.py:48-62``).
Package ``__init__`` modules of the reference are bypassed so that only the
paged engine modules load.

Only the quantizer is taken this way: it is the one function on the path whose
bit-exact behaviour (f16 rounding order, half-to-even ties) no closed form in
the reference's tests pins.  Usage: ``python tests/golden/make_golden.py
[/root/reference]``.
"""

from __future__ import annotations

import sys
import types
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def _install_stub(reference_src):
    core = types.ModuleType("mlx.core")
    core.array, core.zeros, core.concatenate = np.array, np.zeros, np.concatenate
    core.float16, core.bfloat16 = np.float16, np.float32
    core.eval = lambda *args: None
    for name in ("pad", "stack", "min", "max", "maximum", "round", "clip", "uint8",
                 "float32", "int32", "where", "exp", "abs", "all", "arange"):
        setattr(core, name, getattr(np, name))
    package = types.ModuleType("mlx")
    package.core = core
    sys.modules["mlx"], sys.modules["mlx.core"] = package, core
    for name, sub in (("mlx_one", ""), ("mlx_one.engine", "engine")):
        module = types.ModuleType(name)
        module.__path__ = [str(Path(reference_src, "mlx_one", sub))]
        sys.modules[name] = module


def _bf16(x):
    bits = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)


def cases():
    """Inputs: name -> float16 array, or bf16-valued float32 array."""
    out = {}
    rng = np.random.default_rng(12)
    # the reference's own round-trip test input (test_paged_hybrid.py:194-196)
    out["ref_test_f16_d37"] = rng.normal(size=(1, 2, 16, 37)).astype(np.float16)
    rng = np.random.default_rng(2026)
    x = rng.normal(size=(1, 8, 16, 128)).astype(np.float32)
    x[..., rng.choice(128, 3, replace=False)] *= 8       # outlier channels
    out["bf16_d128_outliers"] = _bf16(x)
    out["bf16_d64"] = _bf16(rng.normal(size=(1, 2, 16, 64)).astype(np.float32) * 3)
    out["f16_d256_wide"] = (rng.normal(size=(1, 1, 16, 256)) * 40).astype(np.float16)
    out["f16_d4_toy"] = rng.normal(size=(1, 1, 16, 4)).astype(np.float16)
    # exact .5 ties: min 0, max 2^b - 1 => scale 1, codes (k + .5) round to even
    ties = np.zeros((1, 2, 16, 32), np.float32)
    for t in range(16):
        ties[0, 0, t] = np.concatenate(([0.0, 255.0], np.arange(30) * 8 + 0.5 + t))[:32]
        ties[0, 1, t] = np.concatenate(([0.0, 15.0], (np.arange(30) % 15) + 0.5))[:32]
    out["f16_ties"] = ties.astype(np.float16)
    # constant and zero groups: scale clamps to f16(1e-6), a subnormal
    const = np.zeros((1, 1, 16, 64), np.float16)
    const[0, 0, :8] = np.float16(3.25)
    const[0, 0, 8:, 32:] = np.float16(-7.0)
    out["f16_constant_groups"] = const
    # scales near f16 rounding boundaries and negative-only groups
    out["f16_negative"] = (-np.abs(rng.normal(size=(1, 2, 16, 32))) * 5 - 1).astype(np.float16)
    out["f16_tiny"] = (rng.normal(size=(1, 1, 16, 32)) * 1e-3).astype(np.float16)
    return out


def main(reference=None):
    reference = Path(reference or "/root/reference")
    _install_stub(reference / "src")
    from mlx_one.engine.paged import dequantize_page, quantize_page

    arrays = {}
    for name, value in cases().items():
        arrays[f"{name}/input"] = value
        for bits in (4, 8):
            codes, scale, bias = quantize_page(value, bits)
            restored = dequantize_page((codes, scale, bias), bits, value.shape[-1])
            arrays[f"{name}/b{bits}/codes"] = np.asarray(codes, np.uint8)
            arrays[f"{name}/b{bits}/scale"] = np.asarray(scale, np.float16)
            arrays[f"{name}/b{bits}/bias"] = np.asarray(bias, np.float16)
            arrays[f"{name}/b{bits}/dequant"] = np.asarray(restored, np.float32)
    target = HERE / "quantize_page_g32.npz"
    np.savez_compressed(target, **arrays)
    print(f"wrote {target} ({target.stat().st_size} bytes, {len(arrays)} arrays)")


if __name__ == "__main__":
    main(*sys.argv[1:])
