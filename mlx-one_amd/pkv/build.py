"""Build libpkv.so (HIP for gfx950) in-tree.

``python -m pkv.build`` (with ``mlx-one_amd`` on ``sys.path``) or
``pkv.build.build()``.  Compiles every ``csrc/*.hip`` with hipcc for gfx950 and
links them into ``pkv/libpkv.so``, the library ``pkv._native`` loads.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent                  # mlx-one_amd/
CSRC = ROOT / "csrc"
INCLUDE = ROOT.parent / "include"      # repo-level public headers (pkv.h)
LIBRARY = PACKAGE / "libpkv.so"
ARCH = "gfx950"

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # keep f32 division / sqrt IEEE-correct (the quantizer is bit-exact)
    "-fno-fast-math", "-ffp-contract=fast-honor-pragmas",
    # no packed-f32 VALU instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: no AGPR<->VGPR copies around the online softmax
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-Wno-unused-result",
]


def sources():
    return sorted(CSRC.glob("*.hip"))


def build(verbose=False, jobs=None):
    """Compile each source to an object (in parallel), then link the library."""
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    objdir = ROOT / "_build"
    objdir.mkdir(exist_ok=True)
    procs, objects = [], []
    for src in sources():
        obj = objdir / (src.stem + ".o")
        objects.append(obj)
        cmd = [hipcc, *FLAGS, "-I", str(CSRC), "-I", str(INCLUDE), "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
    failed = []
    for src, proc in procs:
        out, _ = proc.communicate()
        text = out.decode(errors="replace")
        noise = "is not a recognized feature for this target"
        lines = [l for l in text.splitlines() if noise not in l]
        if lines and (verbose or proc.returncode):
            print("\n".join(lines), file=sys.stderr)
        if proc.returncode:
            failed.append(src.name)
    if failed:
        raise RuntimeError(f"hipcc failed for {', '.join(failed)}")
    tmp = str(LIBRARY) + ".tmp"
    cmd = [hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objects), "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
