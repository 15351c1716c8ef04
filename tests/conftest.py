"""Test configuration: import paths and the ``gpu`` marker.

``-m "not gpu"`` runs the CPU suite (oracle pinning, host logic, ABI symbol
checks); ``-m gpu`` runs the parity tests on an MI355X through the C ABI.
"""

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
for path in (ROOT / "mlx-one_amd", ROOT, Path(__file__).resolve().parent):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libpkv.so")
