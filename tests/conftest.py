"""Test configuration: registers the ``gpu`` marker and puts the package
(tiga-lang_amd/) and the repository root (oracle/) on sys.path."""

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "tiga-lang_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
