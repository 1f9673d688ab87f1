"""Shared pytest setup: the `gpu` marker and import paths.

GPU tests (marked ``gpu``) need an MI355X and the built HIP library; the
rest run on any CPU against the oracle and the library's exported symbols.
"""
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
for path in (ROOT, ROOT / "falcon-ocr-cpu_amd", ROOT / "oracle", ROOT / "tests"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")
