"""Test configuration: the `gpu` marker (tests that need an MI355X) and the oracle build.

CPU tests (-m "not gpu") check the oracle against the reference's golden values, the reference kernels (when the
prebuilt oracle/_ref library is present) and closed forms, plus the host logic and the exported C-ABI symbols. GPU
tests (-m gpu) are the parity tests proper: the HIP path through the C-ABI against the oracle, bit for bit.
"""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "tests"))
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct MI355X (gfx950) and the built HIP library")
    oracle_so = ROOT / "oracle" / "liboracle.so"
    if not oracle_so.exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle"), "liboracle.so"], check=True, capture_output=True)
