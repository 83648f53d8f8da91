import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _ensure_built():
    """Builds the in-tree libraries only if they are missing."""
    lib = os.path.join(ROOT, "m1moe_amd", "libm1moe_hip.so")
    orc = os.path.join(ROOT, "oracle", "liboracle_m1moe.so")
    if not os.path.exists(orc):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True)
    if not os.path.exists(lib):
        subprocess.run(["make", "-j8", "-C", os.path.join(ROOT, "m1moe_amd", "csrc")], check=True)


_ensure_built()
