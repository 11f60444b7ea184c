"""pytest configuration: the `gpu` marker and import paths.

`-m "not gpu"` runs on any host (oracle checks, host logic, C-ABI symbol
checks); `-m gpu` needs an MI355X and the built libm2ssd.so.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "mamba2-jax-pallas_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")
