"""Shared test setup: import paths and the ``gpu`` marker.

``-m "not gpu"`` runs the oracle, host-logic and ABI-load tests on any machine;
``-m gpu`` runs the parity tests through the C ABI on an MI355X.
"""

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "sgl-afd-plugin_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libafd.so")
