"""Shared pytest setup: import paths and the ``gpu`` marker.

``-m "not gpu"`` runs here (no GPU): the oracle against golden vectors and
invariants, host-side logic and the C-ABI library's exports.  ``-m gpu``
runs on an MI355X: the HIP kernels through the C ABI against the oracle.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("", "flash-attention-cpu_amd", "oracle", "tests"):
    p = os.path.join(ROOT, sub) if sub else ROOT
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD MI355X (gfx950); runs on the GPU box")
