"""pytest configuration: the ``gpu`` marker and import paths.

``-m "not gpu"`` runs everywhere (oracle checks, C-ABI loading and
validation, host logic); ``-m gpu`` needs an MI355X and calls the HIP
kernels through the C ABI.
"""

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "triton-kernels_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP kernels are launched)")
