"""pytest configuration: markers and import paths.

``gpu`` marks tests that need an MI355X (run on the GPU box with ``-m gpu``);
everything else runs on the CPU container.
"""

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "cayley-delta-state-space-model_amd")
for p in (ROOT, PKG_DIR):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")
