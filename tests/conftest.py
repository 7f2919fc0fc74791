"""pytest configuration: the `gpu` marker and import paths.

GPU tests are marked ``@pytest.mark.gpu`` and run on an MI355X with
``python -m pytest tests -m gpu``; everything else runs on CPU.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "w4a16-gemm_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP extension")
