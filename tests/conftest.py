"""pytest configuration: the ``gpu`` marker and import paths.

``astra-cuda_amd/`` holds the ``astra_cuda`` package (the drop-in module) and
its HIP sources; the repository root holds ``oracle/`` (the CPU checker).
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "astra-cuda_amd"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (HIP device) to run")
