"""pytest configuration: import paths and the `gpu` marker.

The product package lives in kairos-sensenova_amd/ (a directory name that is
not a Python identifier), so its parent is put on sys.path; the repository
root is on sys.path for the test-only oracle package.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "kairos-sensenova_amd"), os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); parity of the kernels against the oracle")
