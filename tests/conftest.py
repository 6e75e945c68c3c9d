"""pytest configuration: the `gpu` marker and import paths.

Tests marked ``gpu`` need an MI355X (they run through the HIP library's C
ABI); everything else runs on the CPU and never loads the HIP library's
compute entry points.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU (runs the HIP path through the C ABI)")
