"""pytest configuration: the `gpu` marker and import paths.

Tests marked `gpu` need a real MI355X and the built library; everything else
runs on the CPU (oracle pinning, ABI surface, runtime validation).
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "catena-lang_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built library")
