"""pytest configuration: the `gpu` marker and import paths.

Tests marked `gpu` need an MI355X (gfx950) and the built HIP library; the
rest run on any CPU. Nothing here imports torch: the HIP library owns its
device memory and streams, and keeping a second HIP runtime out of the
process avoids two copies of libamdhip64 side by side.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "wpc-engine_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")
