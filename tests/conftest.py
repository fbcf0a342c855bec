"""pytest configuration: the `gpu` marker, import paths and process exit.

Tests marked `gpu` need an MI355X (gfx950) and the built HIP library; the
rest run on any CPU. Nothing here imports torch: the HIP library owns its
device memory and streams, and keeping a second HIP runtime out of the
process avoids two copies of libamdhip64 side by side.

A session that touched the GPU ends through wpcg.finish after pytest has
written its report: every native handle is released (newest first), then
the process leaves normally, or through os._exit with pytest's exit status
when WPCG_HARD_EXIT=1; see wpcg.NORMAL_EXIT.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "wpc-engine_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

_exit_status = {"code": 0}


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


def pytest_sessionfinish(session, exitstatus):
    _exit_status["code"] = int(exitstatus)


@pytest.hookimpl(trylast=True)
def pytest_unconfigure(config):
    wpcg = sys.modules.get("wpcg")
    if wpcg is not None and wpcg.gpu_used():
        wpcg.finish(_exit_status["code"])
