"""The host parsers and the malformed-file tests under AddressSanitizer and
UndefinedBehaviorSanitizer.

The library reads untrusted files on the host: the artifact's JSON meta
(csrc/meta_json.cpp, csrc/json.cpp), safetensors checkpoints and their index
(csrc/safetensors.cpp), config.json, and the block bytes it transcodes
(csrc/transcode.cpp) or encodes (csrc/encode.cpp). This test builds the
host C++ of the library with -fsanitize=address,undefined
(wpc-engine_amd/asan.mk; the gfx950 kernels are linked unchanged and are
not run here) and runs the CPU tests that feed those readers broken input
(every safetensors format check broken in turn, truncated and malformed
meta files, shape and block-count errors, the header and sort-order tests)
in a child Python with the sanitizer runtime preloaded. Any
out-of-bounds access, use after free or undefined behaviour aborts the
child, and the child's pytest must pass.
"""
import glob
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "wpc-engine_amd")
SUITES = ["tests/test_safetensors.py", "tests/test_capi_host.py", "tests/test_encode.py",
          "tests/test_golden.py"]


def _runtime():
    hits = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return hits[-1] if hits else None


def test_parsers_clean_under_asan_and_ubsan():
    rt = _runtime()
    if rt is None:
        pytest.skip("ROCm clang's AddressSanitizer runtime is not installed")
    r = subprocess.run(["make", "-s", "-j8", "-f", "asan.mk"], cwd=PKG, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    env = dict(os.environ)
    env.update(WPCG_LIB=os.path.join(PKG, "_build", "asan", "libwpcg_asan.so"), LD_PRELOAD=rt,
               # the HIP runtime's own allocations live to exit; leaks are not what is checked
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-m", "not gpu", "-p", "no:cacheprovider",
                        *SUITES], cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    out = r.stdout[-4000:] + r.stderr[-4000:]
    assert r.returncode == 0, out
    assert "ERROR: AddressSanitizer" not in out and "runtime error:" not in out, out
    assert "libwpcg_asan.so" in subprocess.run(
        [sys.executable, "-c", "import wpcg; print(wpcg.LIB_PATH)"], cwd=ROOT,
        env=dict(env, PYTHONPATH=PKG), capture_output=True, text=True).stdout
