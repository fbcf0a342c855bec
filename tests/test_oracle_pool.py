"""The oracle's persistent worker pool (oracle/wpc_oracle.c, parallel_rows)
under alternating thread counts.

Rows are split over threads as the reference's rayon pool splits them
(wpc-runtime/src/wpc_weights_v4.rs:165-193); each row is independent, so
every call must return the one-thread result bit for bit, whatever workers
sat out the previous call. tests/c/oracle_pool_stress.c alternates 16, 3, 8,
2, ... threads over thousands of small calls; it runs once as a plain build
and once under ThreadSanitizer, which reports any unsynchronised access
between the caller publishing a job and a worker reading it.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = [os.path.join(ROOT, "tests", "c", "oracle_pool_stress.c"), os.path.join(ROOT, "oracle", "wpc_oracle.c")]


def _build_and_run(tmp_path, flags, iters, env=None):
    exe = str(tmp_path / "stress")
    cc = shutil.which("gcc") or "cc"
    r = subprocess.run([cc, "-std=c11", "-ffp-contract=off", *flags, "-o", exe, *SRC, "-lm", "-lpthread"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    r = subprocess.run([exe, str(iters)], capture_output=True, text=True, timeout=600, env=env)
    return r


def test_pool_alternating_thread_counts(tmp_path):
    r = _build_and_run(tmp_path, ["-O2", "-pthread"], 20000)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "20000 calls agree" in r.stdout


def test_pool_with_a_stalled_worker(tmp_path):
    """OR_POOL_STALL_US puts a 50 us sleep in the worker between reading the
    job generation and reading `want` and the job: the window in which the
    next call can publish a new job. Read without the pool's lock (as the
    pool once read them) a non-participating worker then runs the next job
    under the old generation and again under the new one, and this stress
    run fails within a few dozen calls; read under the lock, every call
    agrees."""
    r = _build_and_run(tmp_path, ["-O2", "-pthread", "-D_DEFAULT_SOURCE", "-DOR_POOL_STALL_US=50"], 3000)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "3000 calls agree" in r.stdout


def test_pool_under_thread_sanitizer(tmp_path):
    probe = subprocess.run([shutil.which("gcc") or "cc", "-fsanitize=thread", "-x", "c", "-", "-o",
                            str(tmp_path / "probe")], input="int main(void){return 0;}",
                           capture_output=True, text=True)
    if probe.returncode != 0:
        pytest.skip("gcc has no ThreadSanitizer runtime here")
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=1:exitcode=66")
    r = _build_and_run(tmp_path, ["-O1", "-g", "-pthread", "-fsanitize=thread"], 1500, env)
    out = r.stdout + r.stderr
    assert "ThreadSanitizer" not in out, out[-4000:]
    assert r.returncode == 0, out[-4000:]
