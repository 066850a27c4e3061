"""The copy threads of the host-to-host entry points (tk_copy_pool.h), on
the CPU: every chunk of every job runs exactly once and only under its own
job, across back-to-back jobs and across the workers' sleep; and
ThreadSanitizer finds no data race in the pool."""
import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
SRC = HERE / "copy_pool_stress.cpp"


def _build_and_run(tmp_path, flags, args):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not found")
    exe = tmp_path / "copy_pool_stress"
    subprocess.run([gxx, "-std=c++17", "-pthread", *flags, "-o", str(exe), str(SRC)],
                   check=True, capture_output=True, text=True, timeout=120)
    r = subprocess.run([str(exe), *map(str, args)], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("ok:"), r.stdout
    return r


def test_copy_pool_runs_every_chunk_once(tmp_path):
    _build_and_run(tmp_path, ["-O2"], [8, 100_000])


def test_copy_pool_under_thread_sanitizer(tmp_path):
    r = _build_and_run(tmp_path, ["-O1", "-g", "-fsanitize=thread"], [4, 10_000])
    assert "ThreadSanitizer" not in r.stderr, r.stderr
