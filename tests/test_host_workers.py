"""The host thread pool used for payload generation in the serving loop and
for the staged uploads of the device pool (csrc/host_workers.h), checked on
the CPU: a small C++ program built with g++ against the header."""
from __future__ import annotations

import os
import pathlib
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
CSRC = ROOT / "15-618_dynamic_sparse_decode_amd" / "csrc"


@pytest.mark.parametrize("threads", ["1", "4", "16"])
def test_host_workers_cover_every_index_once(tmp_path, threads):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    exe = tmp_path / "host_workers_check"
    subprocess.run(["g++", "-std=c++17", "-O2", "-pthread", f"-I{CSRC}",
                    str(ROOT / "tests" / "native" / "host_workers_check.cpp"), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    env = dict(os.environ, DSD_HOST_THREADS=threads)
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120, env=env)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert f"host workers ok: {threads} threads" in proc.stdout, proc.stdout
