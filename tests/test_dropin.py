"""The drop-in check: the reference's own test programs, benchmark and demo,
compiled unchanged against include/dsd/ and linked to libdsd.so (with the
CPU rows from oracle/liboracle_cpu.so), must pass as they do against the
reference's library.

The binaries are built in this container by `make -C oracle dropin` from the
reference's sources where they lie (outputs only under oracle/_ref/dropin/,
which is git-ignored and travels to the GPU box prebuilt).  Where they were
not built (no reference tree), the tests skip.

  tests/test_page_pool.cpp, tests/test_reference.cpp    CPU
  tests/test_device_page_pool.cpp, test_dense_cuda.cpp,
  test_sparse_cuda.cpp, test_continuous_batching.cpp     GPU (they print
      "skipped: no visible sm90 GPU" and exit 0 without one, so the GPU
      marker is what makes them meaningful)
  benchmarks/bench_decode.cpp                            GPU: its accuracy
      lines (sparse_gpu vs sparse_cpu, dense_gpu vs dense_cpu) are checked
"""
from __future__ import annotations

import pathlib
import re
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
DROPIN = ROOT / "oracle" / "_ref" / "dropin"


def run(name, *args, timeout=300):
    exe = DROPIN / name
    if not exe.exists():
        pytest.skip(f"{exe} not built (needs the reference tree: make -C oracle dropin)")
    print(f"[dropin] {name} {' '.join(args)}", flush=True)
    proc = subprocess.run([str(exe), *args], capture_output=True, text=True, timeout=timeout)
    return proc


@pytest.mark.parametrize("name,expect", [
    ("test_page_pool", "page pool tests passed"),
    ("test_reference", "reference tests passed"),
])
def test_reference_cpu_tests_pass_against_libdsd(name, expect):
    proc = run(name)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert expect in proc.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("name,expect", [
    ("test_device_page_pool", "device page pool tests passed"),
    ("test_dense_cuda", "dense cuda tests passed"),
    ("test_sparse_cuda", "sparse cuda tests passed"),
    ("test_continuous_batching", "continuous batching tests passed"),
])
def test_reference_gpu_tests_pass_against_libdsd(name, expect):
    proc = run(name)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "skipped" not in proc.stdout, proc.stdout
    assert expect in proc.stdout, proc.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("args", [
    # top_k batch min max seed iters warmup heads head_dim page  (argv order)
    ("8", "4", "64", "300", "7", "1", "0", "4", "16", "16"),
    ("8", "4", "512", "1024", "3", "1", "0", "32", "128", "16"),
])
def test_reference_bench_decode_accuracy_lines(args):
    proc = run("bench_decode", *args)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    out = proc.stdout
    diffs = dict(re.findall(r"(avg_max_abs_diff_\w+)=([-+0-9.eE]+)", out))
    assert "avg_max_abs_diff_sparse_gpu_vs_sparse_cpu" in diffs, out
    assert float(diffs["avg_max_abs_diff_sparse_gpu_vs_sparse_cpu"]) <= 1e-4
    if "avg_max_abs_diff_dense_gpu_vs_dense_cpu" in diffs:
        assert float(diffs["avg_max_abs_diff_dense_gpu_vs_dense_cpu"]) <= 1e-4


@pytest.mark.gpu
@pytest.mark.parametrize("args", [
    # requests, max active, window, prompt min/max, decode min/max, seed, heads,
    # head_dim, page size, top-k, then admission mode, preadmit, precompute,
    # GPU synthetic append, lazy release, output mode, timing mode (argv order)
    ("8", "4", "4", "64", "512", "2", "6", "7", "32", "128", "16", "4",
     "1", "1", "1", "1", "1", "1", "1"),                       # published flags, fused step
    ("8", "4", "4", "64", "512", "2", "6", "7", "32", "128", "16", "4"),  # driver defaults
    ("8", "4", "4", "64", "512", "2", "6", "7", "32", "64", "16", "4",
     "1", "1", "1", "1", "1", "0", "0"),                       # three-kernel step, no outputs
])
@pytest.mark.parametrize("table", ["1", "0"])
def test_reference_continuous_driver_staged_steps_verified(args, table):
    """The reference's continuous driver against libdsd.so with
    DSD_VERIFY_STAGED=1: every step the loop stages (queries read from the
    pinned payload rows or the staging; candidate lists packed on the device
    from the page table, or with DSD_DEVICE_TABLE=0 copied from the host
    cache) is run again through RunBatch's packing path on the host cache's
    page lists and must match it bit for bit; with the table, the device's
    page lists must also equal the host cache's (the reference's page order)
    at every step.  Either failure ends the run."""
    import os
    exe = DROPIN / "bench_continuous_decode"
    if not exe.exists():
        pytest.skip(f"{exe} not built (needs the reference tree: make -C oracle dropin)")
    print(f"[dropin] bench_continuous_decode {' '.join(args)} (verified, table {table})",
          flush=True)
    env = dict(os.environ, DSD_VERIFY_STAGED="1", DSD_DEVICE_TABLE=table)
    proc = subprocess.run([str(exe), *args], capture_output=True, text=True, timeout=300, env=env)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "continuous_sparse_tokens_per_second=" in proc.stdout, proc.stdout
    # the continuous and the serial run each report their running total
    counts = [int(n) for n in re.findall(r"dsd: (\d+) staged steps verified", proc.stderr)]
    assert len(counts) >= 2 and counts[0] > 0 and counts[-1] > counts[0], proc.stderr
