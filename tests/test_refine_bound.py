"""The refined score intervals (csrc/refine_lane.h: the per-lane arithmetic
of RefineScores, which settles near-ties at the top-k boundary without the
exact sequential chain) checked on the CPU.  tests/native/refine_check.cpp
runs the header's code for every lane layout a workgroup uses (1, 2, 4 or
8 waves per page) on random, cancelling, spread, subnormal, zero and
tie-heavy rows, and requires every interval to contain the reference's
sequential float sum (src/reference_kernels.cpp:13-19) and the random rows'
intervals to be at least 10 times narrower than the first-pass bound.
Three plausible slips, planted in a copy of the header, must each make the
check fail."""
from __future__ import annotations

import pathlib
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
CSRC = ROOT / "15-618_dynamic_sparse_decode_amd" / "csrc"
SRC = ROOT / "tests" / "native" / "refine_check.cpp"
FLAGS = ["-std=c++17", "-O2", "-ffp-contract=off", "-Wall", "-Wextra"]


def build(tmp_path, include_dir, name):
    exe = tmp_path / name
    subprocess.run(["g++", *FLAGS, f"-I{include_dir}", str(SRC), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    return exe


def test_refined_intervals_contain_the_sequential_sum(tmp_path):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    exe = build(tmp_path, CSRC, "refine_check")
    proc = subprocess.run([str(exe), "60"], capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "refine_check ok" in proc.stdout


SLIPS = {
    # a tie on the grid taken as a known error (it depends on the last bit)
    "tie-as-known": [("const bool settled = first || (known && !tie);",
                      "const bool settled = first || known;"),
                     ("(known && !tie && small && !first)", "(known && small && !first)")],
    # the previous accumulator's binade not required to reach this grid
    "no-previous-binade": [(" && s.prev >= cert;", ";")],
    # half a spacing of one binade too small for the unknown steps
    "half-too-small": [("int fh = static_cast<int>(ehi) - 920;",
                        "int fh = static_cast<int>(ehi) - 921;")],
}


@pytest.mark.parametrize("slip", sorted(SLIPS))
def test_planted_slips_in_the_bound_are_caught(tmp_path, slip):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    text = (CSRC / "refine_lane.h").read_text()
    for old, new in SLIPS[slip]:
        assert old in text, old
        text = text.replace(old, new)
    mutated = tmp_path / "mut"
    mutated.mkdir()
    (mutated / "refine_lane.h").write_text(text)
    exe = build(tmp_path, mutated, "refine_check_" + slip)
    proc = subprocess.run([str(exe), "60"], capture_output=True, text=True, timeout=300)
    assert proc.returncode == 1, proc.stdout
    assert "MISS" in proc.stdout
