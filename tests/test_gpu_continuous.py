"""BASELINE config 5 through the serving loop, checked step by step against
the oracle (tests/native/continuous_check.cpp).

    128 requests, at most 32 active, arrivals over a 64-step window,
    prompts U[1024, 4096], decode U[16, 64], 32 x 128, page 16, top-k 8,
    direct GPU upload admission, lazy release off, seed 7

The loop runs as the reference's RunContinuousSparseDecode
(src/continuous_batching.cpp:392-741) is run: its workload is the
reference's BuildSyntheticContinuousWorkload (pinned bit for bit in
tests/test_generators.py) and its decode tokens come from the reference's
DeterministicTokenVector, U(-1, 1).  Every 7th step's requests are rebuilt
independently from those generators and the oracle's sparse_cpu rows must
give the same selection (id for id) and outputs within 1e-4.  Both ways of
holding the next query are covered: generated in the loop (into the
pipelined loop's pinned payload slabs, or copied into the step's staging
when the host waits for every step) and precomputed into pinned rows the
step reads in place.
The third case runs the loop on BASELINE config 5's own data: N(0, 1)
prompts, decode K/V and queries (DSD_PAYLOAD_DIST=normal), rebuilt by the
oracle's restatement of that generator."""
from __future__ import annotations

import os
import pathlib
import re
import subprocess

import pytest

pytestmark = pytest.mark.gpu

EXE = pathlib.Path(__file__).resolve().parent / "native" / "build" / "continuous_check"
CONFIG5 = ["128", "32", "64", "1024", "4096", "16", "64", "7", "32", "128", "16", "8"]


@pytest.mark.parametrize("precompute,dist,pipeline", [("0", "uniform", "1"), ("1", "uniform", "1"),
                                                      ("0", "normal", "1"), ("0", "uniform", "0")])
def test_config5_serving_loop_steps_match_the_oracle(gpu, precompute, dist, pipeline):
    # dist "normal": BASELINE config 5's own data, N(0, 1) prompts, decode K/V
    # and queries (DSD_PAYLOAD_DIST=normal); the reference's U(-1, 1) is the
    # default.  pipeline "1" (the default): unobserved steps, their appends
    # and releases are enqueued without host waits; "0" (DSD_PIPELINE=0):
    # the host waits for every step.
    if not EXE.exists():
        pytest.fail(f"{EXE} is not built (__graft_entry__.build() builds tests/native)")
    print(f"[continuous_check] config 5, every 7th step, precompute={precompute}, "
          f"payloads {dist}, pipeline {pipeline}", flush=True)
    env = dict(os.environ, DSD_PAYLOAD_DIST=dist, DSD_PIPELINE=pipeline)
    proc = subprocess.run([str(EXE), *CONFIG5, "7", precompute], capture_output=True,
                          text=True, timeout=900, env=env)
    out = proc.stdout + proc.stderr
    assert proc.returncode == 0, out[-4000:]
    summary = re.search(r"continuous check: (\d+) steps, (\d+) request-steps, max abs diff "
                        r"(\S+), (\d+) failures", out)
    assert summary is not None, out[-4000:]
    loop = re.search(r"loop: .*", out)
    print(loop.group(0) if loop else "", summary.group(0), sep="\n", flush=True)
    steps, request_steps, diff, failures = summary.groups()
    assert int(failures) == 0 and int(steps) >= 10 and int(request_steps) >= 200, out[-4000:]
    assert float(diff) <= 1e-4
