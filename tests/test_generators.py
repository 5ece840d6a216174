"""The serving loop's generators, pinned to the reference.

* oracle_mt19937_draws is MT19937 (Matsumoto and Nishimura 1998): the C++
  standard's known answer ([rand.predef]: the 10000th output of a
  default-seeded std::mt19937 is 4123659995) and numpy's independent MT19937
  with the same seeding.
* oracle_mix_seed / oracle_token_vector restate MixSeed and
  DeterministicTokenVector (reference src/continuous_batching.cpp:44-59), the
  per-step decode payloads of the loop (queries, appended keys and values):
  equal bit for bit to the reference's own functions compiled in oracle/_ref.
* this build's BuildSyntheticContinuousWorkload (libdsd.so) against the
  reference's (src/continuous_batching.cpp:336-381): same requests, arrivals,
  lengths and the same bytes of every prompt key, value and initial query
  (FNV-1a fingerprints), at BASELINE config 5's counts.

The reference-backed checks need oracle/_ref (built where the reference tree
exists) and skip elsewhere."""
from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np
import pytest

import _oracle as orc

ROOT = pathlib.Path(__file__).resolve().parents[1]
NATIVE = ROOT / "tests" / "native"
REF = orc.REF_LIB
needs_ref = pytest.mark.skipif(not REF.exists(), reason="oracle/_ref not built (no reference tree)")


def draws(seed, n):
    out = np.empty(n, np.uint32)
    orc.lib().oracle_mt19937_draws(ctypes.c_uint32(seed), n, orc.P(out))
    return out


def token_vector(count, rid, step, stream):
    out = np.empty(count, np.float32)
    orc.lib().oracle_token_vector(count, rid, step, stream, orc.P(out))
    return out


def test_mt19937_known_answer_and_numpy():
    assert int(draws(5489, 10000)[-1]) == 4123659995
    for seed in (0, 1, 7, 5489, 0x9e3779b9, 0xffffffff):
        bg = np.random.MT19937()
        bg._legacy_seeding(seed)
        expect = np.array([bg.random_raw() for _ in range(1500)], np.uint64).astype(np.uint32)
        assert np.array_equal(draws(seed, 1500), expect), seed


def test_token_vectors_lie_in_the_open_range():
    v = token_vector(100000, 3, 4, 1)
    assert v.min() >= -1.0 and v.max() < 1.0
    assert abs(float(v.mean())) < 0.01
    assert not np.array_equal(v[:50], token_vector(50, 3, 4, 2))   # stream enters
    assert not np.array_equal(v[:50], token_vector(50, 3, 5, 1))   # step enters
    assert not np.array_equal(v[:50], token_vector(50, 4, 4, 1))   # request enters


@needs_ref
def test_token_vectors_equal_the_references():
    ref = ctypes.CDLL(str(REF))
    ref.ref_mix_seed.restype = ctypes.c_uint
    orc.lib().oracle_mix_seed.restype = ctypes.c_uint32
    for rid, step, stream in [(0, 0, 0), (0, 1, 0), (5, 3, 1), (5, 3, 2), (127, 63, 0),
                              (127, 64, 2), (1 << 20, 7, 1), (2147483647, 2147483647, 2)]:
        assert ref.ref_mix_seed(rid, step, stream) == orc.lib().oracle_mix_seed(rid, step, stream)
        n = 4096
        want = np.empty(n, np.float32)
        ref.ref_token_vector(n, rid, step, stream, want.ctypes.data_as(ctypes.c_void_p))
        got = token_vector(n, rid, step, stream)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (rid, step, stream)


def ref_workload(heads, head_dim, ps, k, n, window, pmin, pmax, dmin, dmax, seed):
    ref = ctypes.CDLL(str(REF))
    meta = np.zeros((n, 4), np.int32)
    hashes = np.zeros((n, 3), np.uint64)
    got = ref.ref_workload_hashes(heads, head_dim, ps, k, n, window, pmin, pmax, dmin, dmax,
                                  seed, meta.ctypes.data_as(ctypes.c_void_p),
                                  hashes.ctypes.data_as(ctypes.c_void_p))
    assert got == n
    return [tuple(int(x) for x in meta[i]) + tuple(int(x) for x in hashes[i]) for i in range(n)]


def our_workload(*args):
    subprocess.run(["make", "-s", "-C", str(NATIVE), "build/workload_dump"], check=True)
    out = subprocess.run([str(NATIVE / "build" / "workload_dump"), *map(str, args)],
                         capture_output=True, text=True, check=True, timeout=600).stdout
    return [tuple(int(x) for x in line.split()) for line in out.strip().splitlines()]


@needs_ref
@pytest.mark.parametrize("args", [
    # BASELINE config 5's counts (128 requests, window 64, prompts 1024-4096,
    # decode 16-64, seed 7) with a narrow token row, so the prompts stay small
    (2, 8, 16, 8, 128, 64, 1024, 4096, 16, 64, 7),
    # config 5's token row (32 x 128) on a few short requests
    (32, 128, 16, 8, 3, 4, 1, 40, 1, 5, 7),
    # the reference test's workload (tests/test_continuous_batching.cpp:124)
    (2, 4, 4, 2, 5, 2, 0, 7, 1, 3, 123),
])
def test_continuous_workload_equals_the_references(args):
    assert our_workload(*args) == ref_workload(*args)


# ---- the N(0, 1) payload mode (DSD_PAYLOAD_DIST=normal) ------------------------
# BASELINE config 5 states N(0, 1) K/V; the reference's generator is
# U(-1, 1) and stays the default.  In the N(0, 1) mode the workload's
# arrivals, prompt lengths and decode counts must still be the reference's
# (the reference stream advances past each payload as before), and every
# payload must equal the oracle's Box-Muller restatement
# (oracle_prompt_normal, oracle_token_vector_normal).

def fnv1a(a):
    h = 1469598103934665603
    for byte in np.ascontiguousarray(a, np.float32).tobytes():
        h = ((h ^ byte) * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return h


def normal_workload(*args, tokens=False):
    import os
    subprocess.run(["make", "-s", "-C", str(NATIVE), "build/workload_dump"], check=True)
    env = dict(os.environ, DSD_PAYLOAD_DIST="normal")
    cmd = [str(NATIVE / "build" / "workload_dump"), *map(str, args)] + (["tokens"] if tokens else [])
    out = subprocess.run(cmd, capture_output=True, text=True, check=True, timeout=600,
                         env=env).stdout
    rows = [line.split() for line in out.strip().splitlines()]
    return ([tuple(int(x) for x in r) for r in rows if r[0] != "T"],
            [tuple(int(x) for x in r[1:]) for r in rows if r[0] == "T"])


@needs_ref
def test_normal_payload_mode_keeps_the_reference_workload_shape():
    args = (2, 8, 16, 8, 128, 64, 1024, 4096, 16, 64, 7)
    got, _ = normal_workload(*args)
    want = ref_workload(*args)
    assert [g[:4] for g in got] == [w[:4] for w in want]
    # the payloads themselves differ from the U(-1, 1) ones
    assert all(g[4] != w[4] for g, w in zip(got[:8], want[:8]))


def test_normal_payloads_equal_the_oracle_restatement():
    H, D, seed = 2, 8, 7
    E = H * D
    args = (H, D, 16, 8, 16, 8, 16, 64, 1, 5, seed)
    specs, tokens = normal_workload(*args, tokens=True)
    lib = orc.lib()
    for rid, arrival, prompt, decode, hk, hv, hq in specs:
        keys = np.empty(prompt * E, np.float32)
        values = np.empty(prompt * E, np.float32)
        query = np.empty(E, np.float32)
        lib.oracle_prompt_normal(seed, rid, prompt, E, orc.P(keys), orc.P(values), orc.P(query))
        assert (fnv1a(keys), fnv1a(values), fnv1a(query)) == (hk, hv, hq), rid
    assert len(tokens) == 5
    for rid, step, stream, h in tokens:
        v = np.empty(E, np.float32)
        lib.oracle_token_vector_normal(E, rid, step, stream, orc.P(v))
        assert fnv1a(v) == h, (rid, step, stream)
    # the restatement is N(0, 1): moments of a long draw
    big = np.empty(200000, np.float32)
    lib.oracle_token_vector_normal(len(big), 3, 4, 1, orc.P(big))
    assert abs(float(big.mean())) < 0.01 and abs(float(big.std()) - 1.0) < 0.01
    assert abs(float(np.mean(np.abs(big))) - np.sqrt(2.0 / np.pi)) < 0.01
