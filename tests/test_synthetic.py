"""The benchmark's synthetic batch generator (dsd_synthetic_batch,
SyntheticBatch.reference): the reference's BuildSyntheticBatch draw order
(src/synthetic_data.cpp:23-68).

* U(-1, 1) mode against the reference's own batches: every golden case
  (tests/golden/reference_cases.npz, written through the compiled
  reference) must come out bit for bit: lengths, page ids, key and value
  pools, queries.
* N(0, 1) mode against a restatement of libstdc++'s
  std::normal_distribution<float> (the Marsaglia polar method, pairs cached
  per distribution object) on the raw std::mt19937 outputs (numpy's MT19937
  with the legacy seeding), with glibc's logf through ctypes, on small
  batches, bit for bit.  A planted slip (the pair's two values returned in
  the other order) must fail."""
from __future__ import annotations

import ctypes
import ctypes.util

import numpy as np
import pytest

GOLDEN = np.load(__import__("pathlib").Path(__file__).resolve().parent / "golden" /
                 "reference_cases.npz")
LIBM = ctypes.CDLL(ctypes.util.find_library("m"))
LIBM.logf.restype = ctypes.c_float
LIBM.logf.argtypes = [ctypes.c_float]
F = np.float32


def canonical(bg):
    """generate_canonical<float, 24> on a 32-bit engine: one output."""
    u = F(float(int(bg.random_raw()))) / F(4294967296.0)
    return u if u < F(1.0) else np.nextafter(F(1.0), F(0.0))


def normals(bg, n, swap=False):
    """n values from one std::normal_distribution<float>(0, 1) object."""
    out, saved = [], None
    while len(out) < n:
        if saved is not None:
            out.append(saved)
            saved = None
            continue
        while True:
            # float(2) * u - 1.0 is evaluated in double, then stored as float
            x = F(float(F(2.0) * canonical(bg)) - 1.0)
            y = F(float(F(2.0) * canonical(bg)) - 1.0)
            r2 = F(F(x * x) + F(y * y))
            if not (r2 > 1.0 or r2 == 0.0):
                break
        mult = np.sqrt(F(F(F(-2.0) * F(LIBM.logf(float(r2)))) / r2))
        first, second = F(y * mult), F(x * mult)
        if swap:
            first, second = second, first
        out.append(F(first * F(1.0) + F(0.0)))
        saved = F(second * F(1.0) + F(0.0))
    return np.array(out, np.float32)


def restated_normal_batch(gpu, H, D, ps, B, lo, hi, seed, swap=False):
    lengths = gpu.reference_context_lengths(B, lo, hi, seed)
    bg = np.random.MT19937()
    bg._legacy_seeding(seed)
    E = H * D
    # advance past the length draws exactly as reference_context_lengths does
    gpu_lengths = []
    span = hi - lo + 1
    for _ in range(B):
        prod = int(bg.random_raw()) * span
        low = prod & 0xFFFFFFFF
        if low < span:
            threshold = ((1 << 32) - span) % span
            while low < threshold:
                prod = int(bg.random_raw()) * span
                low = prod & 0xFFFFFFFF
        gpu_lengths.append(lo + (prod >> 32))
    assert gpu_lengths == list(lengths)
    pages = sum(-(-n // ps) for n in lengths)
    kp = np.zeros((pages, ps, E), np.float32)
    vp = np.zeros_like(kp)
    q = np.zeros((B, E), np.float32)
    g = 0
    for r, n in enumerate(lengths):
        for j in range(-(-n // ps)):
            t = min(ps, n - j * ps)
            row = pages - 1 - g
            kp[row, :t] = normals(bg, t * E, swap).reshape(t, E)
            vp[row, :t] = normals(bg, t * E, swap).reshape(t, E)
            g += 1
        q[r] = normals(bg, E, swap)
    return lengths, kp, vp, q


CASES = sorted({k.split("/")[0] for k in GOLDEN.files if not k.startswith("baseline")})


@pytest.mark.parametrize("name", CASES)
def test_uniform_mode_is_the_reference_batch(dsd, name):
    H, D, ps, k, B, lo, hi, seed = [int(x) for x in GOLDEN[f"{name}/config"]]
    b = dsd.SyntheticBatch.reference(H, D, ps, B, lo, hi, seed, "uniform")
    assert b.context_lengths == GOLDEN[f"{name}/context_tokens"].tolist()
    assert b.cand_ids.tolist() == GOLDEN[f"{name}/cand_ids"].tolist()
    for mine, key in ((b.key_pool, "key_pool"), (b.value_pool, "value_pool"),
                      (b.queries, "queries")):
        assert np.array_equal(mine.reshape(-1).view(np.uint32),
                              GOLDEN[f"{name}/{key}"].view(np.uint32)), key


@pytest.mark.parametrize("shape", [(2, 4, 4, 3, 1, 9, 5), (1, 8, 2, 2, 3, 7, 11)])
def test_normal_mode_is_the_polar_method_on_the_reference_engine(dsd, shape):
    H, D, ps, B, lo, hi, seed = shape
    b = dsd.SyntheticBatch.reference(H, D, ps, B, lo, hi, seed, "normal")
    lengths, kp, vp, q = restated_normal_batch(dsd, H, D, ps, B, lo, hi, seed)
    assert b.context_lengths == list(lengths)
    for mine, want in ((b.key_pool, kp), (b.value_pool, vp), (b.queries, q)):
        assert np.array_equal(mine.view(np.uint32), want.view(np.uint32))
    # a planted slip: the cached value handed out first
    _, kp2, _, _ = restated_normal_batch(dsd, H, D, ps, B, lo, hi, seed, swap=True)
    assert not np.array_equal(b.key_pool.view(np.uint32), kp2.view(np.uint32))
