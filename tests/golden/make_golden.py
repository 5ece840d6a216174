"""Writes tests/golden/reference_cases.npz from the reference's own CPU code.

Run in the build container only (it needs oracle/_ref/libdsd_ref.so, which
oracle/Makefile compiles from /root/reference).  For each test configuration
the reference's tests use (tests/test_sparse_cuda.cpp:120-132,217-251,
tests/test_dense_cuda.cpp:373-431, tests/test_reference.cpp:379-386) it calls
BuildSyntheticBatch (src/synthetic_data.cpp:23-68) and records the inputs and
the reference's sparse_cpu (src/decode_pipeline.cpp:13-46) and dense_cpu
(src/reference_kernels.cpp:196-203) outputs.  The fixture is data only.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import ctypes
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parent.parent
REF_LIB = ROOT / "oracle" / "_ref" / "libdsd_ref.so"

# name: (heads, head_dim, page_size, top_k, batch, min_ctx, max_ctx, seed, tolerance)
CASES = {
    "sparse_small": (2, 8, 4, 2, 3, 5, 19, 11, 1e-5),          # test_sparse_cuda.cpp:217-227
    "sparse_ragged": (4, 16, 16, 3, 4, 33, 97, 7, 2e-5),       # :229-239
    "sparse_wide": (2, 64, 8, 4, 2, 17, 45, 17, 5e-5),         # :241-251
    "sparse_large_candidates": (2, 16, 8, 8, 2, 160, 184, 123, 3e-5),  # :120-132
    "sparse_zero_selection": (2, 16, 8, 0, 1, 9, 9, 41, 1e-6),  # :86-118
    "reference_topk_covers_all": (2, 8, 4, 64, 3, 12, 12, 123, 1e-5),  # test_reference.cpp:379-399
    "dense_small": (2, 8, 4, 8, 3, 5, 19, 11, 1e-5),           # test_dense_cuda.cpp:373-383
    "dense_ragged": (4, 16, 16, 8, 5, 33, 97, 7, 2e-5),        # :385-395
    "dense_wide": (2, 64, 8, 16, 4, 17, 45, 17, 5e-5),         # :397-407
    "dense_very_wide": (2, 80, 8, 16, 4, 17, 45, 19, 5e-5),    # :409-419
    "dense_max_width": (2, 128, 8, 16, 2, 9, 25, 29, 1e-4),    # :421-431
    "no_output_fast_path": (2, 16, 8, 4, 2, 32, 48, 88, 1e-5),  # test_sparse_cuda.cpp:171-205
}


def P(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def build_case(ref, spec):
    H, D, ps, k, B, lo, hi, seed, tol = spec
    ref.ref_batch_build.restype = ctypes.c_void_p
    h = ctypes.c_void_p(ref.ref_batch_build(H, D, ps, k, B, lo, hi, seed))
    cap, tot = ctypes.c_int(), ctypes.c_int()
    ref.ref_batch_info(h, ctypes.byref(cap), ctypes.byref(tot))
    E, cap, tot = H * D, cap.value, tot.value
    ctx = np.zeros(B, np.int32)
    off = np.zeros(B + 1, np.int32)
    ids = np.zeros(max(tot, 1), np.int32)
    tc = np.zeros(cap, np.int32)
    kp = np.zeros(cap * ps * E, np.float32)
    vp = np.zeros_like(kp)
    sm = np.zeros(cap * E, np.float32)
    q = np.zeros(B * E, np.float32)
    ref.ref_batch_get(h, P(ctx), P(off), P(ids), P(tc), P(kp), P(vp), P(sm), P(q))
    kk = max(k, 1)
    scores = np.zeros(max(tot, 1), np.float32)
    sel = np.full(B * kk, -1, np.int32)
    counts = np.zeros(B, np.int32)
    sparse_out = np.zeros(B * E, np.float32)
    ref.ref_batch_sparse_cpu(h, P(scores), P(sel), P(counts), P(sparse_out))
    dense_out = np.zeros(B * E, np.float32)
    ref.ref_batch_dense_cpu(h, P(dense_out))
    ref.ref_batch_free(h)
    return {
        "config": np.array([H, D, ps, k, B, lo, hi, seed], np.int64),
        "tolerance": np.array(tol, np.float64),
        "context_tokens": ctx, "cand_offsets": off, "cand_ids": ids[:tot],
        "token_counts": tc, "key_pool": kp, "value_pool": vp, "summaries": sm,
        "queries": q, "ref_scores": scores[:tot], "ref_selected": sel,
        "ref_counts": counts, "ref_sparse_out": sparse_out, "ref_dense_out": dense_out,
    }


def main() -> int:
    if not REF_LIB.exists():
        print(f"{REF_LIB} missing: run `make -C oracle ref` first", file=sys.stderr)
        return 1
    ref = ctypes.CDLL(str(REF_LIB))
    arrays = {}
    for name, spec in CASES.items():
        for key, value in build_case(ref, spec).items():
            arrays[f"{name}/{key}"] = value
    # Config-2 shape under the reference draw order (U(-1,1), 32x128, ps16,
    # k8, B=16, ctx 512-2048, seed 7): context lengths, candidate ids and the
    # reference's selections only (its payloads are ~630 MB).
    big = build_case(ref, (32, 128, 16, 8, 16, 512, 2048, 7, 1e-4))
    for key in ("config", "context_tokens", "cand_offsets", "cand_ids", "ref_selected",
                "ref_counts"):
        arrays[f"baseline_config2_uniform/{key}"] = big[key]
    out = HERE / "reference_cases.npz"
    np.savez_compressed(out, **arrays)
    print(f"wrote {out} ({out.stat().st_size / 1024:.0f} KiB, {len(CASES)} cases)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
