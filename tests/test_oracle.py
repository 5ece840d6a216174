"""Pins the CPU oracle (oracle/dsd_oracle.c) before it is trusted as checker.

1. Golden vectors: the reference's own sparse_cpu / dense_cpu outputs on the
   reference's test configurations (tests/golden/reference_cases.npz, written
   by tests/golden/make_golden.py from the reference's CPU code) -- bit-exact.
2. The reference's CPU units compiled here (oracle/_ref), on further seeds,
   when that build exists (build container only).
3. What the mathematics fixes: closed-form summaries, a brute-force top-k,
   textbook softmax attention in float64, the sparse == dense invariant,
   k = 0 and empty-context zeros, and the tie-break known answer.
"""
from __future__ import annotations

import ctypes
import pathlib

import numpy as np
import pytest

import _oracle as orc

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden" / "reference_cases.npz"


def load_cases():
    data = np.load(GOLDEN)
    cases = {}
    for key in data.files:
        name, field = key.split("/", 1)
        cases.setdefault(name, {})[field] = data[key]
    return cases


CASES = load_cases()
SMALL_CASES = sorted(n for n in CASES if n != "baseline_config2_uniform")


def unpack(case):
    H, D, ps, k, B, lo, hi, seed = (int(x) for x in case["config"])
    return H, D, ps, k, B


@pytest.mark.parametrize("name", SMALL_CASES)
def test_oracle_matches_reference_golden_bit_exact(name):
    c = CASES[name]
    H, D, ps, k, B = unpack(c)
    E = H * D
    scores, selected, outs = orc.sparse_batch(
        c["queries"], c["key_pool"], c["value_pool"], c["summaries"], c["token_counts"],
        c["cand_offsets"], c["cand_ids"], H, D, ps, k)
    assert scores.view(np.uint32).tolist() == c["ref_scores"].view(np.uint32).tolist()
    kk = max(k, 1)
    for r in range(B):
        cnt = int(c["ref_counts"][r])
        assert selected[r].tolist() == c["ref_selected"][r * kk:r * kk + cnt].tolist()
    assert np.array_equal(outs.reshape(-1).view(np.uint32), c["ref_sparse_out"].view(np.uint32))
    dense = orc.dense_batch(c["queries"], c["key_pool"], c["value_pool"], c["token_counts"],
                            c["cand_offsets"], c["cand_ids"], H, D, ps)
    assert np.array_equal(dense.reshape(-1).view(np.uint32), c["ref_dense_out"].view(np.uint32))


@pytest.mark.parametrize("name", SMALL_CASES)
def test_oracle_summaries_match_reference_cache(name):
    c = CASES[name]
    H, D, ps, k, B = unpack(c)
    E = H * D
    tc = c["token_counts"]
    mine = orc.pool_summaries(c["key_pool"], tc, E)
    ref = c["summaries"].reshape(len(tc), E)
    live = tc > 0
    assert np.array_equal(mine[live].view(np.uint32), ref[live].view(np.uint32))


def test_reference_context_lengths_match_reference_draws(dsd):
    big = CASES["baseline_config2_uniform"]
    lengths = dsd.reference_context_lengths(16, 512, 2048, 7)
    assert lengths == big["context_tokens"].tolist()
    assert lengths == [629, 861, 1710, 1002, 1185, 2015, 1623, 1212, 2015, 985, 1339, 917,
                       1282, 645, 622, 1156]
    assert sum((c + 15) // 16 for c in lengths) == 1207
    for name in SMALL_CASES:
        H, D, ps, k, B, lo, hi, seed = (int(x) for x in CASES[name]["config"])
        assert dsd.reference_context_lengths(B, lo, hi, seed) == \
            CASES[name]["context_tokens"].tolist()


def test_synthetic_batch_layout_matches_reference(dsd):
    """LIFO ids, logical candidate order and capacity as BuildSyntheticBatch."""
    c = CASES["sparse_ragged"]
    H, D, ps, k, B = unpack(c)
    batch = dsd.SyntheticBatch(H, D, ps, c["context_tokens"], seed=0)
    assert batch.capacity == len(c["token_counts"])
    assert batch.cand_offsets.tolist() == c["cand_offsets"].tolist()
    assert batch.cand_ids.tolist() == c["cand_ids"].tolist()
    assert batch.token_counts.tolist() == c["token_counts"].tolist()
    big = CASES["baseline_config2_uniform"]
    pages = [(x + 15) // 16 for x in big["context_tokens"].tolist()]
    ids = 1207 - 1 - np.arange(1207)
    assert np.cumsum([0] + pages).tolist() == big["cand_offsets"].tolist()
    assert ids.tolist() == big["cand_ids"].tolist()


# ---- against the reference binary compiled here (build container only) -------
REF = orc.REF_LIB


@pytest.mark.skipif(not REF.exists(), reason="oracle/_ref not built (no reference tree)")
@pytest.mark.parametrize("spec", [
    (2, 8, 4, 3, 5, 5, 40, 1), (4, 32, 16, 4, 3, 100, 300, 99), (1, 4, 1, 2, 2, 3, 9, 5),
    (8, 16, 8, 16, 4, 64, 512, 2024), (3, 12, 5, 7, 3, 20, 90, 77), (2, 128, 16, 64, 2, 600, 900, 3),
])
def test_oracle_matches_compiled_reference(spec):
    import importlib.util
    gen = importlib.util.spec_from_file_location(
        "make_golden", pathlib.Path(__file__).resolve().parent / "golden" / "make_golden.py")
    mg = importlib.util.module_from_spec(gen)
    gen.loader.exec_module(mg)
    ref = ctypes.CDLL(str(REF))
    H, D, ps, k, B, lo, hi, seed = spec
    c = mg.build_case(ref, (*spec, 0.0))
    scores, selected, outs = orc.sparse_batch(
        c["queries"], c["key_pool"], c["value_pool"], c["summaries"], c["token_counts"],
        c["cand_offsets"], c["cand_ids"], H, D, ps, k)
    assert np.array_equal(scores.view(np.uint32), c["ref_scores"].view(np.uint32))
    kk = max(k, 1)
    for r in range(B):
        cnt = int(c["ref_counts"][r])
        assert selected[r].tolist() == c["ref_selected"][r * kk:r * kk + cnt].tolist()
    assert np.array_equal(outs.reshape(-1).view(np.uint32), c["ref_sparse_out"].view(np.uint32))
    dense = orc.dense_batch(c["queries"], c["key_pool"], c["value_pool"], c["token_counts"],
                            c["cand_offsets"], c["cand_ids"], H, D, ps)
    assert np.array_equal(dense.reshape(-1).view(np.uint32), c["ref_dense_out"].view(np.uint32))


@pytest.mark.skipif(not REF.exists(), reason="oracle/_ref not built (no reference tree)")
@pytest.mark.parametrize("metadata_only", [0, 1])
def test_append_summary_matches_compiled_reference(metadata_only):
    # oracle_append_summary against the reference's own running mean
    # (PagedKvCache::AppendToken / AppendTokenMetadataOnly,
    # src/paged_kv_cache.cpp:231-238, 299-306): 29 decode tokens appended to
    # one request, fresh pages forced at two places, the summary of every page
    # it holds compared bit for bit.  A reciprocal multiply in place of the
    # division (a plausible slip) must not reproduce the reference.
    ref = ctypes.CDLL(str(REF))
    H, D, ps, cap, T = 2, 16, 5, 64, 29
    E = H * D
    rng = np.random.default_rng(17 + metadata_only)
    keys = rng.standard_normal((T, E)).astype(np.float32)
    keys[::7] *= np.float32(1e3)
    keys[3::11] *= np.float32(1e-3)
    values = rng.standard_normal((T, E)).astype(np.float32)
    force = np.zeros(T, np.uint8)
    force[[9, 17]] = 1
    summ = np.zeros((cap, E), np.float32)
    counts = np.zeros(cap, np.int32)
    fp = ctypes.POINTER(ctypes.c_float)
    ip = ctypes.POINTER(ctypes.c_int)
    ref.ref_append_tokens.restype = ctypes.c_int
    n = ref.ref_append_tokens(H, D, ps, cap, T, keys.ctypes.data_as(fp), values.ctypes.data_as(fp),
                              force.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)),
                              metadata_only, cap, summ.ctypes.data_as(fp), counts.ctypes.data_as(ip))
    # the same appends through the oracle (and through the slip)
    pages, slip = [], []
    for t in range(T):
        if force[t] or not pages or pages[-1][1] >= ps:
            pages.append([np.zeros(E, np.float32), 0])
            slip.append(np.zeros(E, np.float32))
        s, c = pages[-1]
        pages[-1][0] = orc.append_summary(s, keys[t], c)
        old, new = np.float32(c), np.float32(c + 1)
        slip[-1] = ((slip[-1] * old).astype(np.float32) + keys[t]).astype(np.float32) * \
            (np.float32(1.0) / new)
        pages[-1][1] = c + 1
    assert n == len(pages)
    assert counts[:n].tolist() == [c for _, c in pages]
    for j in range(n):
        assert np.array_equal(summ[j].view(np.uint32), pages[j][0].view(np.uint32)), j
    assert any(not np.array_equal(summ[j].view(np.uint32), slip[j].astype(np.float32).view(np.uint32))
               for j in range(n))


# ---- closed forms and invariants -------------------------------------------
def test_summary_closed_form_arithmetic_sequence():
    # test_reference.cpp:252-307 pattern: keys 1..(4*8); the per-element mean of
    # 4 rows of a step-1 sequence is exactly first_row + 12 (a power-of-two
    # count makes the host rule exact).
    E, T = 8, 4
    keys = np.arange(1, T * E + 1, dtype=np.float32)
    s = orc.page_summary(keys, T, E)
    assert s.tolist() == (np.arange(1, E + 1, dtype=np.float32) + 12.0).tolist()
    # zero tokens -> zeros
    assert orc.page_summary(keys, 0, E).tolist() == [0.0] * E


def test_summary_host_rule_is_reciprocal_multiply_not_division():
    # count 3: s = fl(sum) * fl(1/3); must differ from sum/3 somewhere and match
    # the explicit float32 restatement exactly.
    rng = np.random.default_rng(5)
    E, T = 4096, 3
    keys = rng.standard_normal((T, E)).astype(np.float32)
    acc = np.zeros(E, np.float32)
    for t in range(T):
        acc = (acc + keys[t]).astype(np.float32)
    expect = (acc * (np.float32(1.0) / np.float32(3.0))).astype(np.float32)
    got = orc.page_summary(keys, T, E)
    assert np.array_equal(got.view(np.uint32), expect.view(np.uint32))
    assert not np.array_equal(got, (acc / np.float32(3.0)).astype(np.float32))


def test_append_summary_closed_form():
    # paged_kv_cache.cpp:231-238 on the test_reference.cpp:140-210 sequences:
    # two prompt tokens then one appended token -> mean of three rows.
    E = 8
    k0 = np.arange(1, E + 1, dtype=np.float32)
    k1 = k0 + E
    k2 = np.arange(1001, 1001 + E, dtype=np.float32)
    s = orc.page_summary(np.concatenate([k0, k1]), 2, E)
    s = orc.append_summary(s, k2, 2)
    np.testing.assert_allclose(s, (k0 + k1 + k2) / 3.0, rtol=0, atol=1e-5)
    # explicit float32 restatement: (s*2 + k)/3 with separate roundings
    s0 = orc.page_summary(np.concatenate([k0, k1]), 2, E)
    expect = ((s0 * np.float32(2.0)).astype(np.float32) + k2).astype(np.float32) / np.float32(3.0)
    assert np.array_equal(s.view(np.uint32), expect.astype(np.float32).view(np.uint32))


def test_score_is_sequential_float32_chain():
    rng = np.random.default_rng(11)
    E, D = 64, 16
    q = rng.standard_normal(E).astype(np.float32)
    summ = rng.standard_normal((3, E)).astype(np.float32)
    got = orc.score_pages(q, summ, np.ones(3, np.int32), np.arange(3), D)
    sc = np.float32(1.0) / np.sqrt(np.float32(D))
    for p in range(3):
        acc = np.float32(0.0)
        for i in range(E):
            acc = np.float32(acc + np.float32(q[i] * summ[p, i]))
        assert got[p].view(np.uint32) == np.float32(acc * sc).view(np.uint32)


def test_select_topk_brute_force_and_tie_rules():
    rng = np.random.default_rng(3)
    for trial in range(200):
        n = int(rng.integers(0, 40))
        k = int(rng.integers(-1, 12))
        # many ties and signed zeros
        scores = rng.choice(np.array([-1.0, -0.0, 0.0, 0.5, 0.5, 2.0], np.float32), size=n)
        ids = rng.permutation(1000)[:n].astype(np.int32)
        got = orc.select_topk(scores, ids, k)
        order = sorted(range(n), key=lambda i: (-float(scores[i]) if scores[i] != 0 else 0.0,
                                                int(ids[i])))
        expect = [int(ids[i]) for i in order[:max(0, min(k, n))]] if k > 0 else []
        assert got.tolist() == expect


def test_tie_break_known_answer():
    # tests/test_sparse_cuda.cpp:134-169: 4 single-token pages, zero keys and a
    # zero query -> identical scores -> the smaller ids {0, 1} win.
    E = 4
    summ = np.zeros((4, E), np.float32)
    scores = orc.score_pages(np.zeros(E, np.float32), summ, np.ones(4, np.int32),
                             np.arange(4), 4)
    assert orc.select_topk(scores, np.arange(4), 2).tolist() == [0, 1]


def test_attention_matches_float64_softmax():
    rng = np.random.default_rng(8)
    H, D, ps, cap = 3, 16, 4, 6
    E = H * D
    kp = rng.standard_normal((cap, ps, E)).astype(np.float32)
    vp = rng.standard_normal((cap, ps, E)).astype(np.float32)
    tc = np.array([4, 2, 4, 1, 3, 4], np.int32)
    q = rng.standard_normal(E).astype(np.float32)
    pages = [4, 0, 3]
    got = orc.attention(q, kp, vp, tc, pages, H, D, ps)
    K = np.concatenate([kp[p, :tc[p]] for p in pages]).astype(np.float64)
    V = np.concatenate([vp[p, :tc[p]] for p in pages]).astype(np.float64)
    for h in range(H):
        sl = slice(h * D, (h + 1) * D)
        logits = K[:, sl] @ q[sl].astype(np.float64) / np.sqrt(D)
        w = np.exp(logits - logits.max())
        w /= w.sum()
        np.testing.assert_allclose(got[sl], w @ V[:, sl], atol=2e-6, rtol=0)
    assert orc.attention(q, kp, vp, tc, [], H, D, ps).tolist() == [0.0] * E


def test_sparse_equals_dense_when_topk_covers_all_pages():
    c = CASES["reference_topk_covers_all"]
    H, D, ps, k, B = unpack(c)
    _, _, outs = orc.sparse_batch(c["queries"], c["key_pool"], c["value_pool"], c["summaries"],
                                  c["token_counts"], c["cand_offsets"], c["cand_ids"], H, D, ps, k)
    dense = orc.dense_batch(c["queries"], c["key_pool"], c["value_pool"], c["token_counts"],
                            c["cand_offsets"], c["cand_ids"], H, D, ps)
    assert orc.max_abs_diff(outs, dense) <= 1e-5


def test_zero_topk_gives_zero_output_and_no_selection():
    c = CASES["sparse_zero_selection"]
    H, D, ps, k, B = unpack(c)
    _, selected, outs = orc.sparse_batch(c["queries"], c["key_pool"], c["value_pool"],
                                         c["summaries"], c["token_counts"], c["cand_offsets"],
                                         c["cand_ids"], H, D, ps, 0)
    assert all(len(s) == 0 for s in selected)
    assert not outs.any()


def test_max_abs_diff_size_mismatch_is_inf():
    assert orc.max_abs_diff(np.zeros(3), np.zeros(4)) == float("inf")


def test_planted_mistakes_are_caught():
    """Each check above would fail for a plausible slip: a dropped term, an
    off-by-one tie rule, a transposed operand."""
    c = CASES["sparse_ragged"]
    H, D, ps, k, B = unpack(c)
    E = H * D
    # dropped last summary element -> scores differ from the golden vector
    summ = c["summaries"].reshape(-1, E).copy()
    summ[:, -1] = 0.0
    s_bad, _, _ = orc.sparse_batch(c["queries"], c["key_pool"], c["value_pool"], summ,
                                   c["token_counts"], c["cand_offsets"], c["cand_ids"],
                                   H, D, ps, k)
    assert not np.array_equal(s_bad.view(np.uint32), c["ref_scores"].view(np.uint32))
    # tie rule flipped (larger id first) -> known answer breaks
    ids = np.arange(4)
    assert orc.select_topk(np.zeros(4, np.float32), ids[::-1].copy(), 2).tolist() == [0, 1]
    # K and V swapped -> outputs leave tolerance
    _, _, o_bad = orc.sparse_batch(c["queries"], c["value_pool"], c["key_pool"], c["summaries"],
                                   c["token_counts"], c["cand_offsets"], c["cand_ids"],
                                   H, D, ps, k)
    assert orc.max_abs_diff(o_bad, c["ref_sparse_out"]) > 1e-2


def test_request_step_equals_the_batched_oracle(dsd):
    """_oracle.request_step (one request from its own page arrays, as the
    full-size GPU tests stream them) selects and attends exactly as
    oracle_sparse_batch over the pool -- including the tie-break on the
    real page ids, which run opposite to the logical order here -- and its
    dense output equals oracle_dense_step's."""
    H, D, ps, k = 4, 16, 8, 3
    E = H * D
    batch = dsd.SyntheticBatch(H, D, ps, [70, 9, 33], seed=5)
    # two requests get duplicated summaries so that scores tie exactly
    kp = batch.key_pool
    r0 = batch.request_ids(0)
    kp[r0[1]] = kp[r0[4]]
    batch.token_counts[r0[1]] = batch.token_counts[r0[4]]
    summ = orc.pool_summaries(kp, batch.token_counts, E)
    _, sel_b, out_b = orc.sparse_batch(batch.queries, kp, batch.value_pool, summ,
                                       batch.token_counts, batch.cand_offsets,
                                       batch.cand_ids, H, D, ps, k)
    dense_b = orc.dense_batch(batch.queries, kp, batch.value_pool, batch.token_counts,
                              batch.cand_offsets, batch.cand_ids, H, D, ps)
    for r in range(batch.batch):
        ids = batch.request_ids(r)
        sel, out, dense = orc.request_step(batch.queries[r], kp[ids], batch.value_pool[ids],
                                           batch.token_counts[ids], ids, H, D, ps, k,
                                           dense=True)
        assert sel.tolist() == sel_b[r].tolist(), r
        assert np.array_equal(out.view(np.uint32), out_b[r].view(np.uint32)), r
        assert np.array_equal(dense.view(np.uint32), dense_b[r].view(np.uint32)), r
