"""Certified scoring (the default selection path) against the oracle.

The certified kernels never compute the reference's sequential score for
most pages; they bound it.  These tests pin the two claims that make the
selection exact: (1) every interval contains the exact sparse_cpu score,
(2) the selected ids equal sparse_cpu's, including inputs built so that
intervals overlap and the exact fallback must decide (permuted summaries:
same products in another order, so the sequential sums differ only by
rounding; duplicated summaries: exactly equal scores)."""
from __future__ import annotations

import os

import numpy as np
import pytest

import _oracle as orc

pytestmark = pytest.mark.gpu


def selected_total(offsets, k):
    return int(sum(min(k, int(n)) for n in np.diff(offsets)))


def run_both_paths(gpu, pool, queries, offs, ids, k):
    total = int(offs[-1])
    with gpu.SparseContext(pool, k, len(offs) - 1, total, selected_total(offs, k)) as ctx:
        cert = ctx.run_batch(queries, offs, ids, output_mode=gpu.OUTPUT_OUTPUTS, want_ids=True)
        bounds = ctx.score_bounds(total)
        rescored = ctx.exact_rescored_pages()
        exact = ctx.run_batch(queries, offs, ids, output_mode=gpu.OUTPUT_DEBUG)
    return cert, bounds, rescored, exact


@pytest.mark.parametrize("seed", [7, 8, 9, 10, 11])
def test_certified_config2_matches_exact_and_oracle(gpu, seed):
    lengths = gpu.reference_context_lengths(16, 512, 2048, seed)
    batch = gpu.SyntheticBatch(32, 128, 16, lengths, seed=seed)
    pool = gpu.DevicePagePool(32, 128, 16, batch.capacity)
    batch.upload(pool)
    cert, (mid, lo, hi), rescored, exact = run_both_paths(
        gpu, pool, batch.queries, batch.cand_offsets, batch.cand_ids, 8)
    ex = exact["scores"]
    assert np.all(lo <= ex) and np.all(ex <= hi), "an interval misses the exact score"
    assert np.all(lo <= mid) and np.all(mid <= hi)
    for r in range(batch.batch):
        assert cert["selected"][r].tolist() == exact["selected"][r].tolist(), (seed, r)
    assert np.array_equal(cert["outputs"].view(np.uint32), exact["outputs"].view(np.uint32))
    # against the oracle as well
    summ = np.zeros((batch.capacity, 4096), np.float32)
    live = batch.live_page_ids()
    summ[live] = orc.pool_summaries(batch.key_pool, batch.token_counts, 4096, live)
    _, selected, outs = orc.sparse_batch(batch.queries, batch.key_pool, batch.value_pool, summ,
                                         batch.token_counts, batch.cand_offsets, batch.cand_ids,
                                         32, 128, 16, 8)
    for r in range(batch.batch):
        assert cert["selected"][r].tolist() == selected[r].tolist()
    assert orc.max_abs_diff(cert["outputs"], outs) <= 1e-4
    pool.close()


@pytest.mark.parametrize("H,D,ps,k,lengths", [
    (4, 16, 16, 3, [33, 97, 60, 41]),       # E = 64: generic certified kernel
    (2, 64, 8, 4, [17, 45, 30]),             # E = 128
    (8, 32, 4, 16, [400, 250, 3]),           # k > 16
    (32, 128, 64, 32, [4100, 9000]),         # page 64, k 32
])
def test_certified_small_shapes_match_oracle(gpu, H, D, ps, k, lengths):
    batch = gpu.SyntheticBatch(H, D, ps, lengths, seed=sum(lengths))
    E = H * D
    pool = gpu.DevicePagePool(H, D, ps, batch.capacity)
    batch.upload(pool)
    cert, (mid, lo, hi), _, exact = run_both_paths(gpu, pool, batch.queries, batch.cand_offsets,
                                                   batch.cand_ids, k)
    assert np.all(lo <= exact["scores"]) and np.all(exact["scores"] <= hi)
    summ = np.zeros((batch.capacity, E), np.float32)
    live = batch.live_page_ids()
    summ[live] = orc.pool_summaries(batch.key_pool, batch.token_counts, E, live)
    _, selected, outs = orc.sparse_batch(batch.queries, batch.key_pool, batch.value_pool, summ,
                                         batch.token_counts, batch.cand_offsets, batch.cand_ids,
                                         H, D, ps, k)
    for r in range(batch.batch):
        assert cert["selected"][r].tolist() == selected[r].tolist(), r
    assert orc.max_abs_diff(cert["outputs"], outs) <= 1e-4


def adversarial_pool(gpu, rng, H=32, D=128, ps=16, groups=6, copies=4):
    """Pages whose summaries are permutations / copies of a few base rows."""
    E = H * D
    cap = groups * copies
    keys = np.empty((cap, ps, E), np.float32)
    base = rng.standard_normal((groups, ps, E)).astype(np.float32)
    for g in range(groups):
        for c in range(copies):
            p = g * copies + c
            if c == 0 or c == 3:
                keys[p] = base[g]                      # identical summaries -> exact ties
            else:
                perm = rng.permutation(E)               # same multiset of values,
                keys[p] = base[g][:, perm]              # other order
    values = rng.standard_normal((cap, ps, E)).astype(np.float32)
    pool = gpu.DevicePagePool(H, D, ps, cap)
    ids = np.arange(cap, dtype=np.int32)
    pool.upload_pages(ids, np.full(cap, ps, np.int32), ids.astype(np.int64) * ps * E, keys, values)
    return pool, keys, values


def test_certified_adversarial_near_ties_take_the_exact_path(gpu):
    rng = np.random.default_rng(99)
    H, D, ps = 32, 128, 16
    E = H * D
    pool, keys, values = adversarial_pool(gpu, rng)
    cap = keys.shape[0]
    # queries constant within permutation groups make permuted pages' scores
    # equal in exact arithmetic; a second query is generic.
    q = np.stack([np.full(E, 0.37, np.float32), rng.standard_normal(E).astype(np.float32)])
    cand = rng.permutation(cap).astype(np.int32)
    offs = np.array([0, cap, 2 * cap], np.int32)
    ids = np.concatenate([cand, cand[::-1]]).astype(np.int32)
    for k in (1, 3, 5, 8, 13):
        cert, (mid, lo, hi), rescored, exact = run_both_paths(gpu, pool, q, offs, ids, k)
        assert np.all(lo <= exact["scores"]) and np.all(exact["scores"] <= hi)
        summ = orc.pool_summaries(keys, np.full(cap, ps, np.int32), E)
        _, selected, outs = orc.sparse_batch(q, keys, values, summ, np.full(cap, ps, np.int32),
                                             offs, ids, H, D, ps, k)
        for r in range(2):
            assert cert["selected"][r].tolist() == selected[r].tolist(), (k, r)
            assert exact["selected"][r].tolist() == selected[r].tolist(), (k, r)
        assert orc.max_abs_diff(cert["outputs"], outs) <= 1e-4
        assert rescored > 0, "near ties should have needed the exact chain"


def test_certified_all_zero_query_ties_resolve_by_page_id(gpu):
    # Every score is exactly +0: all intervals overlap, every relevant page is
    # rescored, and the smallest ids win (test_sparse_cuda.cpp:134-169 at scale).
    rng = np.random.default_rng(5)
    pool, keys, values = adversarial_pool(gpu, rng, groups=3, copies=4)
    cap = keys.shape[0]
    cand = rng.permutation(cap).astype(np.int32)
    with gpu.SparseContext(pool, 4, 1, cap, 4) as ctx:
        res = ctx.run_batch(np.zeros((1, 4096), np.float32), np.array([0, cap], np.int32), cand,
                            output_mode=gpu.OUTPUT_OUTPUTS, want_ids=True)
    assert res["selected"][0].tolist() == [0, 1, 2, 3]


def test_certified_large_requests_match_oracle(gpu):
    # More than 256 candidates per request: the bitonic certified select
    # (up to 2048 candidates), random data, k = 64.
    lengths = [5000, 32768]                       # 313 and 2048 pages of 16
    batch = gpu.SyntheticBatch(32, 128, 16, lengths, seed=41)
    pool = gpu.DevicePagePool(32, 128, 16, batch.capacity)
    batch.upload(pool)
    k = 64
    cert, (mid, lo, hi), _, exact = run_both_paths(gpu, pool, batch.queries, batch.cand_offsets,
                                                   batch.cand_ids, k)
    assert np.all(lo <= exact["scores"]) and np.all(exact["scores"] <= hi)
    summ = np.zeros((batch.capacity, 4096), np.float32)
    live = batch.live_page_ids()
    summ[live] = orc.pool_summaries(batch.key_pool, batch.token_counts, 4096, live)
    _, selected, outs = orc.sparse_batch(batch.queries, batch.key_pool, batch.value_pool, summ,
                                         batch.token_counts, batch.cand_offsets, batch.cand_ids,
                                         32, 128, 16, k)
    for r in range(batch.batch):
        assert cert["selected"][r].tolist() == selected[r].tolist(), r
        assert exact["selected"][r].tolist() == selected[r].tolist(), r
    assert orc.max_abs_diff(cert["outputs"], outs) <= 1e-4
    pool.close()


@pytest.mark.parametrize("k", [40, 100])
def test_certified_large_request_many_flags(gpu, k):
    # 320 candidates in one request built from permuted and duplicated rows,
    # with a constant query: hundreds of overlapping intervals, so the exact
    # chain runs in several groups of pages.
    rng = np.random.default_rng(7 + k)
    H, D, ps = 32, 128, 16
    E = H * D
    pool, keys, values = adversarial_pool(gpu, rng, groups=80, copies=4)
    cap = keys.shape[0]
    q = np.stack([np.full(E, 0.37, np.float32)])
    ids = rng.permutation(cap).astype(np.int32)
    offs = np.array([0, cap], np.int32)
    cert, (mid, lo, hi), rescored, exact = run_both_paths(gpu, pool, q, offs, ids, k)
    assert np.all(lo <= exact["scores"]) and np.all(exact["scores"] <= hi)
    summ = orc.pool_summaries(keys, np.full(cap, ps, np.int32), E)
    _, selected, outs = orc.sparse_batch(q, keys, values, summ, np.full(cap, ps, np.int32),
                                         offs, ids, H, D, ps, k)
    assert cert["selected"][0].tolist() == selected[0].tolist()
    assert exact["selected"][0].tolist() == selected[0].tolist()
    assert orc.max_abs_diff(cert["outputs"], outs) <= 1e-4
    assert rescored > 32, "expected several chain groups"
    pool.close()


def extreme_summaries(kind, rng, cap, E):
    """Summary rows that strain the float error bound of the certified score."""
    if kind == "cancel":        # partial sums swing by 1e4, scores end near 0
        sign = np.where(np.arange(E) % 2 == 0, 1.0, -1.0)
        rows = 1e4 * sign + 1e-3 * rng.standard_normal((cap, E))
    elif kind == "grow_cancel":  # the first half climbs, the second half cancels it
        sign = np.where(np.arange(E) < E // 2, 1.0, -1.0)
        rows = 3e3 * sign * (1.0 + 1e-4 * rng.standard_normal((cap, E)))
    elif kind == "wide_range":   # magnitudes 1e-22 .. 1e16, random signs
        rows = 10.0 ** rng.uniform(-22, 16, (cap, E)) * rng.choice([-1.0, 1.0], (cap, E))
    elif kind == "subnormal":    # products in the subnormal range (|q s| ~ 1e-44 .. 1e-40)
        rows = 10.0 ** rng.uniform(-23, -21, (cap, E)) * rng.choice([-1.0, 1.0], (cap, E))
    else:
        raise ValueError(kind)
    return rows.astype(np.float32)


@pytest.mark.parametrize("kind", ["cancel", "grow_cancel", "wide_range", "subnormal"])
def test_certified_intervals_hold_on_extreme_summaries(gpu, kind):
    # Summary rows are uploaded verbatim (not key means), so scores can be
    # dominated by cancellation, span 38 orders of magnitude, or be built
    # from subnormal products.  Every interval must still contain the exact
    # sequential score, and the selection must equal sparse_cpu's.
    rng = np.random.default_rng({"cancel": 1, "grow_cancel": 2, "wide_range": 3,
                                 "subnormal": 4}[kind])
    H, D, ps, cap = 32, 128, 16, 96
    E = H * D
    summ = extreme_summaries(kind, rng, cap, E)
    keys = rng.standard_normal((cap, ps, E)).astype(np.float32)
    values = rng.standard_normal((cap, ps, E)).astype(np.float32)
    pool = gpu.DevicePagePool(H, D, ps, cap)
    page_ids = np.arange(cap, dtype=np.int32)
    pool.upload_pages(page_ids, np.full(cap, ps, np.int32), page_ids.astype(np.int64) * ps * E,
                      keys, values, summ)
    if kind == "wide_range":
        q = (10.0 ** rng.uniform(-22, 16, (2, E)) * rng.choice([-1.0, 1.0], (2, E)))
    elif kind == "subnormal":
        q = 10.0 ** rng.uniform(-23, -21, (2, E)) * rng.choice([-1.0, 1.0], (2, E))
    else:
        q = 1.0 + 1e-3 * rng.standard_normal((2, E))
    q = q.astype(np.float32)
    cand = rng.permutation(cap).astype(np.int32)
    offs = np.array([0, cap, 2 * cap], np.int32)
    ids = np.concatenate([cand, cand[::-1]]).astype(np.int32)
    counts = np.full(cap, ps, np.int32)
    for k in (1, 4, 8):
        cert, (mid, lo, hi), rescored, exact = run_both_paths(gpu, pool, q, offs, ids, k)
        ex = exact["scores"]
        assert np.all(np.isfinite(ex))
        assert np.all(lo <= ex) and np.all(ex <= hi), (kind, k, "an interval misses the exact score")
        _, selected, outs = orc.sparse_batch(q, keys, values, summ, counts, offs, ids, H, D, ps, k)
        for r in range(2):
            assert cert["selected"][r].tolist() == selected[r].tolist(), (kind, k, r)
        assert orc.max_abs_diff(cert["outputs"], outs) <= 1e-4
    pool.close()


@pytest.mark.parametrize("query", ["zero", "random"])
def test_certified_large_request_ties_and_duplicates(gpu, query):
    # 700 candidates (the selection kernel for more than 256): 350 pages each
    # listed twice.  With a zero query every score is +0, so the radix select
    # runs down to the id bits and every interval overlaps (all rescored); with
    # a random query the duplicates are exact ties of the same page.
    rng = np.random.default_rng(11 if query == "zero" else 12)
    H, D, ps, cap = 32, 128, 16, 350
    E = H * D
    keys = rng.standard_normal((cap, ps, E)).astype(np.float32)
    values = rng.standard_normal((cap, ps, E)).astype(np.float32)
    pool = gpu.DevicePagePool(H, D, ps, cap)
    page_ids = np.arange(cap, dtype=np.int32)
    counts = np.full(cap, ps, np.int32)
    pool.upload_pages(page_ids, counts, page_ids.astype(np.int64) * ps * E, keys, values)
    ids = np.concatenate([rng.permutation(cap), rng.permutation(cap)]).astype(np.int32)
    offs = np.array([0, ids.size], np.int32)
    q = (np.zeros((1, E)) if query == "zero" else rng.standard_normal((1, E))).astype(np.float32)
    summ = orc.pool_summaries(keys, counts, E)
    for k in (1, 64, 200):
        with gpu.SparseContext(pool, k, 1, ids.size, k) as ctx:
            res = ctx.run_batch(q, offs, ids, output_mode=gpu.OUTPUT_OUTPUTS, want_ids=True)
        _, selected, outs = orc.sparse_batch(q, keys, values, summ, counts, offs, ids, H, D, ps, k)
        assert res["selected"][0].tolist() == selected[0].tolist(), (query, k)
        assert orc.max_abs_diff(res["outputs"], outs) <= 1e-4
    pool.close()


@pytest.mark.parametrize("n_cand,k,near_count,fused_env", [
    (40, 8, 8, None), (600, 8, 8, None), (40, 8, 12, None), (600, 8, 12, None),
    (40, 2, 2, "0"), (40, 8, 8, "0"),
])
def test_refined_intervals_settle_near_ties_without_the_chain(gpu, n_cand, k, near_count,
                                                              fused_env):
    # near_count pages whose exact scores differ by about 1e-3: the score
    # pass's intervals (several 1e-3 wide at these magnitudes) overlap, the
    # refined intervals (the rounding error of each addition accounted for
    # exactly where its binade is certain, a few 1e-5 wide) do not.  With 8
    # such pages (every one flagged) the selection must be settled without
    # any exact chain, every interval (refined or not) must contain the
    # exact score.  With more flagged pages than
    # half the workgroup's waves (8 of 16; 2 of the 4 in the three-kernel
    # select for at most 256 candidates, DSD_FUSED_STEP=0) the refinement
    # is skipped and the flagged pages take the exact chain.  40 candidates
    # take the single-launch step unless it is switched off, 600 the
    # three-kernel step.
    rng = np.random.default_rng(n_cand)
    H, D, ps = 32, 128, 16
    E = H * D
    scale = 1.0 / np.sqrt(np.float32(D))
    q = rng.standard_normal(E).astype(np.float32)
    m = int(np.argmax(np.abs(q)))
    base = (0.2 * q + 0.25 * rng.standard_normal(E)).astype(np.float32)
    summ = (0.25 * rng.standard_normal((n_cand, E))).astype(np.float32)
    near = np.arange(near_count)
    for j in near:
        row = base.copy()
        row[m] = np.float32(row[m] + j * 1e-3 / (q[m] * scale))
        summ[j] = row
    keys = rng.standard_normal((n_cand, ps, E)).astype(np.float32)
    values = rng.standard_normal((n_cand, ps, E)).astype(np.float32)
    pool = gpu.DevicePagePool(H, D, ps, n_cand)
    page_ids = np.arange(n_cand, dtype=np.int32)
    counts = np.full(n_cand, ps, np.int32)
    pool.upload_pages(page_ids, counts, page_ids.astype(np.int64) * ps * E, keys, values, summ)
    ids = rng.permutation(n_cand).astype(np.int32)
    offs = np.array([0, n_cand], np.int32)
    old = os.environ.get("DSD_FUSED_STEP")
    if fused_env is not None:
        os.environ["DSD_FUSED_STEP"] = fused_env
    try:
        cert, (mid, lo, hi), rescored, exact = run_both_paths(gpu, pool, q[None, :], offs, ids,
                                                              k)
    finally:
        if old is None:
            os.environ.pop("DSD_FUSED_STEP", None)
        else:
            os.environ["DSD_FUSED_STEP"] = old
    limit = 2 if (fused_env == "0" and n_cand <= 256) else 8
    ex = exact["scores"]
    assert np.all(lo <= ex) and np.all(ex <= hi), "an interval misses the exact score"
    _, selected, outs = orc.sparse_batch(q[None, :], keys, values, summ, counts, offs, ids,
                                         H, D, ps, k)
    assert cert["selected"][0].tolist() == selected[0].tolist()
    assert sorted(selected[0].tolist()) == list(range(near_count - k, near_count))
    assert orc.max_abs_diff(cert["outputs"], outs) <= 1e-4
    if near_count > limit:
        # the members overlap each other; the outsiders within an interval's
        # width of the smallest member are flagged too
        assert limit < rescored <= near_count, f"{rescored} pages took the exact chain"
        pool.close()
        return
    assert rescored == 0, f"{rescored} pages needed the exact chain"
    # Both step forms keep the refined intervals in LDS: the intervals the
    # step leaves are the score pass's (refined ones are below 2e-4 here),
    # so a select replay starts again from first-pass intervals.
    where = np.argsort(ids)                          # candidate position of each page id
    widths = (hi - lo)[where[near]]
    assert np.all(widths > 2e-4), widths
    pool.close()


@pytest.mark.parametrize("k", [1, 8])
def test_midpoint_order_reversed_by_certification(gpu, k):
    # Every request's k-th and (k+1)-th pages (A and B) have the same
    # products in another order: B permutes A's summary within a block where
    # the query is constant, so their exact scores agree and the reference's
    # sequential sums differ by rounding only, while their values are
    # unrelated.  The score-pass midpoints then order A and B at random: in
    # some requests (asserted) the certified selection takes the page whose
    # midpoint is the lower one, and the selected ids and the outputs (which
    # differ a lot between A and B) must still be sparse_cpu's.
    rng = np.random.default_rng(1000 + k)
    H, D, ps = 32, 128, 16
    E = H * D
    B = 48
    block = np.arange(1024, 2048)
    q0 = rng.standard_normal(E).astype(np.float32)
    q0[block] = 0.37
    queries = np.empty((B, E), np.float32)
    for r in range(B):
        q = (q0 + 0.05 * rng.standard_normal(E)).astype(np.float32)
        q[block] = 0.37
        queries[r] = q
    n_high, n_low = k - 1, 24
    cap = n_high + n_low + 2 * B
    summ = np.empty((cap, E), np.float32)
    for p in range(n_high):
        summ[p] = (0.3 * q0 + 0.02 * rng.standard_normal(E)).astype(np.float32)
    for p in range(n_high, n_high + n_low):
        summ[p] = (0.02 * rng.standard_normal(E)).astype(np.float32)
    first_pair = n_high + n_low
    for r in range(B):
        a = (0.15 * q0 + 0.02 * rng.standard_normal(E)).astype(np.float32)
        b = a.copy()
        b[block] = a[block][rng.permutation(block.size)]
        summ[first_pair + 2 * r] = a
        summ[first_pair + 2 * r + 1] = b
    keys = rng.standard_normal((cap, ps, E)).astype(np.float32)
    values = rng.standard_normal((cap, ps, E)).astype(np.float32)
    counts = np.full(cap, ps, np.int32)
    pool = gpu.DevicePagePool(H, D, ps, cap)
    page_ids = np.arange(cap, dtype=np.int32)
    pool.upload_pages(page_ids, counts, page_ids.astype(np.int64) * ps * E, keys, values, summ)
    shared = np.arange(first_pair, dtype=np.int32)
    lists = [rng.permutation(np.concatenate([shared, [first_pair + 2 * r, first_pair + 2 * r + 1]]))
             .astype(np.int32) for r in range(B)]
    offs = np.zeros(B + 1, np.int32)
    offs[1:] = np.cumsum([len(x) for x in lists])
    ids = np.concatenate(lists).astype(np.int32)
    total = int(offs[-1])
    with gpu.SparseContext(pool, k, B, total, selected_total(offs, k)) as ctx:
        cert = ctx.run_batch(queries, offs, ids, output_mode=gpu.OUTPUT_OUTPUTS, want_ids=True)
        launch = ctx.last_launch()
        mid, lo, hi = ctx.score_bounds(total)
    assert launch["fused"] == 1, launch
    _, selected, outs = orc.sparse_batch(queries, keys, values, summ, counts, offs, ids,
                                         H, D, ps, k)
    reversed_pairs = 0
    for r in range(B):
        assert cert["selected"][r].tolist() == selected[r].tolist(), r
        pa, pb = first_pair + 2 * r, first_pair + 2 * r + 1
        at = {int(p): offs[r] + i for i, p in enumerate(lists[r])}
        ma, mb = mid[at[pa]], mid[at[pb]]
        won = pa if pa in selected[r].tolist() else pb
        assert (pa in selected[r].tolist()) != (pb in selected[r].tolist())
        if ma != mb and (pa if ma > mb else pb) != won:
            reversed_pairs += 1
    assert orc.max_abs_diff(cert["outputs"], outs) <= 1e-4
    assert reversed_pairs > 0, "no request had its midpoint order reversed by certification"
    pool.close()


@pytest.mark.parametrize("batch,tie_request,near_count", [
    (1, 0, 8),     # one head per workgroup: 32 workgroups share the request
    (16, 5, 8),    # two heads: 16 workgroups
    (16, 15, 3),
    (16, 9, 2),    # two flagged pages
    (40, 0, 8),    # eight heads: 4 workgroups, two flagged pages each
    (64, 63, 8),
])
def test_refinement_shared_by_the_requests_workgroups(gpu, batch, tie_request, near_count):
    """One request of the batch has near_count pages within about 1e-3 of
    each other among its top-8; in the single-launch step its workgroups
    refine the flagged pages between them (page f by workgroup f mod the
    request's workgroups) and exchange the intervals.  Every request's ids
    must equal the oracle's, no page may need the exact chain (the refined
    intervals settle it), and the outputs must be within 1e-4; the near
    pages' first-pass intervals must overlap (the step had to refine)."""
    rng = np.random.default_rng(1000 + batch + tie_request)
    H, D, ps, k = 32, 128, 16, 8
    E = H * D
    scale = 1.0 / np.sqrt(np.float32(D))
    sizes = [40 if r == tie_request else 9 for r in range(batch)]
    offs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    n_pages = int(offs[-1])
    queries = rng.standard_normal((batch, E)).astype(np.float32)
    summ = (0.25 * rng.standard_normal((n_pages, E))).astype(np.float32)
    q = queries[tie_request]
    m = int(np.argmax(np.abs(q)))
    base = (0.2 * q + 0.25 * rng.standard_normal(E)).astype(np.float32)
    first = int(offs[tie_request])
    for j in range(near_count):
        row = base.copy()
        row[m] = np.float32(row[m] + j * 1e-3 / (q[m] * scale))
        summ[first + j] = row
    keys = rng.standard_normal((n_pages, ps, E)).astype(np.float32)
    values = rng.standard_normal((n_pages, ps, E)).astype(np.float32)
    pool = gpu.DevicePagePool(H, D, ps, n_pages)
    try:
        page_ids = np.arange(n_pages, dtype=np.int32)
        counts = np.full(n_pages, ps, np.int32)
        pool.upload_pages(page_ids, counts, page_ids.astype(np.int64) * ps * E, keys, values,
                          summ)
        ids = np.concatenate([rng.permutation(np.arange(offs[r], offs[r + 1]))
                              for r in range(batch)]).astype(np.int32)
        print(f"shared refinement: batch {batch}, near-tie request {tie_request}", flush=True)
        with gpu.SparseContext(pool, k, batch, n_pages, selected_total(offs, k)) as ctx:
            res = ctx.run_batch(queries, offs, ids, output_mode=gpu.OUTPUT_OUTPUTS,
                                want_ids=True)
            info = ctx.last_launch()
            rescored = ctx.exact_rescored_pages()
            ctx.device_status()
            _, lo, hi = ctx.score_bounds(n_pages)
        assert info["fused"] == 1, info
        at = {int(p): i for i, p in enumerate(ids)}
        near = [at[first + j] for j in range(near_count)]
        assert any(lo[x] <= hi[y] and lo[y] <= hi[x] for x in near for y in near if x != y), \
            "the near pages' first-pass intervals do not overlap"
        _, selected, outs = orc.sparse_batch(queries, keys, values, summ, counts, offs, ids,
                                             H, D, ps, k)
        for r in range(batch):
            assert res["selected"][r].tolist() == selected[r].tolist(), r
        if near_count >= k:
            assert sorted(selected[tie_request].tolist()) == list(
                range(first + near_count - k, first + near_count))
        assert rescored == 0, f"{rescored} pages took the exact chain"
        assert orc.max_abs_diff(res["outputs"], outs) <= 1e-4
    finally:
        pool.close()
