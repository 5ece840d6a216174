"""GPU parity of the sparse and dense decode steps through the C ABI.

Bar: selected page ids bit-exact vs sparse_cpu
(the reference tie-break included), outputs within max-abs 1e-4 (the
reference's own test tolerances where tighter), dense_gpu within 1e-4 of
dense_cpu.  Scores in debug mode and device summaries are also bit-exact.
Inputs: the reference's own test batches (golden fixture) and the
BASELINE.json configurations (N(0,1) data).
"""
from __future__ import annotations

import numpy as np
import pytest

import _oracle as orc
from test_oracle import CASES, SMALL_CASES, unpack

pytestmark = pytest.mark.gpu

BASELINE_TOL = 1e-4


def upload_fixture(gpu, c):
    H, D, ps, k, B = unpack(c)
    E = H * D
    tc = c["token_counts"]
    pool = gpu.DevicePagePool(H, D, ps, len(tc))
    live = np.nonzero(tc)[0].astype(np.int32)
    pool.upload_pages(live, tc[live], live.astype(np.int64) * ps * E, c["key_pool"],
                      c["value_pool"])
    return pool, live


def selected_total(offsets, k):
    return int(sum(min(k, int(n)) for n in np.diff(offsets)))


@pytest.mark.parametrize("name", [n for n in SMALL_CASES if not n.startswith("dense_")])
def test_sparse_matches_reference_cases(gpu, name):
    c = CASES[name]
    H, D, ps, k, B = unpack(c)
    E = H * D
    tol = float(c["tolerance"])
    pool, live = upload_fixture(gpu, c)
    # device summaries == the reference cache's summaries, bit for bit
    dev = pool.download_summaries(live)
    ref = c["summaries"].reshape(-1, E)[live]
    assert np.array_equal(dev.view(np.uint32), ref.view(np.uint32))
    offs, ids = c["cand_offsets"], c["cand_ids"]
    with gpu.SparseContext(pool, k, B, len(ids), selected_total(offs, k)) as ctx:
        res = ctx.run_batch(c["queries"], offs, ids)
    assert np.array_equal(res["scores"].view(np.uint32), c["ref_scores"].view(np.uint32))
    kk = max(k, 1)
    for r in range(B):
        cnt = int(c["ref_counts"][r])
        assert res["selected"][r].tolist() == c["ref_selected"][r * kk:r * kk + cnt].tolist()
    diff = orc.max_abs_diff(res["outputs"], c["ref_sparse_out"])
    assert diff <= tol, (name, diff)
    assert res["timings"]["attention_ms"] >= 0.0
    pool.close()


@pytest.mark.parametrize("name", [n for n in SMALL_CASES if n.startswith("dense_")
                                  or n == "reference_topk_covers_all"])
def test_dense_matches_reference_cases(gpu, name):
    c = CASES[name]
    pool, _ = upload_fixture(gpu, c)
    out, kernel_ms = gpu.dense_run_batch(pool, c["queries"], c["cand_offsets"], c["cand_ids"])
    diff = orc.max_abs_diff(out, c["ref_dense_out"])
    assert diff <= float(c["tolerance"]), (name, diff)
    assert kernel_ms >= 0.0
    pool.close()


def test_dense_zero_context_gives_zeros(gpu):
    # tests/test_dense_cuda.cpp:57-87: a request with no pages -> zeros.
    pool = gpu.DevicePagePool(2, 16, 8, 4)
    q = np.full((1, 32), 0.25, np.float32)
    out, _ = gpu.dense_run_batch(pool, q, np.array([0, 0], np.int32), np.zeros(0, np.int32))
    assert not out.any()


def test_tie_break_prefers_smaller_page_ids(gpu):
    # tests/test_sparse_cuda.cpp:134-169: four single-token pages appended to
    # one request (LIFO ids 3,2,1,0), zero keys, values i, zero query.
    H, D, ps, k = 1, 4, 1, 2
    pool = gpu.DevicePagePool(H, D, ps, 4)
    page_ids = np.array([3, 2, 1, 0], np.int32)
    keys = np.zeros((4, 4), np.float32)
    values = np.repeat(np.arange(4, dtype=np.float32)[:, None], 4, axis=1)
    pool.upload_pages(page_ids, np.ones(4, np.int32), np.arange(4, dtype=np.int64) * 4, keys,
                      values)
    with gpu.SparseContext(pool, k, 1, 4, 2) as ctx:
        res = ctx.run_batch(np.zeros((1, 4), np.float32), np.array([0, 4], np.int32), page_ids)
    assert res["selected"][0].tolist() == [0, 1]


def test_no_output_fast_path_leaves_timings_zero(gpu):
    # tests/test_sparse_cuda.cpp:171-205
    c = CASES["no_output_fast_path"]
    H, D, ps, k, B = unpack(c)
    pool, _ = upload_fixture(gpu, c)
    offs, ids = c["cand_offsets"], c["cand_ids"]
    with gpu.SparseContext(pool, k, B, len(ids), selected_total(offs, k)) as ctx:
        res = ctx.run_batch(c["queries"], offs, ids, output_mode=gpu.OUTPUT_NONE,
                            timing_mode=gpu.TIMING_NONE)
    assert "selected" not in res
    t = res["timings"]
    assert t["kernel_ms"] == 0.0 and t["score_ms"] == 0.0 and t["attention_ms"] == 0.0


def test_capacity_and_id_errors(gpu):
    c = CASES["sparse_small"]
    H, D, ps, k, B = unpack(c)
    pool, _ = upload_fixture(gpu, c)
    offs, ids = c["cand_offsets"], c["cand_ids"]
    total, sel = len(ids), selected_total(offs, k)
    with gpu.SparseContext(pool, k, B - 1, total, sel) as ctx:
        with pytest.raises(gpu.InvalidArgument, match="batch exceeds"):
            ctx.run_batch(c["queries"], offs, ids)
    with gpu.SparseContext(pool, k, B, total - 1, sel) as ctx:
        with pytest.raises(gpu.InvalidArgument, match="candidate page count"):
            ctx.run_batch(c["queries"], offs, ids)
    with gpu.SparseContext(pool, k, B, total, sel - 1) as ctx:
        with pytest.raises(gpu.InvalidArgument, match="selected page count"):
            ctx.run_batch(c["queries"], offs, ids)
    bad = ids.copy()
    bad[0] = pool.capacity
    with gpu.SparseContext(pool, k, B, total, sel) as ctx:
        with pytest.raises(gpu.OutOfRange):
            ctx.run_batch(c["queries"], offs, bad)
    with pytest.raises(gpu.InvalidArgument, match="head_dim"):
        gpu.SparseContext(gpu.DevicePagePool(1, 256, 4, 1), 1, 1, 1, 1)


def check_batch_against_oracle(gpu, batch, top_k, tol=BASELINE_TOL):
    H, D, ps = batch.num_heads, batch.head_dim, batch.page_size
    E = H * D
    pool = gpu.DevicePagePool(H, D, ps, batch.capacity)
    batch.upload(pool)
    live = batch.live_page_ids()
    dev_summ = pool.download_summaries(live)
    summaries = np.zeros((batch.capacity, E), np.float32)
    summaries[live] = dev_summ
    ref = orc.pool_summaries(batch.key_pool, batch.token_counts, E, live)
    assert np.array_equal(dev_summ.view(np.uint32), ref.view(np.uint32))
    sel_total = selected_total(batch.cand_offsets, top_k)
    with gpu.SparseContext(pool, top_k, batch.batch, batch.total_candidates, sel_total) as ctx:
        res = ctx.run_batch(batch.queries, batch.cand_offsets, batch.cand_ids)
    scores, selected, outs = orc.sparse_batch(
        batch.queries, batch.key_pool, batch.value_pool, summaries, batch.token_counts,
        batch.cand_offsets, batch.cand_ids, H, D, ps, top_k)
    assert np.array_equal(res["scores"].view(np.uint32), scores.view(np.uint32))
    for r in range(batch.batch):
        assert res["selected"][r].tolist() == selected[r].tolist(), r
    diff = orc.max_abs_diff(res["outputs"], outs)
    assert diff <= tol, diff
    return pool, res, outs


def test_baseline_config1_single_request(gpu):
    # B=1, 1024 tokens, 32x128, ps16 (64 pages), k8, seed 7.
    batch = gpu.SyntheticBatch(32, 128, 16, [1024], seed=7)
    pool, res, _ = check_batch_against_oracle(gpu, batch, 8)
    # dense over the same inputs vs dense_cpu
    dense, _ = gpu.dense_run_batch(pool, batch.queries, batch.cand_offsets, batch.cand_ids)
    ref = orc.dense_batch(batch.queries, batch.key_pool, batch.value_pool, batch.token_counts,
                          batch.cand_offsets, batch.cand_ids, 32, 128, 16)
    assert orc.max_abs_diff(dense, ref) <= BASELINE_TOL


def test_baseline_config2_ragged_batch(gpu):
    # B=16, ctx U[512,2048] in the reference draw order
    # (mt19937 seed 7 -> 1207 pages), 32x128, ps16, k8, N(0,1).
    lengths = gpu.reference_context_lengths(16, 512, 2048, 7)
    batch = gpu.SyntheticBatch(32, 128, 16, lengths, seed=7)
    assert batch.total_candidates == 1207
    pool, res, outs = check_batch_against_oracle(gpu, batch, 8)
    dense, _ = gpu.dense_run_batch(pool, batch.queries, batch.cand_offsets, batch.cand_ids)
    ref = orc.dense_batch(batch.queries, batch.key_pool, batch.value_pool, batch.token_counts,
                          batch.cand_offsets, batch.cand_ids, 32, 128, 16)
    assert orc.max_abs_diff(dense, ref) <= BASELINE_TOL


def test_config3_shape_long_context_topk64(gpu):
    # BASELINE configs[2] shape per request (32768 tokens = 2048 pages of 16,
    # k = 64, seed 11) on 2 of its 32 requests: exercises k > 16 (the
    # reference's CUB path) and a 2048-candidate select.
    batch = gpu.SyntheticBatch(32, 128, 16, [32768, 32768], seed=11)
    check_batch_against_oracle(gpu, batch, 64)


def test_config4_shape_page64_topk32(gpu):
    # BASELINE configs[3] shape (ps 64, k 32, ctx U[4096,16384], seed 13) on
    # 4 of its 64 requests.
    lengths = gpu.reference_context_lengths(4, 4096, 16384, 13)
    batch = gpu.SyntheticBatch(32, 128, 64, lengths, seed=13)
    check_batch_against_oracle(gpu, batch, 32)


def test_ties_and_signed_zero_scores_select_like_sparse_cpu(gpu):
    # Duplicate summaries give exactly equal scores; zero summaries give +/-0.
    rng = np.random.default_rng(21)
    H, D, ps, k = 2, 8, 2, 5
    E = H * D
    cap = 24
    keys = np.zeros((cap, ps, E), np.float32)
    base = rng.standard_normal((3, ps, E)).astype(np.float32)
    for p in range(cap):
        keys[p] = base[p % 3] if p % 4 else 0.0
    values = rng.standard_normal((cap, ps, E)).astype(np.float32)
    pool = gpu.DevicePagePool(H, D, ps, cap)
    ids = np.arange(cap, dtype=np.int32)
    pool.upload_pages(ids, np.full(cap, ps, np.int32), ids.astype(np.int64) * ps * E, keys,
                      values)
    cand = rng.permutation(cap).astype(np.int32)
    offs = np.array([0, 10, 10, 24], np.int32)
    q = rng.standard_normal((3, E)).astype(np.float32)
    q[1] = -0.0
    with gpu.SparseContext(pool, k, 3, cap, 3 * k) as ctx:
        res = ctx.run_batch(q, offs, cand)
    summ = orc.pool_summaries(keys, np.full(cap, ps, np.int32), E)
    scores, selected, outs = orc.sparse_batch(q, keys, values, summ, np.full(cap, ps, np.int32),
                                              offs, cand, H, D, ps, k)
    assert np.array_equal(res["scores"].view(np.uint32), scores.view(np.uint32))
    for r in range(3):
        assert res["selected"][r].tolist() == selected[r].tolist()
    assert orc.max_abs_diff(res["outputs"], outs) <= 1e-5


def test_device_resident_step_matches_host_step(gpu):
    import torch
    lengths = gpu.reference_context_lengths(16, 512, 2048, 7)
    batch = gpu.SyntheticBatch(32, 128, 16, lengths, seed=3)
    pool = gpu.DevicePagePool(32, 128, 16, batch.capacity)
    batch.upload(pool)
    sel_total = selected_total(batch.cand_offsets, 8)
    dev = torch.device("cuda:0")
    q = torch.from_numpy(batch.queries).to(dev)
    offs = torch.from_numpy(batch.cand_offsets).to(dev)
    ids = torch.from_numpy(batch.cand_ids).to(dev)
    out = torch.zeros_like(q)
    sel = torch.full((batch.batch, 8), -1, dtype=torch.int32, device=dev)
    counts = torch.zeros(batch.batch, dtype=torch.int32, device=dev)
    with gpu.SparseContext(pool, 8, batch.batch, batch.total_candidates, sel_total) as ctx:
        host = ctx.run_batch(batch.queries, batch.cand_offsets, batch.cand_ids)
        stream = torch.cuda.Stream()
        with torch.cuda.stream(stream):
            ctx.run_batch_device(batch.batch, batch.total_candidates, batch.max_candidates,
                                 q.data_ptr(), offs.data_ptr(), ids.data_ptr(), out.data_ptr(),
                                 d_selected=sel.data_ptr(), d_counts=counts.data_ptr(),
                                 stream=stream.cuda_stream)
        stream.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), host["outputs"].view(np.uint32))
    got = sel.cpu().numpy()
    for r in range(batch.batch):
        assert got[r, :counts[r].item()].tolist() == host["selected"][r].tolist()


def test_staged_rows_step_matches_host_step(gpu):
    """Queries read in place from pinned rows (dsd_sparse_run_staged_rows)
    give the host step's outputs and ids bit for bit: rows scattered over a
    dsd_host_alloc block, one row taken from the staging itself, and a
    second, smaller step after the first."""
    import ctypes
    lengths = gpu.reference_context_lengths(16, 512, 2048, 7)
    batch = gpu.SyntheticBatch(32, 128, 16, lengths, seed=5)
    pool = gpu.DevicePagePool(32, 128, 16, batch.capacity)
    batch.upload(pool)
    B, E = batch.batch, 32 * 128
    q = batch.queries.reshape(B, E)
    sel_total = selected_total(batch.cand_offsets, 8)
    perm = np.random.default_rng(1).permutation(2 * B)[:B]
    with gpu.SparseContext(pool, 8, B, batch.total_candidates, sel_total) as ctx, \
            gpu.HostBlock(2 * B * E) as block:
        host = ctx.run_batch(batch.queries, batch.cand_offsets, batch.cand_ids,
                             output_mode=gpu.OUTPUT_OUTPUTS, want_ids=True)
        rows = []
        for r in range(B):
            block.array[perm[r] * E:(perm[r] + 1) * E] = q[r]
            rows.append(block.address + 4 * int(perm[r]) * E)
        staging_q = ctx.run_staged_rows(rows[:1], batch.cand_offsets[:2],
                                        batch.cand_ids[:batch.cand_offsets[1]])["staging_queries"]
        ctypes.memmove(staging_q + 4 * 3 * E, q[3].ctypes.data, 4 * E)
        rows[3] = staging_q + 4 * 3 * E
        got = ctx.run_staged_rows(rows, batch.cand_offsets, batch.cand_ids, want_ids=True)
        assert np.array_equal(got["outputs"].view(np.uint32),
                              host["outputs"].reshape(B, E).view(np.uint32))
        for r in range(B):
            assert got["selected"][r].tolist() == host["selected"][r].tolist()
        # a smaller step: the last five requests, rows in reverse block order
        sub = slice(B - 5, B)
        offs = batch.cand_offsets[B - 5:] - batch.cand_offsets[B - 5]
        ids = batch.cand_ids[batch.cand_offsets[B - 5]:]
        small = ctx.run_staged_rows(rows[sub], offs, ids, want_ids=True)
        assert np.array_equal(small["outputs"].view(np.uint32),
                              host["outputs"].reshape(B, E)[sub].view(np.uint32))
        for i in range(5):
            assert small["selected"][i].tolist() == host["selected"][B - 5 + i].tolist()


def test_staged_rows_are_checked_before_the_device(gpu):
    lengths = [64, 96]
    batch = gpu.SyntheticBatch(2, 64, 16, lengths, seed=2)
    pool = gpu.DevicePagePool(2, 64, 16, batch.capacity)
    batch.upload(pool)
    E = 2 * 64
    with gpu.SparseContext(pool, 2, 2, batch.total_candidates, 4) as ctx, \
            gpu.HostBlock(2 * E) as block:
        base = block.address
        cases = [
            ([base, batch.queries.ctypes.data], "not in dsd_host_alloc"),   # pageable memory
            ([base, base + 4], "aligned"),                                 # misaligned
            ([base, base + 4 * (E + 4)], "not in dsd_host_alloc"),          # runs past the end
            ([base, 0], "non-null"),
        ]
        for rows, msg in cases:
            with pytest.raises(gpu.InvalidArgument, match=msg):
                ctx.run_staged_rows(rows, batch.cand_offsets, batch.cand_ids)
        block.array[:] = batch.queries.reshape(-1)
        ok = ctx.run_staged_rows([base, base + 4 * E], batch.cand_offsets, batch.cand_ids)
        ref = ctx.run_batch(batch.queries, batch.cand_offsets, batch.cand_ids,
                            output_mode=gpu.OUTPUT_OUTPUTS)
        assert np.array_equal(ok["outputs"].view(np.uint32),
                              ref["outputs"].reshape(2, E).view(np.uint32))
        # an empty step needs no rows; a freed block no longer qualifies
        lib = gpu.load_library()
        assert lib.dsd_sparse_run_staged_rows(ctx.handle, 0, None, gpu.OUTPUT_OUTPUTS,
                                              gpu.TIMING_NONE, None, None, None) == 0
        other = gpu.HostBlock(E)
        rows = [base, other.address]
        other.array[:] = batch.queries.reshape(-1)[E:]
        again = ctx.run_staged_rows(rows, batch.cand_offsets, batch.cand_ids)
        assert np.array_equal(again["outputs"].view(np.uint32), ok["outputs"].view(np.uint32))
        addr = other.address
        other.close()
        with pytest.raises(gpu.InvalidArgument, match="not in dsd_host_alloc"):
            ctx.run_staged_rows(rows, batch.cand_offsets, batch.cand_ids)
        import ctypes
        assert lib.dsd_host_free(ctypes.c_void_p(addr)) == 1  # freed twice
        # a batch beyond the staging's capacity fails before the staging is read
        assert lib.dsd_sparse_run_staged(ctx.handle, 3, gpu.OUTPUT_OUTPUTS, gpu.TIMING_NONE,
                                         None, None, None) == 1
        assert b"capacity" in lib.dsd_last_error()
        rows3 = (ctypes.c_void_p * 3)(base, base, base)
        assert lib.dsd_sparse_run_staged_rows(ctx.handle, 3, rows3, gpu.OUTPUT_OUTPUTS,
                                              gpu.TIMING_NONE, None, None, None) == 1
        with pytest.raises(gpu.InvalidArgument, match="capacity"):
            ctx.run_staged_rows([base] * 3, np.array([0, 1, 2, 3], np.int32),
                                batch.cand_ids[:3])
