"""The single-launch step (fused score -> select -> attention, one kernel)
against the three-kernel step and the oracle.

The fused kernel is the default for E = 4096, head_dim 128 and up to 256
candidates per request; DSD_FUSED_STEP=0 at context creation selects the
three-kernel step.  Both use the same certified selection and the same
attention arithmetic, so selections must be equal and outputs bit-equal."""
from __future__ import annotations

import os

import numpy as np
import pytest

import _oracle as orc

pytestmark = pytest.mark.gpu

H, D, PS = 32, 128, 16
E = H * D


def make_ctx(gpu, pool, k, batch, fused):
    total = int(batch.cand_offsets[-1])
    sel = int(sum(min(k, int(n)) for n in np.diff(batch.cand_offsets)))
    old = os.environ.get("DSD_FUSED_STEP")
    os.environ["DSD_FUSED_STEP"] = "1" if fused else "0"
    try:
        return gpu.SparseContext(pool, k, batch.batch, max(total, 1), max(sel, 1))
    finally:
        if old is None:
            del os.environ["DSD_FUSED_STEP"]
        else:
            os.environ["DSD_FUSED_STEP"] = old


def oracle_step(batch, queries, k):
    summ = np.zeros((batch.capacity, E), np.float32)
    live = batch.live_page_ids()
    if len(live):
        summ[live] = orc.pool_summaries(batch.key_pool, batch.token_counts, E, live)
    return orc.sparse_batch(queries, batch.key_pool, batch.value_pool, summ, batch.token_counts,
                            batch.cand_offsets, batch.cand_ids, H, D, PS, k)


@pytest.mark.parametrize("seed", [7, 8, 21])
def test_fused_equals_three_kernel_step_and_oracle(gpu, seed):
    lengths = gpu.reference_context_lengths(16, 512, 2048, seed)
    batch = gpu.SyntheticBatch(H, D, PS, lengths, seed=seed)
    pool = gpu.DevicePagePool(H, D, PS, batch.capacity)
    batch.upload(pool)
    with make_ctx(gpu, pool, 8, batch, True) as f, make_ctx(gpu, pool, 8, batch, False) as u:
        rf = f.run_batch(batch.queries, batch.cand_offsets, batch.cand_ids,
                         output_mode=gpu.OUTPUT_OUTPUTS, want_ids=True)
        ru = u.run_batch(batch.queries, batch.cand_offsets, batch.cand_ids,
                         output_mode=gpu.OUTPUT_OUTPUTS, want_ids=True)
    _, selected, outs = oracle_step(batch, batch.queries, 8)
    for r in range(batch.batch):
        assert rf["selected"][r].tolist() == selected[r].tolist(), (seed, r)
        assert ru["selected"][r].tolist() == selected[r].tolist(), (seed, r)
    assert np.array_equal(rf["outputs"].view(np.uint32), ru["outputs"].view(np.uint32))
    assert orc.max_abs_diff(rf["outputs"], outs) <= 1e-4
    pool.close()


def test_fused_consecutive_steps_reuse_the_step_state(gpu):
    # Ticket counters, arrival counters and ready epochs are reset by the
    # kernel itself; five launches in a row with different queries must each
    # match the oracle.
    lengths = [0, 17, 300, 1, 2000, 16, 4095]   # empty request, 1-token page, 256 pages
    batch = gpu.SyntheticBatch(H, D, PS, lengths, seed=3)
    assert batch.max_candidates == 256
    pool = gpu.DevicePagePool(H, D, PS, batch.capacity)
    batch.upload(pool)
    rng = np.random.default_rng(11)
    with make_ctx(gpu, pool, 8, batch, True) as ctx:
        for step in range(5):
            q = rng.standard_normal((batch.batch, E)).astype(np.float32) * (1 + step)
            res = ctx.run_batch(q, batch.cand_offsets, batch.cand_ids,
                                output_mode=gpu.OUTPUT_OUTPUTS, want_ids=True)
            _, selected, outs = oracle_step(batch, q, 8)
            for r in range(batch.batch):
                assert res["selected"][r].tolist() == selected[r].tolist(), (step, r)
            assert orc.max_abs_diff(res["outputs"], outs) <= 1e-4, step
            assert not res["outputs"][0].any(), "empty request must give zeros"
    pool.close()


@pytest.mark.parametrize("k", [0, 1, 3, 64, 256])
def test_fused_top_k_edges(gpu, k):
    lengths = [40, 700, 0, 2048]
    batch = gpu.SyntheticBatch(H, D, PS, lengths, seed=k + 5)
    pool = gpu.DevicePagePool(H, D, PS, batch.capacity)
    batch.upload(pool)
    with make_ctx(gpu, pool, k, batch, True) as ctx:
        res = ctx.run_batch(batch.queries, batch.cand_offsets, batch.cand_ids,
                            output_mode=gpu.OUTPUT_OUTPUTS, want_ids=True)
    _, selected, outs = oracle_step(batch, batch.queries, k)
    for r in range(batch.batch):
        assert res["selected"][r].tolist() == selected[r].tolist(), (k, r)
    assert orc.max_abs_diff(res["outputs"], outs) <= 1e-4
    if k == 0:
        assert not res["outputs"].any()
    pool.close()


def test_fused_phase_timings_are_reported(gpu):
    lengths = gpu.reference_context_lengths(16, 512, 2048, 7)
    batch = gpu.SyntheticBatch(H, D, PS, lengths, seed=7)
    pool = gpu.DevicePagePool(H, D, PS, batch.capacity)
    batch.upload(pool)
    with make_ctx(gpu, pool, 8, batch, True) as ctx:
        ctx.run_batch(batch.queries, batch.cand_offsets, batch.cand_ids,
                      output_mode=gpu.OUTPUT_OUTPUTS)
        t = ctx.run_batch(batch.queries, batch.cand_offsets, batch.cand_ids,
                          output_mode=gpu.OUTPUT_OUTPUTS)["timings"]
    assert t["kernel_ms"] > 0.0
    for key in ("score_ms", "topk_ms", "attention_ms"):
        assert 0.0 <= t[key] <= t["kernel_ms"] * 1.5 + 0.05, (key, t)
    assert t["score_ms"] > 0.0 and t["attention_ms"] > 0.0
    pool.close()


def test_fused_device_path_reports_understated_max_candidates(gpu):
    # The device entry point trusts max_candidates; a request larger than the
    # max_candidates the caller stated is caught by the kernel's own check,
    # gives zeros for that request, and is reported at the next synchronising
    # call.
    import torch

    lengths = [300 * PS, 40]                     # 300 candidates in request 0
    batch = gpu.SyntheticBatch(H, D, PS, lengths, seed=9)
    pool = gpu.DevicePagePool(H, D, PS, batch.capacity)
    batch.upload(pool)
    dev = torch.device("cuda:0")
    q = torch.from_numpy(batch.queries).to(dev)
    offs = torch.from_numpy(batch.cand_offsets).to(dev)
    ids = torch.from_numpy(batch.cand_ids).to(dev)
    out = torch.full((batch.batch, E), 7.0, device=dev)
    with make_ctx(gpu, pool, 8, batch, True) as ctx:
        ctx.run_batch_device(batch.batch, batch.total_candidates, 200, q.data_ptr(),
                             offs.data_ptr(), ids.data_ptr(), out.data_ptr(),
                             stream=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        with pytest.raises(gpu.InvalidArgument, match="max_candidates"):
            ctx.exact_rescored_pages()
        assert not out[0].any().item()
        # the context stays usable with a correct max_candidates
        ctx.run_batch_device(batch.batch, batch.total_candidates, batch.max_candidates,
                             q.data_ptr(), offs.data_ptr(), ids.data_ptr(), out.data_ptr(),
                             stream=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert ctx.exact_rescored_pages() >= 0
    pool.close()


def test_fused_duplicate_candidate_ids_are_both_kept(gpu):
    # A request that lists a page twice: the reference comparator sees two
    # equal (score, id) keys and gathers the page twice; the ranks must stay
    # a permutation (equal keys by position) so every member slot is written.
    lengths = [600, 300, 900]
    batch = gpu.SyntheticBatch(H, D, PS, lengths, seed=17)
    pool = gpu.DevicePagePool(H, D, PS, batch.capacity)
    batch.upload(pool)
    offs = batch.cand_offsets.copy()
    ids = [list(batch.cand_ids[offs[r]:offs[r + 1]]) for r in range(batch.batch)]
    summ = np.zeros((batch.capacity, E), np.float32)
    live = batch.live_page_ids()
    summ[live] = orc.pool_summaries(batch.key_pool, batch.token_counts, E, live)
    q = batch.queries
    # duplicate request 0's best page and request 2's third best page
    for r, pick in ((0, 0), (2, 2)):
        sc = summ[ids[r]] @ q[r]
        best = ids[r][int(np.argsort(-sc, kind="stable")[pick])]
        ids[r].insert(len(ids[r]) // 2, best)
    new_offs = np.zeros(batch.batch + 1, np.int32)
    new_offs[1:] = np.cumsum([len(x) for x in ids])
    new_ids = np.concatenate([np.asarray(x, np.int32) for x in ids])
    k = 6
    sel_total = int(sum(min(k, len(x)) for x in ids))
    _, selected, outs = orc.sparse_batch(q, batch.key_pool, batch.value_pool, summ,
                                         batch.token_counts, new_offs, new_ids, H, D, PS, k)
    assert sum(list(selected[r]).count(ids[r][len(ids[r]) // 2]) for r in (0, 2)) >= 2
    for fused in (True, False):
        old = os.environ.get("DSD_FUSED_STEP")
        os.environ["DSD_FUSED_STEP"] = "1" if fused else "0"
        try:
            ctx = gpu.SparseContext(pool, k, batch.batch, int(new_offs[-1]), sel_total)
        finally:
            if old is None:
                del os.environ["DSD_FUSED_STEP"]
            else:
                os.environ["DSD_FUSED_STEP"] = old
        with ctx:
            res = ctx.run_batch(q, new_offs, new_ids, output_mode=gpu.OUTPUT_OUTPUTS,
                                want_ids=True)
        for r in range(batch.batch):
            assert res["selected"][r].tolist() == selected[r].tolist(), (fused, r)
        assert orc.max_abs_diff(res["outputs"], outs) <= 1e-4, fused
    pool.close()


def test_fused_large_batch_of_small_requests(gpu):
    # 300 small requests, some empty: 8 heads per workgroup, 4 workgroups per
    # request (1200 in all, several dispatch waves), every request group
    # waiting only on its own slices.
    rng = np.random.default_rng(23)
    lengths = [int(x) for x in rng.integers(0, 70, size=300)]
    batch = gpu.SyntheticBatch(H, D, PS, lengths, seed=23)
    pool = gpu.DevicePagePool(H, D, PS, batch.capacity)
    batch.upload(pool)
    k = 2
    with make_ctx(gpu, pool, k, batch, True) as f, make_ctx(gpu, pool, k, batch, False) as u:
        rf = f.run_batch(batch.queries, batch.cand_offsets, batch.cand_ids,
                         output_mode=gpu.OUTPUT_OUTPUTS, want_ids=True)
        ru = u.run_batch(batch.queries, batch.cand_offsets, batch.cand_ids,
                         output_mode=gpu.OUTPUT_OUTPUTS, want_ids=True)
    _, selected, outs = oracle_step(batch, batch.queries, k)
    for r in range(batch.batch):
        assert rf["selected"][r].tolist() == selected[r].tolist(), r
        assert ru["selected"][r].tolist() == selected[r].tolist(), r
    # 8 heads per workgroup here (2 waves per head): the same selection,
    # the softmax merged in another order than the 8-wave attention kernel.
    assert orc.max_abs_diff(rf["outputs"], ru["outputs"]) <= 1e-5
    assert orc.max_abs_diff(rf["outputs"], outs) <= 1e-4
    pool.close()


@pytest.mark.parametrize("seed", [31, 32])
def test_fused_skewed_lengths(gpu, seed):
    # Very uneven requests (1 to 256 candidates, empty ones, equal sizes in
    # several places), two launches in a row; 24 requests: 4 heads per
    # workgroup, so 8 slices per request and up to 32 candidates per slice
    # (the launch form whose slices pipeline several score passes).
    rng = np.random.default_rng(seed)
    lengths = [int(x) for x in rng.choice([0, 5, 16, 200, 1000, 4096, 4096, 2500], size=24)]
    batch = gpu.SyntheticBatch(H, D, PS, lengths, seed=seed)
    pool = gpu.DevicePagePool(H, D, PS, batch.capacity)
    batch.upload(pool)
    k = 8
    with make_ctx(gpu, pool, k, batch, True) as f:
        for _ in range(2):
            rf = f.run_batch(batch.queries, batch.cand_offsets, batch.cand_ids,
                             output_mode=gpu.OUTPUT_OUTPUTS, want_ids=True)
    _, selected, outs = oracle_step(batch, batch.queries, k)
    for r in range(batch.batch):
        assert rf["selected"][r].tolist() == selected[r].tolist(), r
    assert orc.max_abs_diff(rf["outputs"], outs) <= 1e-4
    pool.close()
