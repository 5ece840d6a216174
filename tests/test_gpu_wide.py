"""The wide single-launch step (WideStepKernel): the certified step for
requests of 257 to 2048 candidates in one launch, score slices, each
request's select (run by its last slice to finish) and the attention items
overlapping.

Its selections must equal the oracle's id for id (SelectTopKPagesCpu,
/root/reference/src/reference_kernels.cpp:82-107) and its outputs be within
1e-4 of sparse_cpu's; against the three-kernel step (DSD_WIDE_STEP=0), which
runs the same score pass, select and attention code in three launches, ids
and outputs must be bit-equal.  Cases: ragged batches mixing short and long
requests, k from 1 to 64 (and k above a request's candidate count), near
ties that the select settles by refinement or the exact chain, an empty
request, the device-buffer entry, back-to-back replays of the launch, pages
of 64 tokens with a partial last page, and a forced wait failure (the test
hook, set from the host) that must be reported and leave the context
usable."""
from __future__ import annotations

import os

import numpy as np
import pytest

import _oracle as orc

pytestmark = pytest.mark.gpu

H, D, PS = 32, 128, 16
E = H * D


def make_ctx(gpu, pool, k, batch_size, total, wide=True):
    sel = batch_size * max(k, 1)
    old = os.environ.get("DSD_WIDE_STEP")
    os.environ["DSD_WIDE_STEP"] = "1" if wide else "0"
    try:
        return gpu.SparseContext(pool, k, batch_size, max(total, 1), sel)
    finally:
        if old is None:
            del os.environ["DSD_WIDE_STEP"]
        else:
            os.environ["DSD_WIDE_STEP"] = old


def oracle(batch, k):
    summ = np.zeros((batch.capacity, E), np.float32)
    live = batch.live_page_ids()
    summ[live] = orc.pool_summaries(batch.key_pool, batch.token_counts, E, live)
    return orc.sparse_batch(batch.queries, batch.key_pool, batch.value_pool, summ,
                            batch.token_counts, batch.cand_offsets, batch.cand_ids, H, D, PS, k)


def run(gpu, pool, batch, k, wide):
    total = int(batch.cand_offsets[-1])
    with make_ctx(gpu, pool, k, batch.batch, total, wide) as ctx:
        res = ctx.run_batch(batch.queries, batch.cand_offsets, batch.cand_ids,
                            output_mode=gpu.OUTPUT_OUTPUTS, want_ids=True)
        res["launch"] = ctx.last_launch()
    return res


@pytest.mark.parametrize("lengths,k,seed", [
    ([5000, 32768, 700, 4100], 64, 3),        # 313, 2048, 44, 257 pages
    ([4112, 4113, 20000, 9000, 300], 8, 4),   # 257 and 258 pages at the edge
    ([16 * 2048, 16 * 300, 17], 1, 5),
    ([16 * 600, 16 * 40], 50, 6),             # k above the short request's 40
])
def test_wide_step_matches_oracle_and_three_kernels(gpu, lengths, k, seed):
    batch = gpu.SyntheticBatch(H, D, PS, lengths, seed=seed)
    pool = gpu.DevicePagePool(H, D, PS, batch.capacity)
    try:
        batch.upload(pool)
        print(f"wide step: lengths {lengths} k {k}", flush=True)
        wide = run(gpu, pool, batch, k, True)
        assert wide["launch"]["wide"] == 1 and wide["launch"]["fused"] == 0
        three = run(gpu, pool, batch, k, False)
        assert three["launch"]["wide"] == 0 and three["launch"]["fused"] == 0
        _, selected, outs = oracle(batch, k)
        for r in range(batch.batch):
            assert wide["selected"][r].tolist() == selected[r].tolist(), r
            assert wide["selected"][r].tolist() == three["selected"][r].tolist(), r
        assert orc.max_abs_diff(wide["outputs"], outs) <= 1e-4
        assert np.array_equal(wide["outputs"].view(np.uint32), three["outputs"].view(np.uint32))
    finally:
        pool.close()


@pytest.mark.parametrize("near_count,k", [(8, 8), (12, 8), (30, 16)])
def test_wide_step_near_ties(gpu, near_count, k):
    # 600 candidates of which near_count score within about 1e-3 of each
    # other at the top-k boundary: the select refines them (8) or chains
    # them exactly (12, 30), inside the wide launch.
    rng = np.random.default_rng(near_count)
    n_cand = 600
    scale = 1.0 / np.sqrt(np.float32(D))
    q = rng.standard_normal(E).astype(np.float32)
    m = int(np.argmax(np.abs(q)))
    base = (0.2 * q + 0.25 * rng.standard_normal(E)).astype(np.float32)
    summ = (0.25 * rng.standard_normal((n_cand, E))).astype(np.float32)
    for j in range(near_count):
        row = base.copy()
        row[m] = np.float32(row[m] + j * 1e-3 / (q[m] * scale))
        summ[j] = row
    keys = rng.standard_normal((n_cand, PS, E)).astype(np.float32)
    values = rng.standard_normal((n_cand, PS, E)).astype(np.float32)
    pool = gpu.DevicePagePool(H, D, PS, n_cand)
    try:
        ids = np.arange(n_cand, dtype=np.int32)
        counts = np.full(n_cand, PS, np.int32)
        pool.upload_pages(ids, counts, ids.astype(np.int64) * PS * E, keys, values, summ)
        cand = rng.permutation(n_cand).astype(np.int32)
        offs = np.array([0, n_cand], np.int32)
        with make_ctx(gpu, pool, k, 1, n_cand) as ctx:
            res = ctx.run_batch(q[None, :], offs, cand, output_mode=gpu.OUTPUT_OUTPUTS,
                                want_ids=True)
            assert ctx.last_launch()["wide"] == 1
        _, selected, outs = orc.sparse_batch(q[None, :], keys, values, summ, counts, offs, cand,
                                             H, D, PS, k)
        assert res["selected"][0].tolist() == selected[0].tolist()
        assert orc.max_abs_diff(res["outputs"], outs) <= 1e-4
    finally:
        pool.close()


def test_wide_step_device_entry_replays_and_empty_request(gpu):
    import torch

    lengths = [16 * 900, 0, 16 * 1500 + 3, 16 * 5]
    batch = gpu.SyntheticBatch(H, D, PS, lengths, seed=9)
    pool = gpu.DevicePagePool(H, D, PS, batch.capacity)
    k = 32
    try:
        batch.upload(pool)
        _, selected, outs = oracle(batch, k)
        dev = torch.device("cuda:0")
        q = torch.from_numpy(batch.queries).to(dev)
        offs = torch.from_numpy(batch.cand_offsets).to(dev)
        ids = torch.from_numpy(batch.cand_ids).to(dev)
        out = torch.full((batch.batch, E), 7.0, device=dev)
        sel = torch.full((batch.batch, k), -1, dtype=torch.int32, device=dev)
        cnt = torch.zeros(batch.batch, dtype=torch.int32, device=dev)
        total = int(batch.cand_offsets[-1])
        stream = torch.cuda.current_stream().cuda_stream
        with make_ctx(gpu, pool, k, batch.batch, total) as ctx:
            ctx.run_batch_device(batch.batch, total, batch.max_candidates, q.data_ptr(),
                                 offs.data_ptr(), ids.data_ptr(), out.data_ptr(),
                                 d_selected=sel.data_ptr(), d_counts=cnt.data_ptr(),
                                 stream=stream)
            assert ctx.last_launch()["wide"] == 1

            def check(what):
                torch.cuda.synchronize()
                ctx.device_status()
                s, c = sel.cpu().numpy(), cnt.cpu().numpy()
                for r in range(batch.batch):
                    assert int(c[r]) == len(selected[r]), (what, r)
                    assert s[r, :int(c[r])].tolist() == selected[r].tolist(), (what, r)
                assert orc.max_abs_diff(out.cpu().numpy(), outs) <= 1e-4, what
                assert not out[1].any().item(), what  # the empty request

            check("step")
            for rep in range(5):
                ctx.replay_stage(3, stream)
            check("replays")
    finally:
        pool.close()


def test_wide_step_wait_that_gives_up_raises_and_recovers(gpu):
    """The test hook makes every wait look for a tag no workgroup writes:
    each request selects nothing, every kernel ends, and the step raises;
    reset, the same context gives the oracle's results."""
    lengths = [16 * 700, 16 * 300]
    batch = gpu.SyntheticBatch(H, D, PS, lengths, seed=10)
    pool = gpu.DevicePagePool(H, D, PS, batch.capacity)
    k = 16
    try:
        batch.upload(pool)
        _, selected, outs = oracle(batch, k)
        total = int(batch.cand_offsets[-1])
        with make_ctx(gpu, pool, k, batch.batch, total) as ctx:
            ctx.set_wait_limit(64, never_ready=True)
            with pytest.raises(gpu.RuntimeFailure, match="timed out"):
                ctx.run_batch(batch.queries, batch.cand_offsets, batch.cand_ids,
                              output_mode=gpu.OUTPUT_OUTPUTS)
            assert ctx.last_launch()["wide"] == 1
            ctx.set_wait_limit(1 << 17, never_ready=False)
            res = ctx.run_batch(batch.queries, batch.cand_offsets, batch.cand_ids,
                                output_mode=gpu.OUTPUT_OUTPUTS, want_ids=True)
            for r in range(batch.batch):
                assert res["selected"][r].tolist() == selected[r].tolist(), r
            assert orc.max_abs_diff(res["outputs"], outs) <= 1e-4
            ctx.device_status()
    finally:
        pool.close()


def test_wide_step_page_size_64_with_partial_pages(gpu):
    """Pages of 64 tokens (BASELINE config 4's size), a request of 300
    pages whose last page is partial next to a short one: the wide launch
    against the oracle and, bit for bit, against the three-kernel form."""
    ps = 64
    lengths = [300 * ps - 5, 40 * ps + 7]
    batch = gpu.SyntheticBatch(H, D, ps, lengths, seed=12)
    pool = gpu.DevicePagePool(H, D, ps, batch.capacity)
    k = 32
    try:
        batch.upload(pool)
        print(f"wide step, page size {ps}: lengths {lengths}", flush=True)
        total = int(batch.cand_offsets[-1])

        def run_form(wide):
            with make_ctx(gpu, pool, k, batch.batch, total, wide) as ctx:
                res = ctx.run_batch(batch.queries, batch.cand_offsets, batch.cand_ids,
                                    output_mode=gpu.OUTPUT_OUTPUTS, want_ids=True)
                res["launch"] = ctx.last_launch()
                ctx.device_status()
            return res

        wide = run_form(True)
        three = run_form(False)
        assert wide["launch"]["wide"] == 1 and three["launch"]["wide"] == 0
        summ = np.zeros((batch.capacity, E), np.float32)
        live = batch.live_page_ids()
        summ[live] = orc.pool_summaries(batch.key_pool, batch.token_counts, E, live)
        _, selected, outs = orc.sparse_batch(batch.queries, batch.key_pool, batch.value_pool,
                                             summ, batch.token_counts, batch.cand_offsets,
                                             batch.cand_ids, H, D, ps, k)
        for r in range(batch.batch):
            assert wide["selected"][r].tolist() == selected[r].tolist(), r
            assert three["selected"][r].tolist() == selected[r].tolist(), r
        assert orc.max_abs_diff(wide["outputs"], outs) <= 1e-4
        assert np.array_equal(wide["outputs"].view(np.uint32), three["outputs"].view(np.uint32))
    finally:
        pool.close()
