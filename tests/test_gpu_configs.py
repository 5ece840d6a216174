"""BASELINE configs 3 and 4 at their full size, in the launch forms the
bench times, against the oracle.

    config 3: B=32, 32768 tokens each (2048 pages of 16), top-k 64, seed 11
              -> the wide single launch: 128 pages per score slice, the
                 2048-candidate certified select by each request's last
                 slice, attention one head per item; bit-equal to the same step
                 in three kernels; also dense over the same pages (the
                 crossover's dense side) against dense_cpu
    config 4: B=64, contexts U[4096, 16384] (seed 13), page 64, top-k 32
              -> the single-launch step, multi-pass form, 8 heads per
                 workgroup

Selections must equal the oracle's sparse_cpu (score -> top-k) id vector for
id vector (the bar of the reference's tests/test_sparse_cuda.cpp:62) and
outputs must be within 1e-4 (BASELINE's bound).  The oracle streams one
request at a time: each worker generates a request's K/V (its own numpy
stream), uploads it, and runs the oracle's score, select and attention on it,
so host memory stays at a few GiB even though config 3 holds 34 GB of K/V in
HBM."""
from __future__ import annotations

import concurrent.futures as cf
import os
import threading

import numpy as np
import pytest

import _oracle as orc

pytestmark = pytest.mark.gpu

TOL = 1e-4
H, D = 32, 128
E = H * D


def stream_oracle(gpu, batch, pool, k, dense=False, workers=8):
    """Upload every request (device summaries) and return the oracle's
    (selected ids per request, sparse outputs [B][E], dense outputs or
    None), one request's K/V in host memory per worker."""
    B = batch.batch
    lock = threading.Lock()
    selected = [None] * B
    sparse_out = np.zeros((B, E), np.float32)
    dense_out = np.zeros((B, E), np.float32) if dense else None

    def work(r):
        keys, values = batch.request_pages(r)
        with lock:
            batch.upload_request(pool, r, keys, values)
        ids = batch.request_ids(r)
        sel, out, dout = orc.request_step(batch.queries[r], keys, values,
                                          batch.token_counts[ids], ids, H, D,
                                          batch.page_size, k, dense=dense)
        selected[r] = sel
        sparse_out[r] = out
        if dense:
            dense_out[r] = dout

    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        for f in [ex.submit(work, r) for r in range(B)]:
            f.result()
    return selected, sparse_out, dense_out


def run_config(gpu, lengths, ps, k, seed, dense=False):
    batch = gpu.SyntheticBatch(H, D, ps, lengths, seed=seed)
    pool = gpu.DevicePagePool(H, D, ps, batch.capacity)
    selected, sparse_out, dense_out = stream_oracle(gpu, batch, pool, k, dense=dense)
    sel_total = int(sum(min(k, int(n)) for n in np.diff(batch.cand_offsets)))
    ctx = gpu.SparseContext(pool, k, batch.batch, batch.total_candidates, sel_total)
    res = ctx.run_batch(batch.queries, batch.cand_offsets, batch.cand_ids,
                        output_mode=gpu.OUTPUT_OUTPUTS, want_ids=True)
    for r in range(batch.batch):
        assert res["selected"][r].tolist() == selected[r].tolist(), r
    diff = orc.max_abs_diff(res["outputs"], sparse_out)
    assert diff <= TOL, diff
    return batch, pool, ctx, res, dense_out


def device_step_equals_host_step(gpu, batch, ctx, res):
    """The device-buffer entry point (what bench.py times) launches the same
    kernels: its outputs equal the host step's bit for bit."""
    import torch

    dev = torch.device("cuda:0")
    q = torch.from_numpy(batch.queries).to(dev)
    offs = torch.from_numpy(batch.cand_offsets).to(dev)
    ids = torch.from_numpy(batch.cand_ids).to(dev)
    out = torch.zeros_like(q)
    torch.cuda.synchronize()
    ctx.run_batch_device(batch.batch, batch.total_candidates, batch.max_candidates,
                         q.data_ptr(), offs.data_ptr(), ids.data_ptr(), out.data_ptr(),
                         stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    ctx.device_status()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), res["outputs"].view(np.uint32))
    return ctx.last_launch()


def test_config3_full_batch_wide_step(gpu):
    lengths = gpu.reference_context_lengths(32, 32768, 32768, 11)
    batch, pool, ctx, res, dense_out = run_config(gpu, lengths, 16, 64, 11, dense=True)
    assert batch.total_candidates == 65536
    info = ctx.last_launch()
    assert info["wide"] == 1 and info["fused"] == 0 and info["certified"] == 1, info
    # 16 score slices of 128 pages and 32 heads per request (1536 items),
    # launched with 768 spare workgroups
    assert info["score_pages_per_group"] == 128 and info["grid"] == 2304, info
    assert device_step_equals_host_step(gpu, batch, ctx, res) == info
    # The same step in three kernels (DSD_WIDE_STEP=0): bit-equal.
    sel_total = int(sum(min(64, int(n)) for n in np.diff(batch.cand_offsets)))
    os.environ["DSD_WIDE_STEP"] = "0"
    try:
        three = gpu.SparseContext(pool, 64, batch.batch, batch.total_candidates, sel_total)
    finally:
        del os.environ["DSD_WIDE_STEP"]
    res3 = three.run_batch(batch.queries, batch.cand_offsets, batch.cand_ids,
                           output_mode=gpu.OUTPUT_OUTPUTS, want_ids=True)
    assert three.last_launch()["wide"] == 0
    for r in range(batch.batch):
        assert res3["selected"][r].tolist() == res["selected"][r].tolist(), r
    assert np.array_equal(res3["outputs"].view(np.uint32), res["outputs"].view(np.uint32))
    three.close()
    # dense_gpu on the identical inputs vs dense_cpu (the crossover's other side)
    dense, _ = gpu.dense_run_batch(pool, batch.queries, batch.cand_offsets, batch.cand_ids)
    diff = orc.max_abs_diff(dense, dense_out)
    assert diff <= TOL, diff
    ctx.close()
    pool.close()


def test_config4_full_batch_multi_pass_fused_step(gpu):
    lengths = gpu.reference_context_lengths(64, 4096, 16384, 13)
    assert sum(lengths) == 686494 and min(lengths) == 4203 and max(lengths) == 16302
    batch, pool, ctx, res, _ = run_config(gpu, lengths, 64, 32, 13)
    assert batch.total_candidates == 10758
    info = ctx.last_launch()
    assert info["fused"] == 1 and info["multi_pass"] == 1, info
    assert info["heads_per_group"] == 8 and info["grid"] == 64 * 4, info
    assert device_step_equals_host_step(gpu, batch, ctx, res) == info
    ctx.close()
    pool.close()
