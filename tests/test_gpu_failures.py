"""Input failures of a step are reported for the launch that met them, and
every kernel still exits normally.

The host-buffer step checks its inputs on the host (as the reference's
RunBatch, src/cuda/sparse_batched_attention.cu:600-608).  The device-buffer
step cannot: its kernels check the CSR and the page ids themselves, skip
what they cannot use (that request selects nothing and its outputs are
zeros) and leave an epoch-tagged failure word that the host step ignores
unless it is its own, and dsd_sparse_device_status reports.  The single-launch
step's bounded waits give up after a spin limit the host sets; a test hook
makes every wait look for a tag no workgroup writes, so that path runs
without any real stall."""
from __future__ import annotations

import os

import numpy as np
import pytest

import _oracle as orc

pytestmark = pytest.mark.gpu

H, D, PS = 32, 128, 16
E = H * D


def make_ctx(gpu, pool, k, batch, fused, max_total=None):
    total = max_total if max_total is not None else int(batch.cand_offsets[-1])
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


def oracle_step(batch, k):
    summ = np.zeros((batch.capacity, E), np.float32)
    live = batch.live_page_ids()
    summ[live] = orc.pool_summaries(batch.key_pool, batch.token_counts, E, live)
    return orc.sparse_batch(batch.queries, batch.key_pool, batch.value_pool, summ,
                            batch.token_counts, batch.cand_offsets, batch.cand_ids, H, D, PS, k)


def device_inputs(batch):
    import torch
    dev = torch.device("cuda:0")
    return (torch.from_numpy(batch.queries).to(dev), torch.from_numpy(batch.cand_offsets).to(dev),
            torch.from_numpy(batch.cand_ids).to(dev),
            torch.full((batch.batch, E), 7.0, device=dev))


def check_against_oracle(res, batch, selected, outs, rows):
    for r in rows:
        assert res["selected"][r].tolist() == selected[r].tolist(), r
        assert orc.max_abs_diff(res["outputs"][r], outs[r]) <= 1e-4, r


@pytest.mark.parametrize("fused", [True, False])
def test_device_failure_does_not_fail_a_later_host_step(gpu, fused):
    """A device-buffer step with an understated max_candidates leaves its
    failure; the next host-buffer step (its own inputs fine) succeeds with
    the oracle's results; dsd_sparse_device_status then reports the earlier
    failure once."""
    import torch

    lengths = [300 * PS, 40, 700]           # request 0: 300 candidates
    batch = gpu.SyntheticBatch(H, D, PS, lengths, seed=19)
    pool = gpu.DevicePagePool(H, D, PS, batch.capacity)
    batch.upload(pool)
    q, offs, ids, out = device_inputs(batch)
    _, selected, outs = oracle_step(batch, 8)
    with make_ctx(gpu, pool, 8, batch, fused) as ctx:
        # understated: 200 < 300 (fused: the kernel checks each request
        # against it; three-kernel: only 200 candidates were scored)
        ctx.run_batch_device(batch.batch, batch.total_candidates, 200, q.data_ptr(),
                             offs.data_ptr(), ids.data_ptr(), out.data_ptr(),
                             stream=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert not got[0].any()                                   # skipped: zeros
        assert orc.max_abs_diff(got[1:], outs[1:]) <= 1e-4        # the others are fine
        res = ctx.run_batch(batch.queries, batch.cand_offsets, batch.cand_ids,
                            output_mode=gpu.OUTPUT_OUTPUTS, want_ids=True)
        check_against_oracle(res, batch, selected, outs, range(batch.batch))
        with pytest.raises(gpu.InvalidArgument, match="max_candidates"):
            ctx.device_status()
        ctx.device_status()                                       # reported once
    pool.close()


@pytest.mark.parametrize("fused", [True, False])
def test_device_csr_beyond_total_is_skipped_and_reported(gpu, fused):
    """offsets[B] above the total_candidates the launch was given: the
    requests whose lists end past it are skipped (no write beyond the
    intervals the context holds), the others match the oracle."""
    import torch

    lengths = [900, 1300, 600]
    batch = gpu.SyntheticBatch(H, D, PS, lengths, seed=23)
    pool = gpu.DevicePagePool(H, D, PS, batch.capacity)
    batch.upload(pool)
    q, offs, ids, out = device_inputs(batch)
    _, selected, outs = oracle_step(batch, 8)
    short = int(batch.cand_offsets[2]) + 3          # request 2's list ends past it
    with make_ctx(gpu, pool, 8, batch, fused, max_total=short) as ctx:
        ctx.run_batch_device(batch.batch, short, batch.max_candidates, q.data_ptr(),
                             offs.data_ptr(), ids.data_ptr(), out.data_ptr(),
                             stream=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert not got[2].any()
        assert orc.max_abs_diff(got[:2], outs[:2]) <= 1e-4
        with pytest.raises(gpu.InvalidArgument):
            ctx.device_status()
    pool.close()


@pytest.mark.parametrize("fused", [True, False])
def test_device_page_id_outside_the_pool_is_reported(gpu, fused):
    """A device CSR listing a page id past the pool's capacity: the id scores
    as an empty page and is never read as K/V (the kernels' own range
    checks); the step finishes and dsd_sparse_device_status raises
    out_of_range."""
    import torch

    lengths = [400, 500]
    batch = gpu.SyntheticBatch(H, D, PS, lengths, seed=29)
    pool = gpu.DevicePagePool(H, D, PS, batch.capacity)
    batch.upload(pool)
    q, offs, ids, out = device_inputs(batch)
    ids[3] = batch.capacity + 1000
    with make_ctx(gpu, pool, 8, batch, fused) as ctx:
        ctx.run_batch_device(batch.batch, batch.total_candidates, batch.max_candidates,
                             q.data_ptr(), offs.data_ptr(), ids.data_ptr(), out.data_ptr(),
                             stream=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert np.isfinite(out.cpu().numpy()).all()
        with pytest.raises(gpu.OutOfRange):
            ctx.device_status()
        # and the host-buffer step still rejects such an id on the host
        bad = batch.cand_ids.copy()
        bad[3] = batch.capacity + 1000
        with pytest.raises(gpu.OutOfRange):
            ctx.run_batch(batch.queries, batch.cand_offsets, bad,
                          output_mode=gpu.OUTPUT_OUTPUTS)
    pool.close()


def test_fused_wait_that_gives_up_raises_and_the_context_recovers(gpu):
    """The single-launch step's waits give up after the spin limit: with the
    test hook every wait looks for a tag no workgroup writes, so each request
    selects nothing, the kernel ends, and the host step raises instead of
    returning zeros.  Reset, the same context gives the oracle's results."""
    import torch

    lengths = gpu.reference_context_lengths(8, 512, 2048, 31)
    batch = gpu.SyntheticBatch(H, D, PS, lengths, seed=31)
    pool = gpu.DevicePagePool(H, D, PS, batch.capacity)
    batch.upload(pool)
    _, selected, outs = oracle_step(batch, 8)
    q, offs, ids, out = device_inputs(batch)
    with make_ctx(gpu, pool, 8, batch, True) as ctx:
        ctx.set_wait_limit(64, never_ready=True)
        with pytest.raises(gpu.RuntimeFailure, match="timed out"):
            ctx.run_batch(batch.queries, batch.cand_offsets, batch.cand_ids,
                          output_mode=gpu.OUTPUT_OUTPUTS)
        ctx.run_batch_device(batch.batch, batch.total_candidates, batch.max_candidates,
                             q.data_ptr(), offs.data_ptr(), ids.data_ptr(), out.data_ptr(),
                             stream=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert not out.any().item()
        with pytest.raises(gpu.RuntimeFailure, match="timed out"):
            ctx.device_status()
        ctx.set_wait_limit(1 << 17, never_ready=False)
        res = ctx.run_batch(batch.queries, batch.cand_offsets, batch.cand_ids,
                            output_mode=gpu.OUTPUT_OUTPUTS, want_ids=True)
        check_against_oracle(res, batch, selected, outs, range(batch.batch))
        ctx.device_status()
    pool.close()


def test_steps_alternating_between_streams_stay_ordered(gpu):
    """Device-buffer steps on two caller streams and host-buffer steps on the
    context's stream, interleaved without host waits: they share the
    context's scratch (publication words, intervals, ids), so each launch on
    a new stream is ordered after the previous stream's work.  Every output
    equals the oracle's."""
    import torch

    lengths = gpu.reference_context_lengths(16, 512, 2048, 37)
    batch = gpu.SyntheticBatch(H, D, PS, lengths, seed=37)
    pool = gpu.DevicePagePool(H, D, PS, batch.capacity)
    batch.upload(pool)
    _, selected, outs = oracle_step(batch, 8)
    q, offs, ids, _ = device_inputs(batch)
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    outs_dev = [torch.zeros((batch.batch, E), device="cuda:0") for _ in range(9)]
    torch.cuda.synchronize()          # the zero fills ran on torch's stream
    results = []
    with make_ctx(gpu, pool, 8, batch, True) as ctx:
        for rnd in range(3):
            for j, s in enumerate((sa, sb, sa)):
                o = outs_dev[3 * rnd + j]
                ctx.run_batch_device(batch.batch, batch.total_candidates, batch.max_candidates,
                                     q.data_ptr(), offs.data_ptr(), ids.data_ptr(),
                                     o.data_ptr(), stream=s.cuda_stream)
                results.append((s, o))
            res = ctx.run_batch(batch.queries, batch.cand_offsets, batch.cand_ids,
                                output_mode=gpu.OUTPUT_OUTPUTS, want_ids=True)
            check_against_oracle(res, batch, selected, outs, range(batch.batch))
        torch.cuda.synchronize()
        for s, o in results:
            assert orc.max_abs_diff(o.cpu().numpy(), outs) <= 1e-4
        ctx.device_status()
    pool.close()
