"""The allocation-free entry point (dsd_sparse_run_batch_device_static: no
context, the library's static device scratch) against the context's
device-buffer entry point (dsd_sparse_run_batch_device) on the same inputs:
selected ids equal id for id and outputs bit for bit (the same kernels run),
on two calls in a row with the second smaller, for the single-launch step
and for the three-kernel step; and sizes beyond the scratch are rejected on
the host."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

H, D, PS = 32, 128, 16
E = H * D


def device(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def sub_batch(batch, n):
    """Requests 0 .. n-1 of a SyntheticBatch (same pool pages)."""
    offs = batch.cand_offsets[:n + 1].copy()
    return batch.queries[:n].copy(), offs, batch.cand_ids[:offs[-1]].copy()


def both_entries(gpu, pool, k, queries, offs, ids, static_ids):
    """(context path, static path) results: outputs, and ids/counts."""
    import torch
    B = len(offs) - 1
    total = int(offs[-1])
    max_n = int(np.max(np.diff(offs)))
    q, o, i = device(queries), device(offs), device(ids)
    out_ctx = torch.zeros((B, E), device="cuda:0")
    out_st = torch.full((B, E), 3.0, device="cuda:0")
    sel_ctx = torch.full((B, max(k, 1)), -1, dtype=torch.int32, device="cuda:0")
    cnt_ctx = torch.full((B,), -1, dtype=torch.int32, device="cuda:0")
    sel_st = torch.full((B, max(k, 1)), -1, dtype=torch.int32, device="cuda:0")
    cnt_st = torch.full((B,), -1, dtype=torch.int32, device="cuda:0")
    fail = torch.zeros(1, dtype=torch.int64, device="cuda:0")
    sel_total = int(sum(min(k, int(n)) for n in np.diff(offs)))
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream().cuda_stream
    with gpu.SparseContext(pool, k, B, total, sel_total) as ctx:
        ctx.run_batch_device(B, total, max_n, q.data_ptr(), o.data_ptr(), i.data_ptr(),
                             out_ctx.data_ptr(), d_selected=sel_ctx.data_ptr(),
                             d_counts=cnt_ctx.data_ptr(), stream=stream)
        torch.cuda.synchronize()
        ctx.device_status()
        info = ctx.last_launch()
    gpu.sparse_run_batch_device_static(
        pool, k, B, total, max_n, q.data_ptr(), o.data_ptr(), i.data_ptr(), out_st.data_ptr(),
        d_selected=sel_st.data_ptr() if static_ids else 0,
        d_counts=cnt_st.data_ptr() if static_ids else 0, d_fail=fail.data_ptr(), stream=stream)
    torch.cuda.synchronize()
    assert int(fail.item()) == 0
    res = {"info": info, "out_ctx": out_ctx.cpu().numpy(), "out_st": out_st.cpu().numpy(),
           "sel_ctx": sel_ctx.cpu().numpy(), "cnt_ctx": cnt_ctx.cpu().numpy(),
           "sel_st": sel_st.cpu().numpy(), "cnt_st": cnt_st.cpu().numpy()}
    assert np.array_equal(res["out_st"].view(np.uint32), res["out_ctx"].view(np.uint32))
    if static_ids:
        assert res["cnt_st"].tolist() == res["cnt_ctx"].tolist()
        for r in range(B):
            c = int(res["cnt_ctx"][r])
            assert res["sel_st"][r, :c].tolist() == res["sel_ctx"][r, :c].tolist(), r
    return res


@pytest.mark.parametrize("lengths,k,fused", [
    (None, 8, True),                                  # the fused step
    ([600 * PS, 40, 2100, 16 * PS], 8, False),        # > 512 candidates: three kernels
])
def test_static_entry_equals_the_context_entry(gpu, lengths, k, fused):
    if lengths is None:
        lengths = gpu.reference_context_lengths(16, 512, 2048, 7)
    batch = gpu.SyntheticBatch(H, D, PS, lengths, seed=43)
    with gpu.DevicePagePool(H, D, PS, batch.capacity) as pool:
        batch.upload(pool)
        # first call: the whole batch, ids and counts in the static scratch
        first = both_entries(gpu, pool, k, batch.queries, batch.cand_offsets, batch.cand_ids,
                             static_ids=False)
        assert first["info"]["fused"] == int(fused), first["info"]
        # second call, right after: a smaller batch, ids returned
        n = max(1, batch.batch // 3)
        second = both_entries(gpu, pool, k, *sub_batch(batch, n), static_ids=True)
        assert second["out_st"].shape[0] == n


def test_static_entry_allocates_nothing(gpu):
    """After a first call on the device (which looks up the scratch's
    address and loads the kernels), further calls -- the fused step and the
    three-kernel step, ids kept in the scratch -- leave the device's free
    memory unchanged: no hipMalloc, no hipFree, no allocating library call."""
    import torch
    batch = gpu.SyntheticBatch(H, D, PS, [300, 517, 600 * PS, 90], seed=5)
    with gpu.DevicePagePool(H, D, PS, batch.capacity) as pool:
        batch.upload(pool)
        B = batch.batch
        cases = []
        for n in (2, B):  # two requests: fused; all four (> 512 candidates): three kernels
            queries, offs, ids = sub_batch(batch, n)
            cases.append((n, int(offs[-1]), int(np.max(np.diff(offs))), device(queries),
                          device(offs), device(ids), torch.zeros((n, E), device="cuda:0")))
        fail = torch.zeros(1, dtype=torch.int64, device="cuda:0")
        stream = torch.cuda.current_stream().cuda_stream

        def calls():
            for n, total, max_n, q, o, i, out in cases:
                gpu.sparse_run_batch_device_static(pool, 8, n, total, max_n, q.data_ptr(),
                                                   o.data_ptr(), i.data_ptr(), out.data_ptr(),
                                                   d_fail=fail.data_ptr(), stream=stream)
            torch.cuda.synchronize()

        calls()
        free_before = torch.cuda.mem_get_info()[0]
        for _ in range(3):
            calls()
        free_after = torch.cuda.mem_get_info()[0]
        assert int(fail.item()) == 0
        assert free_after == free_before, (free_before, free_after)


def test_static_entry_rejects_sizes_beyond_its_scratch(gpu):
    batch = gpu.SyntheticBatch(H, D, PS, [64], seed=1)
    with gpu.DevicePagePool(H, D, PS, batch.capacity) as pool:
        for b, total, k, msg in [(1025, 4, 8, "1024 requests"), (1, 65537, 8, "65536 candidates"),
                                 (1024, 4, 65, "selected ids")]:
            with pytest.raises(gpu.InvalidArgument, match=msg):
                gpu.sparse_run_batch_device_static(pool, k, b, total, 4, 16, 16, 16, 16)
