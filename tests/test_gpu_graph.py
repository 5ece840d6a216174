"""The device step captured into a HIP graph (torch.cuda.CUDAGraph on a side
stream) and replayed: the context entry point (dsd_sparse_run_batch_device)
and the allocation-free one (dsd_sparse_run_batch_device_static), for the
single-launch step and the three-kernel step.  For 600-page requests the
context runs the wide single launch (captured too), or three kernels when
created with DSD_WIDE_STEP=0; the static entry runs three kernels there.

The fused and wide steps' workgroups exchange their score intervals through
words tagged with the launch's epoch.  A captured launch takes its epoch from
a device counter that a one-thread kernel, captured with it, advances on
every replay (for the wide step the same kernel also advances the count that
picks which of two item-counter sets the replay uses); with an epoch frozen at capture, a replay would read the
previous replay's intervals as current.  So the queries change between
replays (and an eager step on other data runs between two of them), and
every replay must give, bit for bit, the ids and outputs of an eager step
on the same queries; the first set is also checked against the oracle."""
from __future__ import annotations

import os

import numpy as np
import pytest

import _oracle as orc

pytestmark = pytest.mark.gpu

H, D, PS = 32, 128, 16
E = H * D


def device(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


@pytest.mark.parametrize("entry", ["context", "context_three", "static"])
@pytest.mark.parametrize("lengths,fused", [
    ([629, 861, 1710, 1002, 1185, 2015], True),       # the single-launch step
    ([600 * PS, 40, 2100, 16 * PS], False),           # > 512 candidates: wide / three kernels
])
def test_graph_replays_follow_new_inputs(gpu, entry, lengths, fused):
    import torch
    k = 8
    batch = gpu.SyntheticBatch(H, D, PS, lengths, seed=61)
    B = len(lengths)
    offs, ids = batch.cand_offsets.copy(), batch.cand_ids.copy()
    total = int(offs[-1])
    max_n = int(np.max(np.diff(offs)))
    sel_total = int(sum(min(k, int(n)) for n in np.diff(offs)))
    rng = np.random.default_rng(62)
    query_sets = [batch.queries.copy()] + [rng.standard_normal((B, E)).astype(np.float32)
                                           for _ in range(3)]
    print(f"[graph] entry={entry} fused={fused} B={B} candidates={total}", flush=True)
    with gpu.DevicePagePool(H, D, PS, batch.capacity) as pool:
        batch.upload(pool)
        q, o, i = device(query_sets[0]), device(offs), device(ids)
        out = torch.zeros((B, E), device="cuda:0")
        sel = torch.full((B, k), -1, dtype=torch.int32, device="cuda:0")
        cnt = torch.full((B,), -1, dtype=torch.int32, device="cuda:0")
        fail = torch.zeros(1, dtype=torch.int64, device="cuda:0")
        ctx = None
        if entry != "static":
            # context_three: DSD_WIDE_STEP=0 at the context's creation, so a
            # wide-shaped step captures the three kernels
            old = os.environ.get("DSD_WIDE_STEP")
            os.environ["DSD_WIDE_STEP"] = "0" if entry == "context_three" else "1"
            try:
                ctx = gpu.SparseContext(pool, k, B, total, sel_total)
            finally:
                if old is None:
                    del os.environ["DSD_WIDE_STEP"]
                else:
                    os.environ["DSD_WIDE_STEP"] = old

        def step(stream):
            if ctx is not None:
                ctx.run_batch_device(B, total, max_n, q.data_ptr(), o.data_ptr(), i.data_ptr(),
                                     out.data_ptr(), d_selected=sel.data_ptr(),
                                     d_counts=cnt.data_ptr(), stream=stream)
            else:
                gpu.sparse_run_batch_device_static(
                    pool, k, B, total, max_n, q.data_ptr(), o.data_ptr(), i.data_ptr(),
                    out.data_ptr(), d_selected=sel.data_ptr(), d_counts=cnt.data_ptr(),
                    d_fail=fail.data_ptr(), stream=stream)

        def result():
            return out.cpu().numpy().copy(), sel.cpu().numpy().copy(), cnt.cpu().numpy().copy()

        def same(got, want, what):
            assert np.array_equal(got[0].view(np.uint32), want[0].view(np.uint32)), what
            assert got[2].tolist() == want[2].tolist(), what
            for r in range(B):
                c = int(want[2][r])
                assert got[1][r, :c].tolist() == want[1][r, :c].tolist(), (what, r)

        eager = []
        main = torch.cuda.current_stream().cuda_stream
        for qs in query_sets:
            q.copy_(torch.from_numpy(qs))
            torch.cuda.synchronize()
            step(main)
            torch.cuda.synchronize()
            eager.append(result())
        wide = not fused and entry == "context"
        if ctx is not None:
            info = ctx.last_launch()
            assert bool(info["fused"]) == fused, info
            assert bool(info["wide"]) == wide, info
        # the first set against the oracle
        summ = orc.pool_summaries(batch.key_pool, batch.token_counts, E)
        _, want_sel, want_out = orc.sparse_batch(query_sets[0], batch.key_pool, batch.value_pool,
                                                 summ, batch.token_counts, offs, ids, H, D, PS, k)
        for r in range(B):
            assert eager[0][1][r, :int(eager[0][2][r])].tolist() == want_sel[r].tolist(), r
        assert orc.max_abs_diff(eager[0][0], want_out) <= 1e-4

        side = torch.cuda.Stream()
        graph = torch.cuda.CUDAGraph()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            step(side.cuda_stream)
        torch.cuda.synchronize()
        if ctx is not None:
            info = ctx.last_launch()
            assert bool(info["fused"]) == fused and bool(info["wide"]) == wide, info
        for rep, idx in enumerate([1, 2, 0, 3, 1, 2]):
            q.copy_(torch.from_numpy(query_sets[idx]))
            out.fill_(7.0)
            sel.fill_(-1)
            cnt.fill_(-1)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            same(result(), eager[idx], f"replay {rep} (query set {idx})")
            if rep == 2:
                # an eager step on other data between two replays
                q.copy_(torch.from_numpy(query_sets[3]))
                torch.cuda.synchronize()
                step(main)
                torch.cuda.synchronize()
                same(result(), eager[3], "eager step between replays")
        if ctx is not None:
            ctx.device_status()
            ctx.close()
        assert int(fail.item()) == 0
