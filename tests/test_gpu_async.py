"""Asynchronous table steps (dsd_sparse_run_table_async, dsd_sparse_async_wait
and dsd_sparse_async_collect, include/dsd_hip.h): the serving loop's step
enqueued without a host wait, with the step's append and release behind it
on the same stream.

Each step's results must be those of the synchronous table step on the same
table state: ids equal to the oracle's (SelectTopKPagesCpu,
/root/reference/src/reference_kernels.cpp:82-107) and outputs within 1e-4,
whether the step's queries were copied at the call or read in place from
pinned rows, and whether the host waited for the previous steps or not
(more steps than the ring holds, so ring slots are reused).  A failure a
step reports is raised by the call that waits for it, and the context keeps
working afterwards."""
from __future__ import annotations

import os

import numpy as np
import pytest

import _oracle as orc
from test_gpu_table import Mirror

pytestmark = pytest.mark.gpu

H, D, PS, K = 32, 128, 16, 8
E = H * D


def setup(gpu, rng, prompts, cap=600, max_slots=8, max_pages=64):
    pool = gpu.DevicePagePool(H, D, PS, cap)
    table = gpu.PageTable(pool, max_slots, max_pages)
    mirror = Mirror(cap, PS, E)
    ctx = gpu.SparseContext(pool, K, max_slots, max_slots * max_pages, max_slots * K)
    for s, tokens in enumerate(prompts):
        keys = rng.standard_normal((tokens, E)).astype(np.float32)
        values = rng.standard_normal((tokens, E)).astype(np.float32)
        table.admit_prompt(s, keys, values)
        mirror.prompt(table.pages(s), keys, values)
    return pool, table, mirror, ctx


def append_behind(rng, table, mirror, slots, fresh):
    """One host-row decode token per slot (enqueued after the step)."""
    before = {s: table.pages(s) for s in slots}
    keys = rng.standard_normal((len(slots), E)).astype(np.float32)
    values = rng.standard_normal((len(slots), E)).astype(np.float32)
    table.append(slots, np.ones(len(slots), np.uint8),
                 fresh_page=np.full(len(slots), 1 if fresh else 0, np.uint8),
                 keys=keys, values=values)
    for i, s in enumerate(slots):
        after = table.pages(s)
        page = int(after[-1])
        if len(after) > len(before[s]):
            mirror.counts[page] = 0
        mirror.append(page, keys[i], values[i])


def check(ctx, batch, expected):
    (_, selected, outs), _, _ = expected
    got = ctx.last_selection(batch)
    for r in range(batch):
        assert got[r].tolist() == selected[r].tolist(), r
    assert orc.max_abs_diff(ctx.staged_outputs(batch), outs) <= 1e-4


def test_async_steps_with_appends_behind_them_match_the_oracle(gpu):
    rng = np.random.default_rng(71)
    prompts = [5 * PS + 3, 17 * PS, 2 * PS - 1, 30 * PS + 7, 9 * PS]
    pool, table, mirror, ctx = setup(gpu, rng, prompts)
    slots = [3, 0, 4, 2, 1]
    B = len(slots)
    steps = 10  # more than the four ring slots
    block = gpu.HostBlock(steps * B * E)
    tickets = []
    try:
        for step in range(steps):
            q = rng.standard_normal((B, E)).astype(np.float32)
            lists = [table.pages(s) for s in slots]
            expected = mirror.oracle_step(q, lists, H, D, K)
            if step % 2 == 0:
                t = ctx.run_table_async(table, slots, queries=q)
            else:
                base = step * B * E
                block.array[base:base + B * E] = q.reshape(-1)
                rows = [block.address + 4 * (base + r * E) for r in range(B)]
                t = ctx.run_table_async(table, slots, query_rows=rows)
            assert t == step + 1
            tickets.append(t)
            append_behind(rng, table, mirror, slots, fresh=step == 0)
            if step % 3 == 0:
                # The step has completed; the append behind it has not
                # changed what it read.
                print(f"async step {step}: waited", flush=True)
                ctx.async_wait(t)
                check(ctx, B, expected)
        # The last steps ran without host waits: the last one's results.
        ctx.async_wait(tickets[-1])
        check(ctx, B, expected)
        recs = ctx.async_collect()
        assert [r["ticket"] for r in recs] == tickets
        assert all(r["batch"] == B for r in recs)
        for a, b in zip(recs, recs[1:]):
            assert a["start_ms"] <= a["done_ms"] <= b["start_ms"] <= b["done_ms"]
        assert ctx.async_collect() == []
    finally:
        ctx.close()
        block.close()
        table.close()
        pool.close()


def test_async_pipeline_with_release_and_readmission(gpu):
    """Steps over changing slot sets, releases and admissions enqueued
    behind them, no waits until the end; the last step's results and every
    step's record."""
    rng = np.random.default_rng(72)
    prompts = [12 * PS, 3 * PS + 5, 20 * PS, 7 * PS + 1]
    pool, table, mirror, ctx = setup(gpu, rng, prompts)
    try:
        slots = [0, 1, 2, 3]
        tickets = []
        for step in range(6):
            q = rng.standard_normal((len(slots), E)).astype(np.float32)
            lists = [table.pages(s) for s in slots]
            expected = mirror.oracle_step(q, lists, H, D, K)
            tickets.append(ctx.run_table_async(table, slots, queries=q,
                                               timing_mode=gpu.TIMING_EVENTS))
            if step == 2:
                table.release([1])
                tokens = 15 * PS + 2
                keys = rng.standard_normal((tokens, E)).astype(np.float32)
                values = rng.standard_normal((tokens, E)).astype(np.float32)
                table.admit_prompt(5, keys, values)
                mirror.prompt(table.pages(5), keys, values)
                slots = [5, 0, 2, 3]
            else:
                append_behind(rng, table, mirror, slots, fresh=False)
        print("async pipeline: collecting", flush=True)
        recs = ctx.async_collect()
        check(ctx, len(slots), expected)
        assert [r["ticket"] for r in recs] == tickets
        for r in recs:
            assert 0.0 < r["kernel_ms"] <= r["done_ms"] - r["start_ms"] + 2e-3
    finally:
        ctx.close()
        table.close()
        pool.close()


def test_async_steps_read_query_rows_in_device_blocks(gpu):
    """Query rows in dsd_device_alloc memory (HBM), mixed with pinned host
    rows in one step, as the pipelined loop's device query store passes
    them; both step forms agree with the oracle."""
    rng = np.random.default_rng(76)
    prompts = [8 * PS + 1, 25 * PS, 13 * PS + 9]
    pool, table, mirror, ctx = setup(gpu, rng, prompts)
    slots = [2, 0, 1]
    dev = gpu.DeviceBlock(4 * len(slots) * E)
    host = gpu.HostBlock(len(slots) * E)
    try:
        for step in range(4):
            q = rng.standard_normal((len(slots), E)).astype(np.float32)
            expected = mirror.oracle_step(q, [table.pages(s) for s in slots], H, D, K)
            rows = []
            for r in range(len(slots)):
                if (r + step) % 2 == 0:
                    off = (step * len(slots) + r) * E
                    dev.upload(q[r], off)
                    rows.append(dev.address + 4 * off)
                else:
                    host.array[r * E:(r + 1) * E] = q[r]
                    rows.append(host.address + 4 * r * E)
            t = ctx.run_table_async(table, slots, query_rows=rows)
            ctx.async_wait(t)
            check(ctx, len(slots), expected)
            res = ctx.run_table(table, slots, query_rows=rows, want_ids=True)
            (_, selected, outs), _, _ = expected
            for r in range(len(slots)):
                assert res["selected"][r].tolist() == selected[r].tolist()
            assert orc.max_abs_diff(res["outputs"], outs) <= 1e-4
            append_behind(rng, table, mirror, slots, fresh=step == 0)
        with pytest.raises(gpu.InvalidArgument):  # past the block's end
            ctx.run_table_async(table, slots[:1], query_rows=[dev.address + 4 * (dev.count - E + 4)])
        ctx.async_collect()
    finally:
        ctx.close()
        dev.close()
        host.close()
        table.close()
        pool.close()


@pytest.mark.parametrize("wide", [True, False])
def test_async_timed_wide_and_three_kernel_steps(gpu, wide):
    """Requests of more than 256 pages take the wide single launch, timed
    as a whole (its stages overlap), or with DSD_WIDE_STEP=0 the
    three-kernel step, timed by stage events."""
    rng = np.random.default_rng(75)
    old = os.environ.get("DSD_WIDE_STEP")
    os.environ["DSD_WIDE_STEP"] = "1" if wide else "0"
    try:
        pool, table, mirror, ctx = setup(gpu, rng, [300 * PS + 5, 20 * PS], cap=800,
                                         max_pages=400)
    finally:
        if old is None:
            del os.environ["DSD_WIDE_STEP"]
        else:
            os.environ["DSD_WIDE_STEP"] = old
    try:
        slots = [0, 1]
        tickets = []
        for step in range(5):
            q = rng.standard_normal((2, E)).astype(np.float32)
            expected = mirror.oracle_step(q, [table.pages(s) for s in slots], H, D, K)
            tickets.append(ctx.run_table_async(table, slots, queries=q,
                                               timing_mode=gpu.TIMING_EVENTS))
            append_behind(rng, table, mirror, slots, fresh=False)
        print(f"timed async steps (wide={wide}): collecting", flush=True)
        recs = ctx.async_collect()
        check(ctx, 2, expected)
        assert [r["ticket"] for r in recs] == tickets
        for r in recs:
            assert r["fused"] == 0 and r["wide"] == int(wide)
            if wide:
                assert r["score_ms"] == r["topk_ms"] == r["attention_ms"] == 0.0
                assert r["kernel_ms"] > 0.0
            else:
                assert min(r["score_ms"], r["topk_ms"], r["attention_ms"]) > 0.0
            assert r["kernel_ms"] <= r["done_ms"] - r["start_ms"] + 2e-3
    finally:
        ctx.close()
        table.close()
        pool.close()


def test_async_failure_is_raised_by_the_wait_and_the_context_recovers(gpu):
    """The fused step's waits forced to give up (test hook, set from the
    host): the step ends with a failure report, which the wait raises."""
    rng = np.random.default_rng(73)
    prompts = [40 * PS, 61 * PS + 3]  # fused-step sizes
    pool, table, mirror, ctx = setup(gpu, rng, prompts)
    try:
        slots = [1, 0]
        q = rng.standard_normal((2, E)).astype(np.float32)
        ctx.set_wait_limit(64, never_ready=True)
        t = ctx.run_table_async(table, slots, queries=q)
        with pytest.raises(gpu.RuntimeFailure, match="timed out"):
            ctx.async_wait(t)
        assert ctx.async_collect() == []  # its record was dropped
        ctx.set_wait_limit(1 << 17, never_ready=False)
        expected = mirror.oracle_step(q, [table.pages(s) for s in slots], H, D, K)
        t = ctx.run_table_async(table, slots, queries=q)
        ctx.async_wait(t)
        check(ctx, 2, expected)
        assert [r["ticket"] for r in ctx.async_collect()] == [t]
    finally:
        ctx.close()
        table.close()
        pool.close()


def test_async_step_rejects_bad_arguments(gpu):
    rng = np.random.default_rng(74)
    pool, table, mirror, ctx = setup(gpu, rng, [4 * PS])
    try:
        q = rng.standard_normal((1, E)).astype(np.float32)
        with pytest.raises(gpu.InvalidArgument):
            ctx.async_wait(5)  # never issued
        # rows outside dsd_host_alloc memory
        with pytest.raises(gpu.InvalidArgument):
            ctx.run_table_async(table, [0], query_rows=[q.ctypes.data])
        assert ctx.run_table_async(table, [], queries=np.zeros((0, E), np.float32)) == 0
        assert ctx.async_collect() == []
    finally:
        ctx.close()
        table.close()
        pool.close()
