"""The device request -> page table (dsd_table_*, include/dsd_hip.h) and the
step that packs its candidate lists on the device (dsd_sparse_run_table).

Page order: tests/native/table_check runs seeded sequences of admissions,
appends and releases on the table and on the host paged KV cache of the
reference API (the reference's PagePool / PagedKvCache order) and compares
every page list and the free stack.  Step parity: a table step's candidate
lists are the table's page lists, its outputs and ids equal the host-CSR
step's bit for bit and the oracle's within 1e-4, including after appended
tokens (running-mean summaries) and releases that recycle pages."""
from __future__ import annotations

import pathlib
import subprocess

import numpy as np
import pytest

import _oracle as orc

pytestmark = pytest.mark.gpu

EXE = pathlib.Path(__file__).resolve().parent / "native" / "build" / "table_check"


@pytest.mark.parametrize("capacity,slots,ops,seed", [(64, 8, 400, 1), (300, 32, 1500, 2),
                                                     (40, 40, 800, 3)])
def test_table_page_order_matches_host_cache(gpu, capacity, slots, ops, seed):
    if not EXE.exists():
        pytest.fail(f"{EXE} is not built (__graft_entry__.build() builds tests/native)")
    print(f"table_check {capacity} {slots} {ops} {seed}", flush=True)
    proc = subprocess.run([str(EXE), str(capacity), str(slots), str(ops), str(seed)],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "table_check ok" in proc.stdout


class Mirror:
    """The pool's contents as the host knows them (keys, values, counts and
    summaries per page id), kept with the host cache's rules, and the
    table's page lists read back from the device."""

    def __init__(self, cap, ps, E):
        self.keys = np.zeros((cap, ps, E), np.float32)
        self.values = np.zeros((cap, ps, E), np.float32)
        self.counts = np.zeros(cap, np.int32)
        self.summ = np.zeros((cap, E), np.float32)
        self.ps, self.E = ps, E

    def prompt(self, pages, keys, values):
        for j, p in enumerate(pages):
            t0, t1 = j * self.ps, min(len(keys), (j + 1) * self.ps)
            n = t1 - t0
            self.keys[p, :n] = keys[t0:t1]
            self.values[p, :n] = values[t0:t1]
            self.counts[p] = n
            self.summ[p] = orc.page_summary(self.keys[p, :n], n, self.E)

    def append(self, page, key, value):
        old = int(self.counts[page])
        self.keys[page, old] = key
        self.values[page, old] = value
        self.summ[page] = orc.append_summary(self.summ[page], key, old) if old else key
        self.counts[page] = old + 1

    def oracle_step(self, queries, lists, H, D, k):
        offs = np.zeros(len(lists) + 1, np.int32)
        offs[1:] = np.cumsum([len(x) for x in lists])
        ids = np.concatenate(lists).astype(np.int32) if lists else np.zeros(0, np.int32)
        return orc.sparse_batch(queries, self.keys, self.values, self.summ, self.counts, offs,
                                ids, H, D, self.ps, k), offs, ids


def check_step(gpu, ctx, table, mirror, slots, queries, H, D, k):
    res = ctx.run_table(table, slots, queries=queries, want_ids=True)
    lists = [table.pages(s) for s in slots]
    offs, ids = ctx.last_csr(len(slots))
    want_offs = np.zeros(len(slots) + 1, np.int32)
    want_offs[1:] = np.cumsum([len(x) for x in lists])
    assert offs.tolist() == want_offs.tolist()
    assert ids.tolist() == np.concatenate(lists).tolist()
    # the same candidate lists through the host CSR: bit-equal
    host = ctx.run_batch(queries, offs, ids, output_mode=gpu.OUTPUT_OUTPUTS, want_ids=True)
    assert np.array_equal(res["outputs"].view(np.uint32), host["outputs"].view(np.uint32))
    for r in range(len(slots)):
        assert res["selected"][r].tolist() == host["selected"][r].tolist()
    (_, selected, outs), _, _ = mirror.oracle_step(queries, lists, H, D, k)
    for r in range(len(slots)):
        assert res["selected"][r].tolist() == selected[r].tolist(), r
    assert orc.max_abs_diff(res["outputs"], outs) <= 1e-4
    return lists


@pytest.mark.parametrize("H,D,ps,k", [(32, 128, 16, 8), (4, 32, 8, 3)])
def test_table_steps_match_csr_steps_and_oracle(gpu, H, D, ps, k):
    rng = np.random.default_rng(H + k)
    E = H * D
    cap, max_slots, max_pages = 400, 12, 64
    pool = gpu.DevicePagePool(H, D, ps, cap)
    table = gpu.PageTable(pool, max_slots, max_pages)
    mirror = Mirror(cap, ps, E)
    ctx = gpu.SparseContext(pool, k, max_slots, max_slots * max_pages, max_slots * k)
    live = {}
    # admissions: prompts of 0..40*ps tokens (an empty one included)
    for s, tokens in enumerate([5 * ps + 3, 0, 17 * ps, 1, 2 * ps - 1, 30 * ps + 7]):
        keys = rng.standard_normal((tokens, E)).astype(np.float32)
        values = rng.standard_normal((tokens, E)).astype(np.float32)
        table.admit_prompt(s, keys, values)
        pages = table.pages(s)
        assert len(pages) == -(-tokens // ps) and pages.tolist() == sorted(pages.tolist())
        mirror.prompt(pages, keys, values)
        live[s] = tokens
    assert table.free_pages() == cap - sum(-(-t // ps) for t in live.values())
    slots = [3, 0, 5, 2, 4, 1]
    q = rng.standard_normal((len(slots), E)).astype(np.float32)
    check_step(gpu, ctx, table, mirror, slots, q, H, D, k)
    # decode tokens with host rows: the first starts a fresh page
    for step in range(ps + 3):
        up = np.ones(len(slots), np.uint8)
        fresh = np.array([1 if step == 0 else 0] * len(slots), np.uint8)
        before = {s: table.pages(s) for s in slots}
        keys = rng.standard_normal((len(slots), E)).astype(np.float32)
        values = rng.standard_normal((len(slots), E)).astype(np.float32)
        table.append(slots, up, fresh_page=fresh, keys=keys, values=values)
        for i, s in enumerate(slots):
            after = table.pages(s)
            page = int(after[-1])
            if len(after) > len(before[s]):
                mirror.counts[page] = 0
            mirror.append(page, keys[i], values[i])
        q = rng.standard_normal((len(slots), E)).astype(np.float32)
        check_step(gpu, ctx, table, mirror, slots, q, H, D, k)
    # release two requests, admit one into their pages
    table.release([0, 3])
    tokens = 9 * ps + 2
    keys = rng.standard_normal((tokens, E)).astype(np.float32)
    values = rng.standard_normal((tokens, E)).astype(np.float32)
    table.admit_prompt(7, keys, values)
    mirror.prompt(table.pages(7), keys, values)
    slots = [7, 5, 2, 4, 1]
    q = rng.standard_normal((len(slots), E)).astype(np.float32)
    check_step(gpu, ctx, table, mirror, slots, q, H, D, k)
    ctx.close()
    table.close()
    pool.close()


def test_table_synthetic_admission_and_append_match_the_pool_calls(gpu):
    # The table's synthetic prompt and decode payloads are the pool calls'
    # (dsd_pool_prefill_synthetic / dsd_pool_append_synthetic) on the same
    # page ids: pages downloaded from both pools must be equal bit for bit.
    H, D, ps = 4, 32, 8
    E = H * D
    cap = 64
    a = gpu.DevicePagePool(H, D, ps, cap)
    b = gpu.DevicePagePool(H, D, ps, cap)
    table = gpu.PageTable(a, 4, 32)
    tokens = 3 * ps + 5
    table.admit_synthetic(1, tokens, 42)
    pages = table.pages(1)
    counts = [min(ps, tokens - j * ps) for j in range(len(pages))]
    b.prefill_synthetic(pages, counts, 42)
    for step in range(ps + 2):
        table.append([1], [1], fresh_page=[1 if step == 0 else 0], request_ids=[42],
                      decode_steps=[step])
    pages_after = table.pages(1)
    # the same tokens through the pool call, page by page
    tail = [int(p) for p in pages_after[len(pages):]]
    off = 0
    for step in range(ps + 2):
        page = tail[0] if step < ps else tail[1]
        off = step if step < ps else step - ps
        b.append_synthetic([page], [off], [off + 1], [42], [step])
    for p in pages_after:
        ka, va = a.download_page(int(p))
        kb, vb = b.download_page(int(p))
        assert ka.size == kb.size > 0
        assert np.array_equal(ka.view(np.uint32), kb.view(np.uint32))
        assert np.array_equal(va.view(np.uint32), vb.view(np.uint32))
    sa = a.download_summaries(pages_after)
    sb = b.download_summaries(pages_after)
    assert np.array_equal(sa.view(np.uint32), sb.view(np.uint32))
    table.close()
    a.close()
    b.close()


def test_table_rejects_what_the_host_mirror_forbids(gpu):
    H, D, ps = 2, 32, 4
    pool = gpu.DevicePagePool(H, D, ps, 10)
    table = gpu.PageTable(pool, 3, 8)
    with pytest.raises(gpu.InvalidArgument):
        table.admit_synthetic(0, 9 * ps, 1)          # beyond max_pages
    table.admit_synthetic(0, 8 * ps, 1)
    with pytest.raises(gpu.InvalidArgument):
        table.admit_synthetic(0, ps, 2)              # slot not empty
    with pytest.raises(gpu.DsdError):
        table.admit_synthetic(1, 3 * ps, 2)          # 2 pages left
    with pytest.raises(gpu.OutOfRange):
        table.release([3])                           # no such slot
    with pytest.raises(gpu.InvalidArgument):
        table.append([1, 1], [1, 1], request_ids=[2, 2], decode_steps=[0, 1])
    table.release([0])
    assert table.free_pages() == 10
    assert sorted(table.free_stack().tolist()) == list(range(10))
    table.close()
    pool.close()


def test_staged_admission_equals_direct_admission(gpu):
    # Prompts uploaded ahead of admission into two staging buffers (reused
    # in turn) and admitted from them give the same pages, page contents and
    # summaries as dsd_table_admit_prompt on a second pool and table.
    H, D, ps = 4, 32, 8
    E = H * D
    cap = 200
    rng = np.random.default_rng(17)
    a = gpu.DevicePagePool(H, D, ps, cap)
    b = gpu.DevicePagePool(H, D, ps, cap)
    ta = gpu.PageTable(a, 6, 40)
    tb = gpu.PageTable(b, 6, 40)
    ta.staging_init(2, 40 * ps)
    prompts = [rng.standard_normal((t, E)).astype(np.float32) for t in (37, 0, 160, 9, 81, 8)]
    values = [rng.standard_normal(p.shape).astype(np.float32) for p in prompts]
    for slot, (k, v) in enumerate(zip(prompts, values)):
        ta.stage_prompt(slot % 2, k, v)
        ta.admit_staged(slot, slot % 2, len(k))
        tb.admit_prompt(slot, k, v)
        if slot == 2:
            ta.release([0])
            tb.release([0])
    for slot in range(1, 6):
        pa, pb = ta.pages(slot), tb.pages(slot)
        assert pa.tolist() == pb.tolist()
        for p in pa:
            ka, va = a.download_page(int(p))
            kb, vb = b.download_page(int(p))
            assert np.array_equal(ka.view(np.uint32), kb.view(np.uint32))
            assert np.array_equal(va.view(np.uint32), vb.view(np.uint32))
        if len(pa):
            assert np.array_equal(a.download_summaries(pa).view(np.uint32),
                                  b.download_summaries(pb).view(np.uint32))
    for t in (ta, tb):
        t.close()
    a.close()
    b.close()
