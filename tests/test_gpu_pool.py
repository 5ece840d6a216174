"""Device page pool behaviour through the C ABI, following the reference's
tests/test_device_page_pool.cpp (fixture :32-63: request 17 with pages of
4, 4 and 2 tokens in a 6-page pool, ids 5, 4, 3 by LIFO allocation), plus
bit-exact device summaries for appended tokens (running mean,
src/paged_kv_cache.cpp:231-238)."""
from __future__ import annotations

import numpy as np
import pytest

import _oracle as orc

pytestmark = pytest.mark.gpu

H, D, PS = 2, 4, 4
E = H * D


def seq(count, start):
    return (start + np.arange(count)).astype(np.float32)


class Fixture:
    """RequestFixture of test_device_page_pool.cpp:32-63 with its LIFO ids."""

    def __init__(self, capacity=6):
        self.capacity = capacity
        self.token_counts = [PS, PS, 2]
        self.page_ids = [capacity - 1 - i for i in range(3)]
        self.keys = [seq(c * E, 100.0 * (i + 1)) for i, c in enumerate(self.token_counts)]
        self.values = [seq(c * E, 1000.0 * (i + 1)) for i, c in enumerate(self.token_counts)]
        # host cache pools [cap][ps][E]
        self.key_pool = np.zeros((capacity, PS, E), np.float32)
        self.value_pool = np.zeros_like(self.key_pool)
        for i, p in enumerate(self.page_ids):
            c = self.token_counts[i]
            self.key_pool[p, :c] = self.keys[i].reshape(c, E)
            self.value_pool[p, :c] = self.values[i].reshape(c, E)

    def upload(self, pool, order=None):
        order = range(3) if order is None else order
        for i in order:
            p = self.page_ids[i]
            pool.upload_pages([p], [self.token_counts[i]], [p * PS * E], self.key_pool,
                              self.value_pool)


def test_logical_and_reverse_upload_round_trip(gpu):
    for order in (None, [2, 1, 0]):
        fx = Fixture()
        pool = gpu.DevicePagePool(H, D, PS, fx.capacity)
        fx.upload(pool, order)
        for i, p in enumerate(fx.page_ids):
            k, v = pool.download_page(p)
            assert k.tolist() == fx.keys[i].tolist()
            assert v.tolist() == fx.values[i].tolist()


def test_batched_upload_from_cache_merges_runs(gpu):
    fx = Fixture()
    pool = gpu.DevicePagePool(H, D, PS, fx.capacity)
    ids = np.array(sorted(fx.page_ids), np.int32)
    counts = np.array([fx.token_counts[fx.page_ids.index(p)] for p in ids], np.int32)
    pool.upload_pages(ids, counts, ids.astype(np.int64) * PS * E, fx.key_pool, fx.value_pool)
    for i, p in enumerate(fx.page_ids):
        k, v = pool.download_page(p)
        assert k.tolist() == fx.keys[i].tolist() and v.tolist() == fx.values[i].tolist()
    st = pool.transfer_stats()
    assert st["h2d_calls"] > 0 and st["h2d_bytes"] >= 2 * 10 * E * 4


def test_metadata_and_reset(gpu):
    fx = Fixture()
    pool = gpu.DevicePagePool(H, D, PS, fx.capacity)
    fx.upload(pool)
    counts, live = pool.download_meta()
    for p in range(fx.capacity):
        if p in fx.page_ids:
            assert counts[p] == fx.token_counts[fx.page_ids.index(p)] and live[p] == 1
        else:
            assert counts[p] == 0 and live[p] == 0
    pool.reset()
    counts, live = pool.download_meta()
    assert not counts.any() and not live.any()
    fx.upload(pool)
    for i, p in enumerate(fx.page_ids):
        k, _ = pool.download_page(p)
        assert k.tolist() == fx.keys[i].tolist()


def test_invalid_usage_raises_reference_exception_types(gpu):
    pool = gpu.DevicePagePool(H, D, PS, 4)
    page = seq(PS * E, 1.0)
    with pytest.raises(gpu.OutOfRange):
        pool.upload_pages([-1], [PS], [0], page, page)
    with pytest.raises(gpu.InvalidArgument):
        pool.upload_pages([0], [0], [0], page, page)
    with pytest.raises(gpu.InvalidArgument):
        pool.upload_pages([0], [PS + 1], [0], page, page)
    with pytest.raises(gpu.RuntimeFailure, match="free device page"):
        pool.download_page(0)
    with pytest.raises(gpu.OutOfRange):
        pool.download_page(4)
    with pytest.raises(gpu.OutOfRange):
        pool.mark_free([7])


def test_incremental_token_upload_and_free(gpu):
    # test_device_page_pool.cpp:232-303 (ps 3, 4-page pool, first page id 3).
    pool = gpu.DevicePagePool(H, D, 3, 4)
    t0k, t0v = seq(E, 10.0), seq(E, 100.0)
    pool.upload_tokens([3], [0], [1], t0k, t0v)
    k, v = pool.download_page(3)
    assert k.tolist() == t0k.tolist() and v.tolist() == t0v.tolist()
    t1k, t1v = seq(E, 20.0), seq(E, 200.0)
    pool.upload_tokens([3], [1], [2], t1k, t1v)
    k, v = pool.download_page(3)
    assert k.tolist() == np.concatenate([t0k, t1k]).tolist()
    assert v.tolist() == np.concatenate([t0v, t1v]).tolist()
    counts, live = pool.download_meta()
    assert counts[3] == 2 and live[3] == 1
    pool.mark_free([3])
    counts, live = pool.download_meta()
    assert counts[3] == 0 and live[3] == 0
    with pytest.raises(gpu.RuntimeFailure):
        pool.download_page(3)
    assert not pool.download_summaries([3]).any()


def test_batched_token_upload_and_reuse(gpu):
    # test_device_page_pool.cpp:305-348
    pool = gpu.DevicePagePool(H, D, 3, 4)
    k0, v0, k1, v1 = seq(E, 11.0), seq(E, 111.0), seq(E, 22.0), seq(E, 222.0)
    pool.upload_tokens([3, 3], [0, 1], [2, 2], np.concatenate([k0, k1]),
                       np.concatenate([v0, v1]))
    k, v = pool.download_page(3)
    assert k.tolist() == np.concatenate([k0, k1]).tolist()
    assert v.tolist() == np.concatenate([v0, v1]).tolist()
    pool.mark_free([3])
    rk, rv = seq(E, 33.0), seq(E, 333.0)
    pool.upload_tokens([3], [0], [1], rk, rv)
    k, v = pool.download_page(3)
    assert k.tolist() == rk.tolist() and v.tolist() == rv.tolist()
    with pytest.raises(gpu.OutOfRange):
        pool.upload_tokens([3], [1], [1], rk, rv)


def test_direct_prompt_upload(gpu):
    # test_device_page_pool.cpp:350-391: ReservePagesForRequest(41, {4,4,2}) in
    # an 8-page pool allocates 7, 6, 5 and sorts them: ids [5, 6, 7].
    pool = gpu.DevicePagePool(H, D, PS, 8)
    counts = np.array([4, 4, 2], np.int32)
    ids = np.array([5, 6, 7], np.int32)
    keys, values = seq(10 * E, 7.0), seq(10 * E, 70.0)
    starts = np.concatenate([[0], np.cumsum(counts)[:-1]]).astype(np.int64) * E
    pool.upload_pages(ids, counts, starts, keys, values)
    tok = 0
    for i, p in enumerate(ids):
        k, v = pool.download_page(p)
        n = counts[i] * E
        assert k.tolist() == keys[tok * E:tok * E + n].tolist()
        assert v.tolist() == values[tok * E:tok * E + n].tolist()
        tok += counts[i]
    # device summaries use the host rule on the uploaded prompt
    dev = pool.download_summaries(ids)
    tok = 0
    for i in range(3):
        ref = orc.page_summary(keys[tok * E:(tok + counts[i]) * E], counts[i], E)
        assert np.array_equal(dev[i].view(np.uint32), ref.view(np.uint32))
        tok += counts[i]


def test_device_running_mean_matches_host_cache_bit_exact(gpu):
    """Tokens appended one by one, in pairs and after a prompt upload: the
    device summary equals PagedKvCache's running mean after every call."""
    rng = np.random.default_rng(4)
    h, d, ps = 32, 128, 16
    e = h * d
    pool = gpu.DevicePagePool(h, d, ps, 3)
    keys = rng.standard_normal((3, ps, e)).astype(np.float32)
    vals = rng.standard_normal((3, ps, e)).astype(np.float32)
    # page 0: 16 single appends; page 1: pairs; page 2: 5-token prompt + appends
    host = [np.zeros(e, np.float32) for _ in range(3)]
    for t in range(ps):
        pool.upload_tokens([0], [t], [t + 1], keys[0, t], vals[0, t])
        host[0] = orc.append_summary(host[0], keys[0, t], t)
        dev = pool.download_summaries([0])[0]
        assert np.array_equal(dev.view(np.uint32), host[0].view(np.uint32)), t
    for t in range(0, ps, 2):
        pool.upload_tokens([1, 1], [t + 1, t], [t + 2, t + 2], keys[1, [t + 1, t]],
                           vals[1, [t + 1, t]])
        host[1] = orc.append_summary(host[1], keys[1, t], t)
        host[1] = orc.append_summary(host[1], keys[1, t + 1], t + 1)
        assert np.array_equal(pool.download_summaries([1])[0].view(np.uint32),
                              host[1].view(np.uint32))
    pool.upload_pages([2], [5], [0], keys[2].reshape(-1), vals[2].reshape(-1))
    host[2] = orc.page_summary(keys[2, :5], 5, e)
    for t in range(5, ps):
        pool.upload_tokens([2], [t], [t + 1], keys[2, t], vals[2, t])
        host[2] = orc.append_summary(host[2], keys[2, t], t)
    assert np.array_equal(pool.download_summaries([2])[0].view(np.uint32),
                          host[2].view(np.uint32))
    k, v = pool.download_page(2)
    assert np.array_equal(k, keys[2].reshape(-1)) and np.array_equal(v, vals[2].reshape(-1))
    # a gap in the prefix cannot be summarised on the device
    with pytest.raises(gpu.InvalidArgument, match="prefix"):
        pool.mark_free([0])
        pool.upload_tokens([0], [3], [4], keys[0, 3], vals[0, 3])


def test_summary_rows_copied_verbatim_when_given(gpu):
    pool = gpu.DevicePagePool(H, D, PS, 2)
    page = seq(PS * E, 1.0)
    rows = np.full((1, E), 0.5, np.float32)
    pool.upload_pages([1], [PS], [0], page, page, rows)
    assert pool.download_summaries([1])[0].tolist() == [0.5] * E
    pool.upload_tokens([0], [0], [1], seq(E, 3.0), seq(E, 4.0), np.full((1, E), -2.0, np.float32))
    assert pool.download_summaries([0])[0].tolist() == [-2.0] * E


@pytest.mark.parametrize("pinned", [False, True])
def test_large_uploads_round_trip(gpu, pinned):
    # Copies of 4 MB and more from pageable memory go through the pool's
    # pinned staging ring (16 MB chunks, 1 MB host-thread tasks); from pinned
    # memory they go straight to the DMA engine.  Either way every byte must
    # land: a 200-page run (50 MB, a partial last chunk), a 77-page run
    # (19.25 MB) and a lone partial page.
    import torch
    h, d, ps = 32, 128, 16
    e = h * d
    pool = gpu.DevicePagePool(h, d, ps, 300)
    page_ids = list(range(10, 210)) + list(range(220, 297)) + [299]
    counts = [ps] * 277 + [7]
    src_offsets = [i * ps * e for i in range(len(page_ids))]
    total = len(page_ids) * ps * e
    rng = np.random.default_rng(5)
    keys = rng.standard_normal(total, dtype=np.float32)
    values = rng.standard_normal(total, dtype=np.float32)
    if pinned:
        tk = torch.empty(total, dtype=torch.float32, pin_memory=True)
        tv = torch.empty(total, dtype=torch.float32, pin_memory=True)
        tk.numpy()[:] = keys
        tv.numpy()[:] = values
        src_k, src_v = tk.numpy(), tv.numpy()
    else:
        src_k, src_v = keys, values
    pool.upload_pages(page_ids, counts, src_offsets, src_k, src_v)
    for i in sorted(set(range(0, len(page_ids), 13)) | {63, 64, 199, 200, 276, 277}):
        k, v = pool.download_page(page_ids[i])
        n = counts[i] * e
        assert k.size == n and v.size == n, (pinned, i)
        np.testing.assert_array_equal(k, keys[src_offsets[i]:src_offsets[i] + n])
        np.testing.assert_array_equal(v, values[src_offsets[i]:src_offsets[i] + n])
    st = pool.transfer_stats()
    assert st["h2d_bytes"] >= 2 * 4 * e * sum(counts)  # keys and values, valid tokens


@pytest.mark.parametrize("heads,head_dim", [(2, 64), (4, 96)])
def test_synthetic_append_summaries_follow_the_running_mean(gpu, heads, head_dim):
    """dsd_pool_append_synthetic (reference AppendTokensSynthetic,
    src/device_page_pool.cpp:904-983, kernel :190-237).  The generated K/V
    values themselves have no reference vectors (the reference's generator
    is device-only), so what is checked is everything around them:
      * every value lies on the reference's grid k/1000, k in [-1000, 1000],
        and rows differ between key and value streams, decode steps and
        requests, and are a function of (request, step) only;
      * each summary equals the oracle's running mean (oracle_append_summary,
        the host rule of src/paged_kv_cache.cpp:231-238) applied to the K rows
        the kernel wrote -- in offset order for several tokens of one page in
        one call, and with the reference's counts (old = the page's token
        count - 1) for a page's single token of a call, also when that token
        is not the page's last;
      * page counts, live flags and the reference's transfer accounting (five
        copies of n ints per call)."""
    ps = 4
    E = heads * head_dim
    pool = gpu.DevicePagePool(heads, head_dim, ps, 8)
    pool.reset_transfer_stats()
    calls = [
        # page, offset, page count after the call, request, decode step
        [(3, 2, 3, 11, 2), (5, 0, 1, 12, 0), (3, 0, 3, 11, 0), (3, 1, 3, 11, 1)],
        [(5, 1, 2, 12, 1), (3, 3, 4, 11, 3)],
        # one token rewriting offset 0 of a 2-token page: old count = 1
        [(5, 0, 2, 12, 5)],
        # the same (request, step) as page 3's offset 0, into another page
        [(6, 0, 1, 11, 0)],
    ]
    summ = {p: np.zeros(E, np.float32) for p in (3, 5, 6)}
    rows = {}
    for toks in calls:
        cols = list(zip(*toks))
        pool.append_synthetic(*[np.array(c, np.int32) for c in cols])
        counts, _ = pool.download_meta()
        pages = sorted({t[0] for t in toks})
        written = {p: pool.download_page(p) for p in pages}
        for p in pages:
            seg = sorted((t for t in toks if t[0] == p), key=lambda t: t[1])
            k_all = written[p][0].reshape(-1, E)
            v_all = written[p][1].reshape(-1, E)
            for page, off, cnt, req, step in seg:
                k, v = k_all[off].copy(), v_all[off].copy()
                rows.setdefault((req, step), (k, v))
                old = cnt - 1 if len(seg) == 1 else off
                summ[p] = orc.append_summary(summ[p], k, old)
    st = pool.transfer_stats()
    assert st["h2d_calls"] == 5 * len(calls)
    assert st["h2d_bytes"] == 5 * 4 * sum(len(c) for c in calls)
    counts, live = pool.download_meta()
    assert counts[[3, 5, 6]].tolist() == [4, 2, 1] and live[[3, 5, 6]].tolist() == [1, 1, 1]
    assert counts[[0, 1, 2, 4, 7]].tolist() == [0] * 5
    got = pool.download_summaries([3, 5, 6])
    for i, p in enumerate((3, 5, 6)):
        assert np.array_equal(got[i].view(np.uint32), summ[p].view(np.uint32)), p
    # the grid, and what enters the generator
    allv = np.concatenate([np.concatenate(kv) for kv in rows.values()])
    grid = np.rint(allv.astype(np.float64) * 1000.0)
    assert np.array_equal(allv, (grid / 1000.0).astype(np.float32))
    assert grid.min() >= -1000 and grid.max() <= 1000
    k0, v0 = rows[(11, 0)]
    assert not np.array_equal(k0, v0)                        # stream enters
    assert not np.array_equal(k0, rows[(11, 1)][0])          # decode step enters
    assert not np.array_equal(rows[(12, 0)][0], k0)          # request enters
    assert len(np.unique(k0)) > E // 2                       # element enters
    k6, v6 = pool.download_page(6)
    assert np.array_equal(k6, k0) and np.array_equal(v6, v0)  # page does not