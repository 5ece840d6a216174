"""Non-finite page summaries (NaN, +-Inf), as a caller's corrupt K data would
make them.  The reference compares scores with > and == (its order is
undefined once a score is NaN: src/reference_kernels.cpp:82-107), so there
is no selection to match; what must hold is that the step stays well
defined: every selected id is one of the request's candidates, none twice,
min(k, n) of them, no device error, and a request of the same batch whose
pages are all finite gets exactly the oracle's selection and outputs.  40
candidates take the single-launch step, 600 the three-kernel step."""
from __future__ import annotations

import numpy as np
import pytest

import _oracle as orc

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n_cand", [40, 600])
def test_nonfinite_summaries_keep_the_selection_well_defined(gpu, n_cand):
    rng = np.random.default_rng(400 + n_cand)
    H, D, ps, k = 32, 128, 16, 8
    E = H * D
    cap = 2 * n_cand
    summ = (0.25 * rng.standard_normal((cap, E))).astype(np.float32)
    # request 0 holds pages [0, n_cand): some of them non-finite
    summ[3, 17] = np.nan
    summ[5, :] = np.inf
    summ[9, 100] = -np.inf
    summ[11, 5] = np.inf
    summ[11, 6] = -np.inf        # inf - inf: NaN in the sum
    keys = rng.standard_normal((cap, ps, E)).astype(np.float32)
    values = rng.standard_normal((cap, ps, E)).astype(np.float32)
    counts = np.full(cap, ps, np.int32)
    page_ids = np.arange(cap, dtype=np.int32)
    q = rng.standard_normal((2, E)).astype(np.float32)
    offs = np.array([0, n_cand, 2 * n_cand], np.int32)
    ids = np.concatenate([rng.permutation(n_cand),
                          n_cand + rng.permutation(n_cand)]).astype(np.int32)
    print(f"[nonfinite] n_cand={n_cand}", flush=True)
    with gpu.DevicePagePool(H, D, ps, cap) as pool:
        pool.upload_pages(page_ids, counts, page_ids.astype(np.int64) * ps * E, keys, values, summ)
        with gpu.SparseContext(pool, k, 2, 2 * n_cand, 2 * k) as ctx:
            got = ctx.run_batch(q, offs, ids, output_mode=gpu.OUTPUT_OUTPUTS, want_ids=True)
            ctx.device_status()
    sel0 = got["selected"][0].tolist()
    assert len(sel0) == k and len(set(sel0)) == k, sel0
    assert set(sel0) <= set(range(n_cand)), sel0
    # the finite request: exactly the oracle's
    _, want_sel, want_out = orc.sparse_batch(q[1:], keys, values, summ, counts,
                                             np.array([0, n_cand], np.int32), ids[n_cand:],
                                             H, D, ps, k)
    assert got["selected"][1].tolist() == want_sel[0].tolist()
    assert orc.max_abs_diff(got["outputs"][1:], want_out) <= 1e-4
