"""ctypes access to the CPU oracle (oracle/liboracle.so) -- the checker.

Test infrastructure: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use it.  Each wrapper names the oracle function it calls;
the oracle functions cite the reference lines they restate.
"""
from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent.parent
ORACLE_DIR = ROOT / "oracle"
ORACLE_LIB = ORACLE_DIR / "liboracle.so"
REF_LIB = ORACLE_DIR / "_ref" / "libdsd_ref.so"

_lib = None


def build_oracle() -> None:
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR), "oracle"], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not ORACLE_LIB.exists():
            build_oracle()
        _lib = ctypes.CDLL(str(ORACLE_LIB))
        _lib.oracle_scale.restype = ctypes.c_float
        _lib.oracle_dot.restype = ctypes.c_float
        _lib.oracle_max_abs_diff.restype = ctypes.c_float
        _lib.oracle_select_topk.restype = ctypes.c_int
        _lib.oracle_sparse_step.restype = ctypes.c_int
    return _lib


def P(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


def scale(head_dim: int) -> float:
    return lib().oracle_scale(head_dim)


def page_summary(keys, token_count: int, elements: int):
    """oracle_page_summary: host rule of src/paged_kv_cache.cpp:87-99."""
    k = f32(keys)
    out = np.empty(elements, np.float32)
    lib().oracle_page_summary(P(k), int(token_count), int(elements), P(out))
    return out


def pool_summaries(key_pool, token_counts, elements: int, page_ids=None):
    """Summaries of the listed pages ([cap][E] when page_ids is None)."""
    kp = f32(key_pool).reshape(len(token_counts), -1)
    ids = range(len(token_counts)) if page_ids is None else page_ids
    out = np.zeros((len(token_counts) if page_ids is None else len(page_ids), elements),
                   np.float32)
    for row, p in enumerate(ids):
        out[row] = page_summary(kp[p], int(token_counts[p]), elements)
    return out


def append_summary(summary, key, old_count: int):
    s = f32(summary).copy()
    k = f32(key)
    lib().oracle_append_summary(P(s), P(k), int(old_count), len(s))
    return s


def score_pages(query, summaries, token_counts, page_ids, head_dim: int):
    q, s, tc, ids = f32(query), f32(summaries), i32(token_counts), i32(page_ids)
    out = np.empty(len(ids), np.float32)
    lib().oracle_score_pages(P(q), P(s), P(tc), P(ids), len(ids), len(q),
                             ctypes.c_float(scale(head_dim)), P(out))
    return out


def select_topk(scores, page_ids, top_k: int):
    s, ids = f32(scores), i32(page_ids)
    out = np.empty(max(1, min(top_k, len(ids))), np.int32)
    n = lib().oracle_select_topk(P(s), P(ids), len(ids), int(top_k), P(out))
    return out[:n].copy()


def attention(query, key_pool, value_pool, token_counts, page_ids, num_heads, head_dim,
              page_size):
    q, kp, vp = f32(query), f32(key_pool), f32(value_pool)
    tc, ids = i32(token_counts), i32(page_ids)
    out = np.empty(num_heads * head_dim, np.float32)
    lib().oracle_attention(P(q), P(kp), P(vp), P(tc), P(ids), len(ids), num_heads,
                           head_dim, page_size, P(out))
    return out


def sparse_batch(queries, key_pool, value_pool, summaries, token_counts, cand_offsets,
                 cand_ids, num_heads, head_dim, page_size, top_k, stage_ms=None):
    """oracle_sparse_batch: sparse_cpu over a CSR batch.  Returns (scores,
    selected list, outputs [B][E])."""
    q, kp, vp, sm = f32(queries), f32(key_pool), f32(value_pool), f32(summaries)
    tc, offs, ids = i32(token_counts), i32(cand_offsets), i32(cand_ids)
    B = len(offs) - 1
    E = num_heads * head_dim
    total = int(offs[-1])
    scores = np.zeros(max(total, 1), np.float32)
    kk = max(top_k, 1)
    sel = np.full(B * kk, -1, np.int32)
    counts = np.zeros(max(B, 1), np.int32)
    outs = np.zeros((B, E), np.float32)
    ms = np.zeros(4, np.float64) if stage_ms is not None else None
    lib().oracle_sparse_batch(P(q), P(kp), P(vp), P(sm), P(tc), P(offs),
                              P(ids if total else np.zeros(1, np.int32)), B, num_heads,
                              head_dim, page_size, int(top_k), P(scores), P(sel), P(counts),
                              P(outs), P(ms))
    if stage_ms is not None:
        stage_ms += ms
    selected = [sel[r * kk: r * kk + counts[r]].copy() for r in range(B)]
    return scores[:total].copy(), selected, outs


def request_step(query, keys, values, counts, page_ids, num_heads, head_dim, page_size, top_k,
                 dense=False):
    """sparse_cpu for one request whose pages are given in logical order:
    keys / values [n][page_size][E], counts [n] and page_ids [n] (distinct).
    Composes the oracle's own rows as oracle_sparse_step does: summaries
    (oracle_page_summary), scores (oracle_score_pages), top-k by (score desc,
    page id asc) over the real ids (oracle_select_topk), then gather +
    attention over the selected pages in selected order (oracle_attention).
    Returns (selected ids, sparse output [E], dense output [E] or None) --
    dense is oracle_attention over every page in logical order (dense_cpu).
    Lets a test stream a large batch one request at a time."""
    E = num_heads * head_dim
    ids = i32(page_ids)
    n = len(ids)
    cnt = i32(counts)
    pos = np.arange(n, dtype=np.int32)
    summ = pool_summaries(keys, cnt, E)
    scores = score_pages(query, summ, cnt, pos, head_dim)
    selected = select_topk(scores, ids, top_k) if n else np.zeros(0, np.int32)
    where = {int(p): j for j, p in enumerate(ids)}
    sel_pos = np.array([where[int(p)] for p in selected], np.int32)
    out = attention(query, keys, values, cnt, sel_pos, num_heads, head_dim, page_size)
    dense_out = None
    if dense:
        dense_out = attention(query, keys, values, cnt, pos, num_heads, head_dim, page_size)
    return selected, out, dense_out


def dense_batch(queries, key_pool, value_pool, token_counts, cand_offsets, cand_ids,
                num_heads, head_dim, page_size):
    offs = i32(cand_offsets)
    E = num_heads * head_dim
    q = f32(queries).reshape(-1, E)
    out = np.zeros((len(offs) - 1, E), np.float32)
    for r in range(len(offs) - 1):
        out[r] = attention(q[r], key_pool, value_pool, token_counts,
                           cand_ids[offs[r]:offs[r + 1]], num_heads, head_dim, page_size)
    return out


def max_abs_diff(a, b) -> float:
    a, b = f32(a).reshape(-1), f32(b).reshape(-1)
    return float(lib().oracle_max_abs_diff(P(a), len(a), P(b), len(b)))
