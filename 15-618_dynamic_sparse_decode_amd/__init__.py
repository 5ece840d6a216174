"""ctypes binding of libdsd_hip.so (the C ABI in include/dsd_hip.h).

Python-side plumbing for tests and bench.py: it forwards every call to the
HIP library and raises if the library is missing or the call fails -- there
is no Python or CPU implementation of the decode step here.  Exceptions
mirror the reference's C++ exception types (include/dsd/cuda_utils.h:43-53,
src/page_pool.cpp:104-120): InvalidArgument ~ std::invalid_argument,
OutOfRange ~ std::out_of_range, RuntimeFailure ~ std::runtime_error.

Also provides the synthetic-input helpers bench.py and the tests share
(reference draw order for context lengths, src/synthetic_data.cpp:29-41).
"""

from __future__ import annotations

import ctypes
import os
import pathlib

import numpy as np

PACKAGE_DIR = pathlib.Path(__file__).resolve().parent
BUILD_DIR = PACKAGE_DIR / "build"
LIB_PATH = BUILD_DIR / "libdsd_hip.so"

OUTPUT_NONE, OUTPUT_OUTPUTS, OUTPUT_DEBUG = 0, 1, 2
SCORE_CERTIFIED, SCORE_EXACT = 0, 1
TIMING_NONE, TIMING_EVENTS = 0, 1


class DsdError(Exception):
    """A non-zero status from libdsd_hip.so."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class InvalidArgument(DsdError, ValueError):
    pass


class OutOfRange(DsdError, IndexError):
    pass


class RuntimeFailure(DsdError, RuntimeError):
    pass


class HipFailure(RuntimeFailure):
    pass


_ERRORS = {1: InvalidArgument, 2: OutOfRange, 3: RuntimeFailure, 4: HipFailure}

_c_int_p = ctypes.POINTER(ctypes.c_int)
_c_float_p = ctypes.POINTER(ctypes.c_float)
_c_i64_p = ctypes.POINTER(ctypes.c_int64)
_c_u8_p = ctypes.POINTER(ctypes.c_uint8)
_c_double_p = ctypes.POINTER(ctypes.c_double)


class TransferStats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in (
        "h2d_bytes", "d2h_bytes", "h2d_calls", "d2h_calls",
        "h2d_large_calls", "d2h_large_calls")]

    def as_dict(self):
        return {n: int(getattr(self, n)) for n, _ in self._fields_}


class PoolArrays(ctypes.Structure):
    _fields_ = [("keys", ctypes.c_void_p), ("values", ctypes.c_void_p),
                ("summaries", ctypes.c_void_p), ("token_counts", ctypes.c_void_p),
                ("live", ctypes.c_void_p), ("k_offsets", ctypes.c_void_p),
                ("v_offsets", ctypes.c_void_p)]


class LaunchInfo(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in (
        "fused", "certified", "multi_pass", "heads_per_group", "grid",
        "score_pages_per_group", "wide")]

    def as_dict(self):
        return {n: int(getattr(self, n)) for n, _ in self._fields_}


class StepTimings(ctypes.Structure):
    _fields_ = [(n, ctypes.c_double) for n in (
        "score_ms", "topk_ms", "attention_ms", "kernel_ms",
        "h2d_ms", "d2h_ms", "launch_ms", "sync_ms")]

    def as_dict(self):
        return {n: float(getattr(self, n)) for n, _ in self._fields_}


class AsyncStep(ctypes.Structure):
    _fields_ = [("ticket", ctypes.c_longlong), ("batch", ctypes.c_int), ("fused", ctypes.c_int)] + [
        (n, ctypes.c_double) for n in (
            "start_ms", "done_ms", "score_ms", "topk_ms", "attention_ms", "kernel_ms")] + [
        ("wide", ctypes.c_int)]

    def as_dict(self):
        return {n: (float(getattr(self, n)) if t is ctypes.c_double else int(getattr(self, n)))
                for n, t in self._fields_}


# name -> (restype, argtypes)
_SIGNATURES = {
    "dsd_last_error": (ctypes.c_char_p, []),
    "dsd_gpu_available": (ctypes.c_int, []),
    "dsd_device_synchronize": (ctypes.c_int, []),
    "dsd_pool_create": (ctypes.c_int, [ctypes.c_int] * 4 + [ctypes.POINTER(ctypes.c_void_p)]),
    "dsd_pool_destroy": (ctypes.c_int, [ctypes.c_void_p]),
    "dsd_pool_reset": (ctypes.c_int, [ctypes.c_void_p]),
    "dsd_pool_upload_pages": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _c_int_p, _c_int_p,
                                             _c_i64_p, _c_float_p, _c_float_p, _c_float_p]),
    "dsd_pool_upload_tokens": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _c_int_p, _c_int_p,
                                              _c_int_p, _c_float_p, _c_float_p, _c_float_p]),
    "dsd_pool_mark_free": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _c_int_p]),
    "dsd_pool_download_page": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _c_float_p,
                                              _c_float_p, _c_int_p]),
    "dsd_pool_download_meta": (ctypes.c_int, [ctypes.c_void_p, _c_int_p, _c_u8_p]),
    "dsd_pool_download_summaries": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _c_int_p,
                                                   _c_float_p]),
    "dsd_pool_device_arrays": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(PoolArrays)]),
    "dsd_pool_prefill_synthetic": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _c_int_p,
                                                  _c_int_p, ctypes.c_int]),
    "dsd_pool_append_synthetic": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int] + [_c_int_p] * 5),
    "dsd_pool_transfer_stats": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(TransferStats)]),
    "dsd_pool_reset_transfer_stats": (ctypes.c_int, [ctypes.c_void_p]),
    "dsd_pool_capacity": (ctypes.c_int, [ctypes.c_void_p]),
    "dsd_sparse_create": (ctypes.c_int, [ctypes.c_void_p] + [ctypes.c_int] * 4
                          + [ctypes.POINTER(ctypes.c_void_p)]),
    "dsd_sparse_destroy": (ctypes.c_int, [ctypes.c_void_p]),
    "dsd_sparse_run_batch": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _c_float_p, _c_int_p,
                                            _c_int_p, ctypes.c_int, ctypes.c_int, _c_float_p,
                                            _c_float_p, _c_int_p, _c_int_p,
                                            ctypes.POINTER(StepTimings)]),
    "dsd_sparse_staging": (ctypes.c_int, [ctypes.c_void_p] + [ctypes.POINTER(ctypes.c_void_p)] * 4),
    "dsd_sparse_run_staged": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                             ctypes.c_int, _c_int_p, _c_int_p,
                                             ctypes.POINTER(StepTimings)]),
    "dsd_sparse_run_staged_rows": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int,
                                                  ctypes.POINTER(ctypes.c_void_p), ctypes.c_int,
                                                  ctypes.c_int, _c_int_p, _c_int_p,
                                                  ctypes.POINTER(StepTimings)]),
    "dsd_host_alloc": (ctypes.c_int, [ctypes.c_size_t, ctypes.POINTER(ctypes.c_void_p)]),
    "dsd_host_free": (ctypes.c_int, [ctypes.c_void_p]),
    "dsd_device_alloc": (ctypes.c_int, [ctypes.c_size_t, ctypes.POINTER(ctypes.c_void_p)]),
    "dsd_device_upload": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]),
    "dsd_device_free": (ctypes.c_int, [ctypes.c_void_p]),
    "dsd_synthetic_batch": (ctypes.c_int, [ctypes.c_int] * 9 + [_c_int_p, _c_float_p, _c_float_p,
                                                                _c_float_p]),
    "dsd_sparse_run_batch_device": (ctypes.c_int, [ctypes.c_void_p] + [ctypes.c_int] * 3
                                    + [ctypes.c_void_p] * 8),
    "dsd_sparse_run_batch_device_static": (ctypes.c_int, [ctypes.c_void_p] + [ctypes.c_int] * 4
                                           + [ctypes.c_void_p] * 9),
    "dsd_sparse_replay_stage": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]),
    "dsd_sparse_stream": (ctypes.c_void_p, [ctypes.c_void_p]),
    "dsd_sparse_set_score_mode": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
    "dsd_sparse_score_bounds": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _c_float_p,
                                               _c_float_p, _c_float_p]),
    "dsd_sparse_exact_rescored_pages": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _c_int_p]),
    "dsd_sparse_device_status": (ctypes.c_int, [ctypes.c_void_p]),
    "dsd_sparse_step_stamps": (ctypes.c_int, [ctypes.c_void_p, _c_int_p, _c_int_p, _c_double_p,
                                              ctypes.c_void_p, ctypes.c_size_t]),
    "dsd_sparse_last_launch": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(LaunchInfo)]),
    "dsd_sparse_set_wait_limit": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint, ctypes.c_int]),
    "dsd_table_create": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                        ctypes.POINTER(ctypes.c_void_p)]),
    "dsd_table_destroy": (ctypes.c_int, [ctypes.c_void_p]),
    "dsd_table_reset": (ctypes.c_int, [ctypes.c_void_p]),
    "dsd_table_slot_pages": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _c_int_p]),
    "dsd_table_free_pages": (ctypes.c_int, [ctypes.c_void_p, _c_int_p]),
    "dsd_table_download": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _c_int_p, ctypes.c_int,
                                          _c_int_p]),
    "dsd_table_free_stack": (ctypes.c_int, [ctypes.c_void_p, _c_int_p, ctypes.c_int, _c_int_p]),
    "dsd_table_admit_prompt": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                              _c_float_p, _c_float_p]),
    "dsd_table_admit_synthetic": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                                 ctypes.c_int]),
    "dsd_table_staging_init": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int]),
    "dsd_table_stage_prompt": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                              _c_float_p, _c_float_p]),
    "dsd_table_admit_staged": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                              ctypes.c_int]),
    "dsd_table_append": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _c_int_p, _c_u8_p,
                                        _c_u8_p, _c_float_p, _c_float_p, _c_int_p, _c_int_p]),
    "dsd_table_release": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _c_int_p, ctypes.c_int]),
    "dsd_sparse_run_table": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                            _c_int_p, _c_float_p, ctypes.POINTER(ctypes.c_void_p),
                                            ctypes.c_int, ctypes.c_int, _c_float_p, _c_int_p,
                                            _c_int_p, ctypes.POINTER(StepTimings)]),
    "dsd_sparse_last_csr": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _c_int_p, _c_int_p,
                                           ctypes.c_int]),
    "dsd_sparse_last_selection": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _c_int_p,
                                                 _c_int_p]),
    "dsd_sparse_run_table_async": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                                  _c_int_p, _c_float_p,
                                                  ctypes.POINTER(ctypes.c_void_p), ctypes.c_int,
                                                  ctypes.c_int, ctypes.POINTER(ctypes.c_longlong),
                                                  ctypes.POINTER(StepTimings)]),
    "dsd_sparse_async_wait": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_longlong]),
    "dsd_sparse_async_collect": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(AsyncStep),
                                                ctypes.c_int, _c_int_p]),
    "dsd_dense_run_batch": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _c_float_p, _c_int_p,
                                           _c_int_p, _c_float_p, _c_double_p]),
    "dsd_dense_run_batch_device": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int] + [ctypes.c_void_p] * 5),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

_LIB = None


def library_path() -> pathlib.Path:
    return pathlib.Path(os.environ.get("DSD_HIP_LIB", str(LIB_PATH)))


def load_library() -> ctypes.CDLL:
    """Load libdsd_hip.so; raises FileNotFoundError when it was not built."""
    global _LIB
    if _LIB is None:
        path = library_path()
        if not path.exists():
            raise FileNotFoundError(
                f"{path} is missing: build it with __graft_entry__.build() "
                f"(make -C 15-618_dynamic_sparse_decode_amd/csrc)")
        lib = ctypes.CDLL(str(path))
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _LIB = lib
    return _LIB


def _check(status: int) -> None:
    if status != 0:
        message = load_library().dsd_last_error().decode()
        raise _ERRORS.get(status, DsdError)(status, message)


def gpu_available() -> bool:
    return bool(load_library().dsd_gpu_available())


def synchronize() -> None:
    _check(load_library().dsd_device_synchronize())


def _ptr(array, ctype):
    if array is None:
        return None
    return array.ctypes.data_as(ctypes.POINTER(ctype))


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


class DevicePagePool:
    """HBM page pool (reference DevicePagePool, include/dsd/device_page_pool.h:17)."""

    def __init__(self, num_heads: int, head_dim: int, page_size: int, capacity_pages: int):
        self._lib = load_library()
        handle = ctypes.c_void_p()
        _check(self._lib.dsd_pool_create(num_heads, head_dim, page_size, capacity_pages,
                                         ctypes.byref(handle)))
        self.handle = handle
        self.num_heads, self.head_dim, self.page_size = num_heads, head_dim, page_size
        self.capacity = capacity_pages
        self.elements = num_heads * head_dim

    def close(self) -> None:
        if self.handle:
            _check(self._lib.dsd_pool_destroy(self.handle))
            self.handle = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self) -> None:
        _check(self._lib.dsd_pool_reset(self.handle))

    def upload_pages(self, page_ids, token_counts, src_offsets, keys, values, summaries=None):
        ids, counts = _i32(page_ids), _i32(token_counts)
        offs = np.ascontiguousarray(src_offsets, dtype=np.int64)
        k, v = _f32(keys), _f32(values)
        s = None if summaries is None else _f32(summaries)
        _check(self._lib.dsd_pool_upload_pages(
            self.handle, len(ids), _ptr(ids, ctypes.c_int), _ptr(counts, ctypes.c_int),
            _ptr(offs, ctypes.c_int64), _ptr(k, ctypes.c_float), _ptr(v, ctypes.c_float),
            _ptr(s, ctypes.c_float)))

    def upload_tokens(self, page_ids, token_offsets, page_token_counts, keys, values,
                      summaries=None):
        ids, offs, counts = _i32(page_ids), _i32(token_offsets), _i32(page_token_counts)
        k, v = _f32(keys), _f32(values)
        s = None if summaries is None else _f32(summaries)
        _check(self._lib.dsd_pool_upload_tokens(
            self.handle, len(ids), _ptr(ids, ctypes.c_int), _ptr(offs, ctypes.c_int),
            _ptr(counts, ctypes.c_int), _ptr(k, ctypes.c_float), _ptr(v, ctypes.c_float),
            _ptr(s, ctypes.c_float)))

    def mark_free(self, page_ids) -> None:
        ids = _i32(page_ids)
        _check(self._lib.dsd_pool_mark_free(self.handle, len(ids), _ptr(ids, ctypes.c_int)))

    def download_page(self, page_id: int):
        k = np.empty(self.page_size * self.elements, np.float32)
        v = np.empty_like(k)
        count = ctypes.c_int()
        _check(self._lib.dsd_pool_download_page(self.handle, int(page_id),
                                                _ptr(k, ctypes.c_float), _ptr(v, ctypes.c_float),
                                                ctypes.byref(count)))
        n = count.value * self.elements
        return k[:n].copy(), v[:n].copy()

    def download_meta(self):
        counts = np.empty(self.capacity, np.int32)
        live = np.empty(self.capacity, np.uint8)
        _check(self._lib.dsd_pool_download_meta(self.handle, _ptr(counts, ctypes.c_int),
                                                _ptr(live, ctypes.c_uint8)))
        return counts, live

    def download_summaries(self, page_ids):
        ids = _i32(page_ids)
        out = np.empty((len(ids), self.elements), np.float32)
        _check(self._lib.dsd_pool_download_summaries(self.handle, len(ids),
                                                     _ptr(ids, ctypes.c_int),
                                                     _ptr(out, ctypes.c_float)))
        return out

    def device_arrays(self) -> dict:
        arr = PoolArrays()
        _check(self._lib.dsd_pool_device_arrays(self.handle, ctypes.byref(arr)))
        return {n: int(getattr(arr, n) or 0) for n, _ in arr._fields_}

    def prefill_synthetic(self, page_ids, token_counts, request_id: int) -> None:
        ids, counts = _i32(page_ids), _i32(token_counts)
        _check(self._lib.dsd_pool_prefill_synthetic(self.handle, len(ids), _ptr(ids, ctypes.c_int),
                                                    _ptr(counts, ctypes.c_int), request_id))

    def append_synthetic(self, page_ids, token_offsets, page_token_counts, request_ids,
                         decode_steps) -> None:
        arrs = [_i32(a) for a in (page_ids, token_offsets, page_token_counts, request_ids,
                                  decode_steps)]
        _check(self._lib.dsd_pool_append_synthetic(self.handle, len(arrs[0]),
                                                   *[_ptr(a, ctypes.c_int) for a in arrs]))

    def transfer_stats(self) -> dict:
        st = TransferStats()
        _check(self._lib.dsd_pool_transfer_stats(self.handle, ctypes.byref(st)))
        return st.as_dict()

    def reset_transfer_stats(self) -> None:
        _check(self._lib.dsd_pool_reset_transfer_stats(self.handle))


class PageTable:
    """Request -> page table and free-page stack of a DevicePagePool in
    device memory (dsd_table_*): admission, append and release are kernels
    on the pool's stream, and SparseContext.run_table packs a step's
    candidate lists on the device from slot ids."""

    def __init__(self, pool, max_slots: int, max_pages: int):
        self._lib = load_library()
        self.pool = pool
        self.max_slots = max_slots
        self.max_pages = max_pages
        handle = ctypes.c_void_p()
        _check(self._lib.dsd_table_create(pool.handle, max_slots, max_pages, ctypes.byref(handle)))
        self.handle = handle

    def close(self) -> None:
        if self.handle:
            _check(self._lib.dsd_table_destroy(self.handle))
            self.handle = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self) -> None:
        _check(self._lib.dsd_table_reset(self.handle))

    def slot_pages(self, slot: int) -> int:
        out = ctypes.c_int()
        _check(self._lib.dsd_table_slot_pages(self.handle, slot, ctypes.byref(out)))
        return out.value

    def free_pages(self) -> int:
        out = ctypes.c_int()
        _check(self._lib.dsd_table_free_pages(self.handle, ctypes.byref(out)))
        return out.value

    def pages(self, slot: int) -> np.ndarray:
        buf = np.zeros(max(1, self.max_pages), np.int32)
        n = ctypes.c_int()
        _check(self._lib.dsd_table_download(self.handle, slot, _ptr(buf, ctypes.c_int),
                                            len(buf), ctypes.byref(n)))
        return buf[:n.value].copy()

    def free_stack(self) -> np.ndarray:
        buf = np.zeros(max(1, self.pool.capacity), np.int32)
        n = ctypes.c_int()
        _check(self._lib.dsd_table_free_stack(self.handle, _ptr(buf, ctypes.c_int), len(buf),
                                              ctypes.byref(n)))
        return buf[:n.value].copy()

    def admit_prompt(self, slot: int, keys, values) -> None:
        k = _f32(keys).reshape(-1)
        v = _f32(values).reshape(-1)
        tokens = k.size // self.pool.elements
        _check(self._lib.dsd_table_admit_prompt(self.handle, slot, tokens,
                                                _ptr(k, ctypes.c_float), _ptr(v, ctypes.c_float)))

    def staging_init(self, buffers: int, max_tokens: int) -> None:
        _check(self._lib.dsd_table_staging_init(self.handle, buffers, max_tokens))

    def stage_prompt(self, buffer: int, keys, values) -> None:
        k = _f32(keys).reshape(-1)
        v = _f32(values).reshape(-1)
        _check(self._lib.dsd_table_stage_prompt(self.handle, buffer, k.size // self.pool.elements,
                                                _ptr(k, ctypes.c_float), _ptr(v, ctypes.c_float)))

    def admit_staged(self, slot: int, buffer: int, tokens: int) -> None:
        _check(self._lib.dsd_table_admit_staged(self.handle, slot, buffer, tokens))

    def admit_synthetic(self, slot: int, tokens: int, request_id: int) -> None:
        _check(self._lib.dsd_table_admit_synthetic(self.handle, slot, tokens, request_id))

    def append(self, slots, upload, fresh_page=None, keys=None, values=None, request_ids=None,
               decode_steps=None) -> None:
        sl = _i32(slots)
        up = np.ascontiguousarray(upload, dtype=np.uint8)
        fr = np.ascontiguousarray(fresh_page, dtype=np.uint8) if fresh_page is not None else None
        k = _f32(keys).reshape(-1) if keys is not None else None
        v = _f32(values).reshape(-1) if values is not None else None
        rq = _i32(request_ids) if request_ids is not None else None
        st = _i32(decode_steps) if decode_steps is not None else None
        _check(self._lib.dsd_table_append(
            self.handle, len(sl), _ptr(sl, ctypes.c_int),
            _ptr(fr, ctypes.c_uint8) if fr is not None else None, _ptr(up, ctypes.c_uint8),
            _ptr(k, ctypes.c_float) if k is not None else None,
            _ptr(v, ctypes.c_float) if v is not None else None,
            _ptr(rq, ctypes.c_int) if rq is not None else None,
            _ptr(st, ctypes.c_int) if st is not None else None))

    def release(self, slots, clear: bool = True) -> None:
        sl = _i32(slots)
        _check(self._lib.dsd_table_release(self.handle, len(sl), _ptr(sl, ctypes.c_int),
                                           int(clear)))


class SparseContext:
    """One sparse decode step per call (reference SparseCudaContext,
    include/dsd/cuda_sparse_attention.h:50-137)."""

    def __init__(self, pool: DevicePagePool, top_k: int, max_batch: int,
                 max_total_candidates: int, max_total_selected: int):
        self._lib = load_library()
        self.pool = pool
        self.top_k = top_k
        self.max_batch = max_batch
        self.max_total_candidates = max_total_candidates
        handle = ctypes.c_void_p()
        _check(self._lib.dsd_sparse_create(pool.handle, top_k, max_batch, max_total_candidates,
                                           max_total_selected, ctypes.byref(handle)))
        self.handle = handle

    def close(self) -> None:
        if self.handle:
            _check(self._lib.dsd_sparse_destroy(self.handle))
            self.handle = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self) -> int:
        return self._lib.dsd_sparse_stream(self.handle) or 0

    def run_batch(self, queries, cand_offsets, cand_ids, output_mode=OUTPUT_DEBUG,
                  timing_mode=TIMING_EVENTS, want_ids=False):
        """Host-buffer step.  Returns a dict with outputs [B][E], in debug mode
        scores [P], and selected (a list of per-request id arrays) in debug
        mode or when want_ids is set with OUTPUT_OUTPUTS."""
        q = _f32(queries).reshape(-1)
        offs = _i32(cand_offsets)
        ids = _i32(cand_ids) if len(cand_ids) else np.zeros(1, np.int32)
        batch = len(offs) - 1
        total = int(offs[-1]) if batch > 0 else 0
        E = self.pool.elements
        out = np.zeros((max(batch, 0), E), np.float32)
        scores = np.zeros(max(total, 1), np.float32)
        sel = np.zeros(max(1, batch * max(1, self.top_k)), np.int32)
        counts = np.zeros(max(batch, 1), np.int32)
        t = StepTimings()
        debug = output_mode == OUTPUT_DEBUG
        ids_out = debug or (want_ids and output_mode == OUTPUT_OUTPUTS)
        _check(self._lib.dsd_sparse_run_batch(
            self.handle, batch, _ptr(q, ctypes.c_float), _ptr(offs, ctypes.c_int),
            _ptr(ids, ctypes.c_int), output_mode, timing_mode,
            _ptr(out, ctypes.c_float) if output_mode != OUTPUT_NONE else None,
            _ptr(scores, ctypes.c_float) if debug else None,
            _ptr(sel, ctypes.c_int) if ids_out else None,
            _ptr(counts, ctypes.c_int) if ids_out else None, ctypes.byref(t)))
        result = {"outputs": out, "timings": t.as_dict()}
        if debug:
            result["scores"] = scores[:total].copy()
        if ids_out:
            selected, w = [], 0
            for r in range(batch):
                c = int(counts[r])
                selected.append(sel[w:w + c].copy())
                w += c
            result["selected"] = selected
        return result

    def run_staged_rows(self, query_rows, cand_offsets, cand_ids, want_ids=False,
                        timing_mode=TIMING_NONE):
        """Host step whose queries are read in place: query_rows[r] is the
        address of request r's E floats inside a HostBlock (or the staging's
        own row r).  The candidate CSR is written into the context's staging
        first.  Returns outputs [B][E] (copied out of the staging) and, with
        want_ids, the selected ids."""
        offs = _i32(cand_offsets)
        ids = _i32(cand_ids)
        batch = len(offs) - 1
        total = int(offs[-1]) if batch > 0 else 0
        E = self.pool.elements
        # the staging holds max_batch + 1 offsets and max_total_candidates ids
        if batch > self.max_batch:
            raise InvalidArgument(1, "request batch exceeds sparse context capacity")
        if total > self.max_total_candidates or len(ids) < total:
            raise InvalidArgument(1, "candidate page count exceeds sparse context capacity")
        if len(query_rows) != batch:
            raise InvalidArgument(1, "one query row per request")
        q_st, off_st, ids_st, out_st = (ctypes.c_void_p() for _ in range(4))
        _check(self._lib.dsd_sparse_staging(self.handle, ctypes.byref(q_st), ctypes.byref(off_st),
                                            ctypes.byref(ids_st), ctypes.byref(out_st)))
        ctypes.memmove(off_st.value, offs.ctypes.data, 4 * (batch + 1))
        if total > 0:
            ctypes.memmove(ids_st.value, ids.ctypes.data, 4 * total)
        rows = (ctypes.c_void_p * max(batch, 1))(*[int(p) for p in query_rows])
        sel = np.zeros(max(1, batch * max(1, self.top_k)), np.int32)
        counts = np.zeros(max(batch, 1), np.int32)
        t = StepTimings()
        _check(self._lib.dsd_sparse_run_staged_rows(
            self.handle, batch, rows, OUTPUT_OUTPUTS, timing_mode,
            _ptr(sel, ctypes.c_int) if want_ids else None,
            _ptr(counts, ctypes.c_int) if want_ids else None, ctypes.byref(t)))
        out = np.zeros((batch, E), np.float32)
        if batch > 0:
            ctypes.memmove(out.ctypes.data, out_st.value, 4 * batch * E)
        result = {"outputs": out, "timings": t.as_dict(), "staging_queries": q_st.value}
        if want_ids:
            selected, w = [], 0
            for r in range(batch):
                c = int(counts[r])
                selected.append(sel[w:w + c].copy())
                w += c
            result["selected"] = selected
        return result

    def run_table(self, table, slots, queries=None, query_rows=None, output_mode=OUTPUT_OUTPUTS,
                  timing_mode=TIMING_NONE, want_ids=False):
        """Step over table slots: request r's candidates are the pages of
        slots[r] (the CSR is built on the device).  queries [B][E] or
        query_rows (addresses of pinned rows).  Returns outputs and, with
        want_ids, the selected ids."""
        sl = _i32(slots)
        batch = len(sl)
        E = self.pool.elements
        out = np.zeros((batch, E), np.float32)
        sel = np.zeros(max(1, batch * max(1, self.top_k)), np.int32)
        counts = np.zeros(max(batch, 1), np.int32)
        q = _f32(queries).reshape(-1) if queries is not None else None
        rows = None
        if query_rows is not None:
            rows = (ctypes.c_void_p * max(batch, 1))(*[int(p) for p in query_rows])
        t = StepTimings()
        _check(self._lib.dsd_sparse_run_table(
            self.handle, table.handle, batch, _ptr(sl, ctypes.c_int),
            _ptr(q, ctypes.c_float) if q is not None else None, rows, output_mode, timing_mode,
            _ptr(out, ctypes.c_float) if output_mode != OUTPUT_NONE else None,
            _ptr(sel, ctypes.c_int) if want_ids else None,
            _ptr(counts, ctypes.c_int) if want_ids else None, ctypes.byref(t)))
        result = {"outputs": out, "timings": t.as_dict()}
        if want_ids:
            selected, w = [], 0
            for r in range(batch):
                c = int(counts[r])
                selected.append(sel[w:w + c].copy())
                w += c
            result["selected"] = selected
        return result

    def run_table_async(self, table, slots, queries=None, query_rows=None,
                        output_mode=OUTPUT_OUTPUTS, timing_mode=TIMING_NONE):
        """run_table enqueued without a wait: returns the step's ticket (0
        for an empty batch).  queries are copied at the call; query_rows
        (addresses in HostBlock memory) are read when the step runs and
        must stay unchanged until async_wait(ticket) returns."""
        sl = _i32(slots)
        batch = len(sl)
        q = _f32(queries).reshape(-1) if queries is not None else None
        rows = None
        if query_rows is not None:
            rows = (ctypes.c_void_p * max(batch, 1))(*[int(p) for p in query_rows])
        ticket = ctypes.c_longlong(0)
        t = StepTimings()
        _check(self._lib.dsd_sparse_run_table_async(
            self.handle, table.handle, batch, _ptr(sl, ctypes.c_int),
            _ptr(q, ctypes.c_float) if q is not None else None, rows, output_mode, timing_mode,
            ctypes.byref(ticket), ctypes.byref(t)))
        return int(ticket.value)

    def async_wait(self, ticket: int) -> None:
        """Blocks until every asynchronous step up to `ticket` has completed
        (raising the failure one of them reported)."""
        _check(self._lib.dsd_sparse_async_wait(self.handle, int(ticket)))

    def async_collect(self):
        """Waits for every enqueued asynchronous step; returns their records
        (dicts, oldest first)."""
        out = []
        buf = (AsyncStep * 64)()
        n = ctypes.c_int(0)
        while True:
            _check(self._lib.dsd_sparse_async_collect(self.handle, buf, 64, ctypes.byref(n)))
            if n.value == 0:
                return out
            out.extend(buf[i].as_dict() for i in range(n.value))

    def last_selection(self, batch):
        """The selected ids of the last step on the context's stream, one
        array per request (synchronous)."""
        kk = max(1, self.top_k)
        sel = np.zeros(max(1, batch * kk), np.int32)
        counts = np.zeros(max(1, batch), np.int32)
        _check(self._lib.dsd_sparse_last_selection(self.handle, batch, _ptr(sel, ctypes.c_int),
                                                   _ptr(counts, ctypes.c_int)))
        result, w = [], 0
        for r in range(batch):
            c = int(counts[r])
            result.append(sel[w:w + c].copy())
            w += c
        return result

    def staged_outputs(self, batch):
        """The staging's outputs [batch][E] (where table steps leave them)."""
        out_st = ctypes.c_void_p()
        _check(self._lib.dsd_sparse_staging(self.handle, None, None, None, ctypes.byref(out_st)))
        E = self.pool.elements
        buf = (ctypes.c_float * (batch * E)).from_address(out_st.value)
        return np.ctypeslib.as_array(buf).reshape(batch, E).copy()

    def last_csr(self, batch):
        """(cand_offsets, cand_ids) of the last step as its kernels read them."""
        offs = np.zeros(batch + 1, np.int32)
        cap = max(1, self.max_total_candidates)
        ids = np.zeros(cap, np.int32)
        _check(self._lib.dsd_sparse_last_csr(self.handle, batch, _ptr(offs, ctypes.c_int),
                                             _ptr(ids, ctypes.c_int), cap))
        return offs, ids[:int(offs[-1])].copy()

    def run_batch_device(self, batch, total_candidates, max_candidates, d_queries,
                         d_cand_offsets, d_cand_ids, d_outputs, d_scores=0, d_selected=0,
                         d_counts=0, stream=0) -> None:
        """Device-resident step: integer device addresses, async on `stream`."""
        _check(self._lib.dsd_sparse_run_batch_device(
            self.handle, batch, total_candidates, max_candidates, d_queries, d_cand_offsets,
            d_cand_ids, d_outputs, d_scores or None, d_selected or None, d_counts or None,
            stream or None))

    def set_score_mode(self, mode: int) -> None:
        _check(self._lib.dsd_sparse_set_score_mode(self.handle, mode))

    def score_bounds(self, n: int):
        """(mid, lo, hi) certified intervals of the last step's first n candidates."""
        mid, lo, hi = (np.empty(n, np.float32) for _ in range(3))
        _check(self._lib.dsd_sparse_score_bounds(self.handle, n, _ptr(mid, ctypes.c_float),
                                                 _ptr(lo, ctypes.c_float),
                                                 _ptr(hi, ctypes.c_float)))
        return mid, lo, hi

    def exact_rescored_pages(self, reset: bool = False) -> int:
        out = ctypes.c_int()
        _check(self._lib.dsd_sparse_exact_rescored_pages(self.handle, int(reset),
                                                         ctypes.byref(out)))
        return out.value

    def last_launch(self) -> dict:
        """Launch form of the last step: fused, certified, multi_pass,
        heads_per_group, grid, score_pages_per_group."""
        info = LaunchInfo()
        _check(self._lib.dsd_sparse_last_launch(self.handle, ctypes.byref(info)))
        return info.as_dict()

    def step_stamps(self):
        """(stamps [grid][per_group] uint64, khz) of the last timed fused step."""
        grid, per, khz = ctypes.c_int(), ctypes.c_int(), ctypes.c_double()
        _check(self._lib.dsd_sparse_step_stamps(self.handle, ctypes.byref(grid), ctypes.byref(per),
                                                ctypes.byref(khz), None, 0))
        out = np.zeros((grid.value, per.value), np.uint64)
        if out.size:
            _check(self._lib.dsd_sparse_step_stamps(self.handle, ctypes.byref(grid),
                                                    ctypes.byref(per), ctypes.byref(khz),
                                                    out.ctypes.data_as(ctypes.c_void_p), out.size))
        return out, khz.value

    def device_status(self) -> None:
        """Synchronize; raise the last unreported input failure of a step."""
        _check(self._lib.dsd_sparse_device_status(self.handle))

    def set_wait_limit(self, spin_limit: int, never_ready: bool = False) -> None:
        _check(self._lib.dsd_sparse_set_wait_limit(self.handle, int(spin_limit),
                                                   int(bool(never_ready))))

    def replay_stage(self, stage: int, stream=0) -> None:
        _check(self._lib.dsd_sparse_replay_stage(self.handle, stage, stream or None))


class HostBlock:
    """Pinned host memory from dsd_host_alloc, viewed as a float32 array;
    rows inside it may be passed to SparseContext.run_staged_rows."""

    def __init__(self, count: int):
        self._lib = load_library()
        p = ctypes.c_void_p()
        _check(self._lib.dsd_host_alloc(4 * count, ctypes.byref(p)))
        self.address = p.value
        self.array = np.ctypeslib.as_array((ctypes.c_float * count).from_address(p.value))

    def close(self) -> None:
        if self.address:
            self.array = None
            _check(self._lib.dsd_host_free(ctypes.c_void_p(self.address)))
            self.address = 0

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class DeviceBlock:
    """Device memory from dsd_device_alloc (float32 elements); rows inside
    it may be passed as query rows, as HostBlock rows may."""

    def __init__(self, count: int):
        self._lib = load_library()
        p = ctypes.c_void_p()
        _check(self._lib.dsd_device_alloc(4 * count, ctypes.byref(p)))
        self.address = p.value
        self.count = count

    def upload(self, values, offset: int = 0) -> None:
        """Copies float32 values into elements [offset, offset + len)."""
        v = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
        _check(self._lib.dsd_device_upload(ctypes.c_void_p(self.address + 4 * offset),
                                           v.ctypes.data_as(ctypes.c_void_p), 4 * v.size))

    def close(self) -> None:
        if self.address:
            _check(self._lib.dsd_device_free(ctypes.c_void_p(self.address)))
            self.address = 0

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def sparse_run_batch_device_static(pool: DevicePagePool, top_k, batch, total_candidates,
                                   max_candidates, d_queries, d_cand_offsets, d_cand_ids,
                                   d_outputs, d_scores=0, d_selected=0, d_counts=0, d_fail=0,
                                   stream=0) -> None:
    """The allocation-free device step (no context; the library's static
    scratch): integer device addresses, async on `stream`."""
    _check(load_library().dsd_sparse_run_batch_device_static(
        pool.handle, top_k, batch, total_candidates, max_candidates, d_queries, d_cand_offsets,
        d_cand_ids, d_outputs, d_scores or None, d_selected or None, d_counts or None,
        d_fail or None, stream or None))


def dense_run_batch(pool: DevicePagePool, queries, cand_offsets, cand_ids):
    """Dense attention over every candidate page (reference DenseCudaContext)."""
    lib = load_library()
    q = _f32(queries).reshape(-1)
    offs = _i32(cand_offsets)
    ids = _i32(cand_ids) if len(cand_ids) else np.zeros(1, np.int32)
    batch = len(offs) - 1
    out = np.zeros((batch, pool.elements), np.float32)
    ms = ctypes.c_double()
    _check(lib.dsd_dense_run_batch(pool.handle, batch, _ptr(q, ctypes.c_float),
                                   _ptr(offs, ctypes.c_int), _ptr(ids, ctypes.c_int),
                                   _ptr(out, ctypes.c_float), ctypes.byref(ms)))
    return out, ms.value


def dense_run_batch_device(pool: DevicePagePool, batch, d_queries, d_cand_offsets, d_cand_ids,
                           d_outputs, stream=0) -> None:
    _check(load_library().dsd_dense_run_batch_device(pool.handle, batch, d_queries,
                                                     d_cand_offsets, d_cand_ids, d_outputs,
                                                     stream or None))


# ---------------------------------------------------------------------------
# Synthetic inputs
# ---------------------------------------------------------------------------
def reference_context_lengths(batch: int, lo: int, hi: int, seed: int):
    """The B context lengths in the reference's draw order: std::mt19937(seed)
    then std::uniform_int_distribution<int>(lo, hi) (src/synthetic_data.cpp:29-41).
    libstdc++ (GCC 11+) maps a 32-bit engine output to [lo, hi] with Lemire's
    multiply-and-reject method (Lemire 2019, "Fast Random Integer Generation in
    an Interval"); numpy's MT19937 with legacy seeding is the same engine."""
    bg = np.random.MT19937()
    bg._legacy_seeding(seed)
    span = hi - lo + 1
    out = []
    for _ in range(batch):
        prod = int(bg.random_raw()) * span
        low = prod & 0xFFFFFFFF
        if low < span:
            threshold = ((1 << 32) - span) % span
            while low < threshold:
                prod = int(bg.random_raw()) * span
                low = prod & 0xFFFFFFFF
        out.append(lo + (prod >> 32))
    return out


class SyntheticBatch:
    """A ragged batch laid out like the reference's BuildSyntheticBatch
    (src/synthetic_data.cpp:23-68): capacity = total pages, LIFO page ids
    (the first page allocated is capacity-1, src/page_pool.cpp:36-45), each
    request's candidates in logical page order.

    Values are i.i.d. N(0,1) float32 from numpy's PCG64.  Each request has
    its own stream, child r of numpy.random.SeedSequence(seed) spawned into
    B + 1 children: its pages' keys ([n_r][page_size][E]), then their values.
    Child B gives the queries ([B][E]).  Streams are independent, so requests
    are generated in parallel (host threads) or one at a time
    (request_pages), and anyone with numpy regenerates the same batch."""

    def __init__(self, num_heads, head_dim, page_size, context_lengths, seed,
                 capacity=None, dtype=np.float32):
        self.num_heads, self.head_dim, self.page_size = num_heads, head_dim, page_size
        self.elements = E = num_heads * head_dim
        self.dtype = dtype
        self.context_lengths = [int(c) for c in context_lengths]
        self.pages_per = [(c + page_size - 1) // page_size for c in self.context_lengths]
        total_pages = sum(self.pages_per)
        self.capacity = capacity if capacity is not None else total_pages
        B = len(self.context_lengths)
        self.cand_offsets = np.zeros(B + 1, np.int32)
        self.cand_offsets[1:] = np.cumsum(self.pages_per)
        ids = np.arange(total_pages, dtype=np.int32)
        self.cand_ids = (self.capacity - 1 - ids).astype(np.int32)
        self.token_counts = np.zeros(self.capacity, np.int32)
        g = 0
        for r, c in enumerate(self.context_lengths):
            for j in range(self.pages_per[r]):
                self.token_counts[self.cand_ids[g]] = min(page_size, c - j * page_size)
                g += 1
        self._streams = np.random.SeedSequence(seed).spawn(B + 1)
        self.queries = np.random.default_rng(self._streams[B]).standard_normal(
            (B, E), dtype=dtype)
        self._key_pool = None
        self._value_pool = None
        self.generator = "per-request PCG64 streams"

    @classmethod
    def reference(cls, num_heads, head_dim, page_size, batch, min_context, max_context, seed,
                  distribution="normal", capacity=None):
        """The batch in the reference's draw order (BuildSyntheticBatch,
        src/synthetic_data.cpp:23-68): one std::mt19937(seed), the context
        lengths, then per request its pages' keys, values, then its query
        (dsd_synthetic_batch).  distribution "uniform" is the reference's
        own U(-1, 1), value for value; "normal" draws
        std::normal_distribution<float>(0, 1) on the same engine in the
        same order.  One engine, so it is generated sequentially."""
        lib = load_library()
        lengths = np.zeros(max(batch, 1), np.int32)
        dist = {"uniform": 0, "normal": 1}[distribution]
        args = [num_heads, head_dim, page_size, batch, min_context, max_context, seed, dist]
        _check(lib.dsd_synthetic_batch(*args, 0, _ptr(lengths, ctypes.c_int), None, None, None))
        self = cls(num_heads, head_dim, page_size, lengths[:batch].tolist(), seed,
                   capacity=capacity)
        E = self.elements
        kp = np.empty((self.capacity, page_size, E), np.float32)
        vp = np.empty_like(kp)
        q = np.empty((batch, E), np.float32)
        _check(lib.dsd_synthetic_batch(*args, self.capacity, _ptr(lengths, ctypes.c_int),
                                       _ptr(kp, ctypes.c_float), _ptr(vp, ctypes.c_float),
                                       _ptr(q, ctypes.c_float)))
        live = np.zeros(self.capacity, bool)
        live[self.cand_ids] = True
        kp[~live] = 0.0
        vp[~live] = 0.0
        self._key_pool, self._value_pool, self.queries = kp, vp, q
        self.generator = f"reference draw order, {distribution}"
        return self

    @property
    def batch(self):
        return len(self.context_lengths)

    @property
    def total_candidates(self):
        return int(self.cand_offsets[-1])

    @property
    def max_candidates(self):
        return int(np.max(np.diff(self.cand_offsets))) if self.batch else 0

    def request_ids(self, r: int):
        """Page ids of request r, in logical order."""
        return self.cand_ids[self.cand_offsets[r]:self.cand_offsets[r + 1]]

    def request_pages(self, r: int, out_keys=None, out_values=None):
        """Keys and values of request r's pages, [n_r][page_size][E] each
        (written into out_keys / out_values when given)."""
        if self._streams is None or self.generator.startswith("reference"):
            raise ValueError("request_pages needs the per-request streams")
        n = self.pages_per[r]
        shape = (n, self.page_size, self.elements)
        k = np.empty(shape, self.dtype) if out_keys is None else out_keys
        v = np.empty(shape, self.dtype) if out_values is None else out_values
        rng = np.random.default_rng(self._streams[r])
        rng.standard_normal(out=k.reshape(-1), dtype=self.dtype)
        rng.standard_normal(out=v.reshape(-1), dtype=self.dtype)
        return k, v

    def _materialize(self):
        import concurrent.futures as cf
        shape = (self.capacity, self.page_size, self.elements)
        kp = np.zeros(shape, self.dtype)
        vp = np.zeros(shape, self.dtype)

        def fill(r):
            n = self.pages_per[r]
            if n == 0:
                return
            # a request's ids are consecutive and descending: rows lo..hi
            hi = int(self.cand_ids[self.cand_offsets[r]])
            lo = hi - n + 1
            k, v = self.request_pages(r)
            kp[lo:hi + 1] = k[::-1]
            vp[lo:hi + 1] = v[::-1]

        with cf.ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1)) as ex:
            list(ex.map(fill, range(self.batch)))
        self._key_pool, self._value_pool = kp, vp

    @property
    def key_pool(self):
        """[capacity][page_size][E] keys (built on first use)."""
        if self._key_pool is None:
            self._materialize()
        return self._key_pool

    @property
    def value_pool(self):
        if self._value_pool is None:
            self._materialize()
        return self._value_pool

    def live_page_ids(self):
        return self.cand_ids.copy()

    def upload(self, pool: DevicePagePool, summaries=None):
        """Upload every live page; the device computes summaries unless given."""
        ids = self.live_page_ids()
        counts = self.token_counts[ids]
        offs = ids.astype(np.int64) * self.page_size * self.elements
        pool.upload_pages(ids, counts, offs, self.key_pool.reshape(-1),
                          self.value_pool.reshape(-1), summaries)

    def upload_request(self, pool: DevicePagePool, r: int, keys, values):
        """Upload request r's pages from request_pages(r)'s arrays (device
        summaries)."""
        ids = self.request_ids(r)
        n = len(ids)
        if n == 0:
            return
        offs = np.arange(n, dtype=np.int64) * self.page_size * self.elements
        pool.upload_pages(ids, self.token_counts[ids], offs, keys.reshape(-1),
                          values.reshape(-1))
