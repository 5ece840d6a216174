"""The C-ABI boundary (include/dsd_hip.h) on a machine without a GPU: the
library loads, exports every declared entry point, maps errors to the
reference's exception types, and does not contain the oracle."""
from __future__ import annotations

import pathlib
import re
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "dsd_hip.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dsd_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_symbols()
    for required in ("dsd_pool_create", "dsd_pool_upload_pages", "dsd_pool_upload_tokens",
                     "dsd_pool_mark_free", "dsd_pool_download_page", "dsd_sparse_create",
                     "dsd_sparse_run_batch", "dsd_sparse_run_batch_device",
                     "dsd_dense_run_batch", "dsd_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol(dsd):
    lib = dsd.load_library()
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, missing
    # the ctypes binding covers the whole header
    assert sorted(dsd.EXPORTED_SYMBOLS) == declared_symbols()


def test_exported_dynamic_symbols_are_the_c_abi(dsd):
    out = subprocess.run(["nm", "-D", "--defined-only", str(dsd.library_path())],
                         capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert set(declared_symbols()) <= exported
    # the product never carries the checker
    assert not any(s.startswith("oracle_") or s.startswith("ref_") for s in exported)


def test_product_does_not_link_the_oracle(dsd):
    out = subprocess.run(["ldd", str(dsd.library_path())], capture_output=True, text=True).stdout
    assert "oracle" not in out and "dsd_ref" not in out


def test_errors_without_gpu(dsd):
    if dsd.gpu_available():
        pytest.skip("a GPU is visible; the no-GPU error path does not apply")
    with pytest.raises(dsd.RuntimeFailure, match="gfx950"):
        dsd.DevicePagePool(2, 4, 4, 4)


def test_invalid_arguments_are_checked_before_the_device(dsd):
    with pytest.raises(dsd.InvalidArgument, match="capacity_pages"):
        dsd.DevicePagePool(2, 4, 4, -1)
    with pytest.raises(dsd.InvalidArgument):
        dsd.DevicePagePool(0, 4, 4, 4)


def test_host_free_takes_only_its_own_blocks(dsd):
    import ctypes
    lib = dsd.load_library()
    assert lib.dsd_host_free(None) == 0
    buf = ctypes.create_string_buffer(64)
    assert lib.dsd_host_free(ctypes.cast(buf, ctypes.c_void_p)) == 1  # invalid_argument
    assert b"dsd_host_alloc" in lib.dsd_last_error()
    out = ctypes.c_void_p()
    assert lib.dsd_host_alloc(0, ctypes.byref(out)) == 1
    assert lib.dsd_host_alloc(16, None) == 1


CPP_LIB = ROOT / "15-618_dynamic_sparse_decode_amd" / "build" / "libdsd.so"


def cpp_exports():
    if not CPP_LIB.exists():
        pytest.skip("libdsd.so not built")
    out = subprocess.run(["nm", "-DC", "--defined-only", str(CPP_LIB)],
                         capture_output=True, text=True, check=True).stdout
    return {line.split(" ", 2)[2] for line in out.splitlines() if " T " in line}


def test_cpp_library_exports_the_reference_api():
    names = cpp_exports()
    for sig in ("dsd::PagePool::allocate_page()", "dsd::PagedKvCache::AppendToken(",
                "dsd::DevicePagePool::UploadPage(", "dsd::SparseCudaContext::RunBatch(",
                "dsd::DenseCudaContext::RunBatch(", "dsd::SparseDecodeCuda(",
                "dsd::DenseAttentionCudaBatch(", "dsd::BuildSyntheticBatch(",
                "dsd::RunContinuousSparseDecode(", "dsd::MakeRequestState("):
        assert any(n.startswith(sig) for n in names), sig


def test_cpp_library_carries_no_cpu_compute_path():
    # the CPU rows live only in the checker (oracle/liboracle_cpu.so)
    names = cpp_exports()
    for cpu in ("dsd::ScorePagesCpu", "dsd::SelectTopKPagesCpu", "dsd::SparseAttentionCpu",
                "dsd::DenseAttentionCpu", "dsd::DecodePipeline::RunNaiveSparseStep(",
                "dsd::DecodePipeline::RunDenseStep("):
        assert not any(n.startswith(cpu) for n in names), cpu
    out = subprocess.run(["ldd", str(CPP_LIB)], capture_output=True, text=True).stdout
    assert "oracle" not in out and "libdsd_hip.so" in out
