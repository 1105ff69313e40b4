"""The C ABI library loads and exports every symbol include/vq2_amd.h
declares; argument validation returns error codes (no GPU work is issued:
every call here is rejected on the host before any HIP call)."""
import ctypes
import subprocess

import pytest
import torch

from compressai_amd import _lib


def test_header_and_binding_agree():
    declared = _lib.header_symbols()
    assert len(declared) >= 12
    assert sorted(declared) == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    L = _lib.load()
    for name in _lib.header_symbols():
        assert hasattr(L, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    for name in _lib.header_symbols():
        assert name in exported, name
    assert L.vq2_version() >= 100


def _err(code):
    assert code != _lib.OK
    return _lib.load().vq2_last_error().decode()


def test_gemv_rejects_bad_arguments_on_host():
    L = _lib.load()
    # n not a multiple of 8
    msg = _err(L.vq2_gemv(1, 0, 1, 12, 1, None, 0, 16, None, 1, 1, 1, 1, 0, 4, 4, 12, 1.0, None))
    assert "multiple of 8" in msg
    # NULL activation
    msg = _err(L.vq2_gemv(None, 0, 1, 16, 1, None, 0, 16, None, 1, 1, 1, 1, 0, 4, 4, 16, 1.0, None))
    assert "NULL" in msg
    # misaligned codebook
    msg = _err(L.vq2_gemv(8, 0, 1, 16, 8, None, 0, 24, None, 1, 8, 1, 8, 0, 4, 4, 16, 1.0, None))
    assert "aligned" in msg
    # idx1 given for a 2 bpw matrix
    msg = _err(L.vq2_gemv(16, 0, 1, 16, 16, 16, 0, 32, None, 1, 16, 1, 16, 0, 4, 4, 16, 1.0, None))
    assert "idx1" in msg
    # bad dtype code
    msg = _err(L.vq2_gemv(16, 7, 1, 16, 16, None, 0, 32, None, 1, 16, 1, 16, 0, 4, 4, 16, 1.0, None))
    assert "dtype" in msg
    # empty problems are a no-op
    assert L.vq2_gemv(None, 0, 0, 16, None, None, 0, None, None, 1, None, 1, None, 0, 4, 4, 16, 1.0, None) == 0


def test_moe_and_rht_reject_bad_arguments_on_host():
    L = _lib.load()
    msg = _err(L.vq2_moe_grouped(16, 0, 0, 1, 16, 5, 8, 16, 4, 32, 1, 16, 1, 16, 0, 1024, 1024, 256, 1.0, None))
    assert "ids dtype" in msg
    msg = _err(L.vq2_moe_grouped(16, 0, 0, 0, 16, 0, 8, 16, 4, 32, 1, 16, 1, 16, 0, 1024, 1024, 256, 1.0, None))
    assert "pairs_per_x" in msg
    msg = _err(L.vq2_rht(16, 0, 12, 32, 0, 12, None, None, 12, 3, 1, 1.0, 0, None))
    assert "power of two" in msg
    msg = _err(L.vq2_rht(16, 0, 2048, 32, 0, 2048, None, None, 2048, 16384, 1, 1.0, 0, None))
    assert "power of two" in msg
    msg = _err(L.vq2_rht(16, 0, 6144, 16, 0, 6144, None, None, 6144, 4096, 1, 1.0, 0, None))
    assert "overlap" in msg
    msg = _err(L.vq2_router_topk(16, 0, 1, 256, 40, None, 0, 0, None, 0, -1, 16, 16, None))
    assert "k=40" in msg
    msg = _err(L.vq2_argmax_rows(16, 0, 1, 0, 16, None, None))
    assert "bad sizes" in msg


def test_sorted_batch_rejects_bad_arguments_on_host():
    """vq2_sorted_gemm_batch / _argmax: batch outside 1..4, a short or
    unaligned activation row, LDS beyond 150 KiB and a bad chunk height are
    refused before any HIP call (the pointers are never dereferenced)."""
    L = _lib.load()

    def mat(rows=512, ng=256, R=205, ipc=10):
        chunks = -(-rows // R)
        return _lib.SortedMat(4096, ipc, ipc, ipc * chunks, R, 0, 4096, 4096, rows)

    m = mat()
    args = lambda batch, stride, mm, n: (4096, 0, batch, stride, 1, ctypes.byref(mm), 4096, None, 1, 1, 0, n, 1.0,
                                         1, None, 0, None)
    assert "batch=5" in _err(L.vq2_sorted_gemm_batch(*args(5, 2048, m, 2048)))
    assert "batch=0" in _err(L.vq2_sorted_gemm_batch(*args(0, 2048, m, 2048)))
    assert "row stride" in _err(L.vq2_sorted_gemm_batch(*args(2, 2040, m, 2048)))
    assert "row stride" in _err(L.vq2_sorted_gemm_batch(*args(2, 2052, m, 2048)))
    # n = 65536 (ng 8192, chunks of at most 15 rows): 2 fp16 rows are 256 KiB of LDS (at
    # batch 3-4 the call runs as 2-row launches, which do not fit either)
    big = mat(rows=64, ng=8192, R=15)
    assert "LDS" in _err(L.vq2_sorted_gemm_batch(*args(4, 65536, big, 65536)))
    assert "LDS" in _err(L.vq2_sorted_gemm_batch(*args(2, 65536, big, 65536)))
    # rows_per_chunk beyond 511 (what 17-bit positions hold for ng = 256)
    assert "rows_per_chunk" in _err(L.vq2_sorted_gemm_batch(*args(2, 2048, mat(R=600), 2048)))
    msg = _err(L.vq2_sorted_gemm_batch_argmax(4096, 0, 3, 2048, ctypes.byref(m), 4096, None, 1, 1, 2048, 1.0,
                                              4096, 1 << 20, None, None, None))
    assert "out_idx" in msg
    assert L.vq2_sorted_gemm_batch_workspace(ctypes.byref(m), 1, 2, 1) == 0


def test_python_entry_points_refuse_cpu_tensors():
    from compressai_amd import kernels as K

    x = torch.zeros(16)
    with pytest.raises(K.Vq2Error, match="GPU tensors"):
        K.vq_rht(x, hb=16)
    with pytest.raises(RuntimeError):
        K.vq_gemv_16(x, torch.zeros(2, 2, dtype=torch.int16), torch.zeros(65536, 8), torch.ones(2), 2, 16)


def test_error_message_is_thread_local():
    import threading

    L = _lib.load()
    L.vq2_rht(16, 0, 12, 32, 0, 12, None, None, 12, 3, 1, 1.0, 0, None)
    seen = {}

    def other():
        seen["msg"] = L.vq2_last_error().decode()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == ""
    assert "power of two" in L.vq2_last_error().decode()


def test_moe_wait_knob_and_status_refuse_bad_arguments_on_host():
    L = _lib.load()
    assert "max_polls" in _err(L.vq2_sorted_moe_set_wait(-1, 0))
    assert "extra_arrivals" in _err(L.vq2_sorted_moe_set_wait(10, 5000))
    assert L.vq2_sorted_moe_set_wait(1 << 20, 0) == _lib.OK     # the production values
    assert "NULL workspace" in _err(L.vq2_sorted_moe_status(None, 0, None))
