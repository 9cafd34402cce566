"""CPU-only checks of libobjeta_hip.so: it loads, exports every function the header
declares, and its host-side rules and error reporting behave. No kernel runs here."""
import ctypes as C

import numpy as np
import pytest

from objeta_amd import _lib
from oracle import oracle as orc


def test_library_loads_and_exports_every_header_function():
    L = _lib.load()
    names = _lib.header_functions()
    assert len(names) > 30
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, f"declared but not exported: {missing}"
    # the ctypes signature table covers the whole header
    assert sorted(_lib.SIGNATURES) == names


def test_format_constants_match_reference():
    L = _lib.load()
    # QuantFormat::block_bytes / block_size (quant.rs:34-51)
    assert [L.objeta_hip_block_bytes(f) for f in range(4)] == [18, 22, 14, 17]
    assert [L.objeta_hip_block_size(f) for f in range(4)] == [32] * 4
    assert L.objeta_hip_block_bytes(7) == -1
    assert L.objeta_hip_quantized_matrix_bytes(0, 1024, 4096) == 2_359_296
    assert L.objeta_hip_quantized_matrix_bytes(0, 768, 2048) == 884_736
    assert L.objeta_hip_quantized_matrix_bytes(1, 4096, 4096) == 11_534_336
    assert L.objeta_hip_quantized_matrix_bytes(2, 14336, 4096) == 25_690_112
    assert L.objeta_hip_quantized_matrix_bytes(0, 4, 33) == -1
    assert L.objeta_hip_abi_version() == 1


def test_errors_are_reported_through_last_error():
    L = _lib.load()
    L.objeta_hip_clear_error()
    rec = _lib.Error()
    assert L.objeta_hip_last_error(C.byref(rec)) == 0 and rec.kind == -1
    # a NULL context is an InvalidInput error with an action and message
    rc = L.objeta_hip_stream_synchronize(None, None)
    assert rc == 5
    assert L.objeta_hip_last_error(C.byref(rec)) == 5
    assert rec.kind == 4 and b"context is NULL" in rec.source_message
    assert rec.file.endswith(b".cpp") and rec.line > 0


def test_fp4_scale_rule_matches_reference_on_every_float():
    """The integer E8M0 rule of the device FP4 quantizer equals the reference's
    ceil(log2f(amax / 6)) (glibc) for every non-negative float amax."""
    L = _lib.load()
    chunk = 1 << 24
    for start in range(0, 1 << 31, chunk):
        bits = np.arange(start, start + chunk, dtype=np.uint32)
        amax = bits.view(np.float32)
        got = np.empty(chunk, np.uint8)
        L.objeta_hip_fp4_scale_raw_host(amax.ctypes.data_as(C.c_void_p), got.ctypes.data_as(C.c_void_p), chunk)
        ref = _oracle_scale_raw(amax)
        bad = np.nonzero(got != ref)[0]
        assert bad.size == 0, f"mismatch at amax bits {bits[bad[:4]]}: {got[bad[:4]]} vs {ref[bad[:4]]}"


def _oracle_scale_raw(amax):
    L = orc.lib()
    out = np.empty(amax.size, np.uint8)
    L.orc_fp4_scale_raw_n(amax.ctypes.data_as(C.c_void_p), out.ctypes.data_as(C.c_void_p), amax.size)
    return out


def test_device_count_without_gpu_is_an_error_or_zero():
    L = _lib.load()
    n = C.c_int32(-1)
    rc = L.objeta_hip_device_count(C.byref(n))
    assert rc in (0, 2)
    if rc == 2:
        assert n.value == 0
