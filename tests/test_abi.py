"""C-ABI checks that need no GPU: the library loads, exports every entry point
include/simp_rt.h declares, and rejects malformed descriptors before any
device work (the error behaviour the reference's loader has only for missing
symbols, runtime/include/kernel_runner.hpp:40-56)."""
import ctypes as C

import numpy as np
import pytest

import simplang_amd as sa
from simplang_amd import host


def test_every_declared_symbol_is_exported():
    names = host.declared_symbols()
    assert "simp_rt_tensor_matmul_i8" in names
    assert "kernel_main" in names and "benchmark_int8_matmul_256" in names
    missing = [n for n in names if not hasattr(sa.lib, n)]
    assert not missing, missing


def test_abi_version():
    assert sa.lib.simp_rt_version() == 1


def _d2(ptr, s0, s1, st0, off=0):
    return [ptr, ptr, off, s0, s1, st0, 1]


@pytest.mark.parametrize("fn", ["simp_rt_tensor_matmul_i8", "simp_rt_matmul_u8s8_i32",
                                "simp_rt_tensor_matmul_nt_i8", "simp_rt_matmul_nt_u8s8_i32"])
def test_gemm_rejects_bad_descriptors(fn):
    f = getattr(sa.lib, fn)
    a = np.zeros((4, 16), np.int8)
    b = np.zeros((16, 8), np.int8)
    c = np.zeros((4, 8), np.int32)
    pa, pb, pc = a.ctypes.data, b.ctypes.data, c.ctypes.data
    nt = "_nt_" in fn
    bd = _d2(pb, 8, 16, 16) if nt else _d2(pb, 16, 8, 8)
    # K mismatch
    rc = f(*_d2(pa, 4, 15, 16), *bd, *_d2(pc, 4, 8, 8))
    assert rc == -1 and b"shape mismatch" in sa.lib.simp_rt_last_error()
    # C shape mismatch
    rc = f(*_d2(pa, 4, 16, 16), *bd, *_d2(pc, 4, 7, 8))
    assert rc == -1
    # inner stride != 1
    bad = [pa, pa, 0, 4, 16, 16, 2]
    assert f(*bad, *bd, *_d2(pc, 4, 8, 8)) == -1
    assert b"inner stride" in sa.lib.simp_rt_last_error()
    # row stride shorter than the row
    assert f(*_d2(pa, 4, 16, 8), *bd, *_d2(pc, 4, 8, 8)) == -1
    # null data pointer with non-empty shape
    assert f(*_d2(None, 4, 16, 16), *bd, *_d2(pc, 4, 8, 8)) == -1
    assert b"null" in sa.lib.simp_rt_last_error()


def test_host_mirror_raises_on_error():
    a = np.zeros((4, 16), np.int8)
    b = np.zeros((15, 8), np.int8)
    c = np.zeros((4, 8), np.int32)
    with pytest.raises(sa.SimpRTError):
        sa.tensor_matmul_i8(a, b, c)


def test_dequant_w4_rejects_out_of_range():
    qw = np.zeros(16, np.int8)
    sc = np.zeros(1, np.float32)
    out = np.zeros(8, np.float32)
    with pytest.raises(sa.SimpRTError, match="too small"):
        sa.dequant_w4(qw, sc, sc, 30, 32, out, 8)       # element 37 is past 32 weights
    with pytest.raises(sa.SimpRTError, match="bad"):
        sa.dequant_w4(qw, sc, sc, -1, 32, out, 1)
