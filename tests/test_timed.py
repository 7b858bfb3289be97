"""Measurement adjuncts on the CPU: the C ABI's timer / timed / vendor-plan
entry points reject bad arguments before touching the GPU, and the Python
harnesses validate in the reference's order with its messages
(bindings/bindings_boo_timed.cu:139-190, bindings/bindings_pbr_timed.cu:
90-121, bindings/bindings_cusparse.cu:57-72).  Their GPU behaviour is in
test_gpu_timed.py."""

import ctypes
import os
from pathlib import Path

import numpy as np
import pytest
import scipy.sparse as sp
import torch

import spmm_amd as S

# SPMM_AMD_LIB: another build of the library (the host-sanitized one of
# `python spmm_amd/build.py san-test`)
LIB = (Path(os.environ['SPMM_AMD_LIB']) if os.environ.get('SPMM_AMD_LIB')
       else Path(__file__).resolve().parents[1] / 'spmm_amd' / 'libspmm_amd.so')


@pytest.fixture(scope='module')
def lib():
    L = ctypes.CDLL(str(LIB))
    L.spmm_last_error.restype = ctypes.c_char_p
    return L


def test_timer_and_timed_calls_reject_null_arguments(lib):
    assert lib.spmm_timer_create(None) == 1 and b'null' in lib.spmm_last_error()
    lib.spmm_timer_destroy(None)  # a null handle is accepted
    ms = ctypes.c_float(-1.0)
    rc = lib.spmm_boo_matmul_timed(None, 0, None, None, ctypes.c_int64(1), ctypes.c_int64(8), None,
                                   ctypes.c_size_t(0), None, None, ctypes.byref(ms))
    assert rc == 1 and b'null timer' in lib.spmm_last_error()
    rc = lib.spmm_pbr_matmul_timed(None, 0, None, None, ctypes.c_int64(1), ctypes.c_int64(8), None, None,
                                   ctypes.byref(ms))
    assert rc == 1 and b'null timer' in lib.spmm_last_error()


def test_vendor_plan_rejects_bad_arguments(lib):
    out = ctypes.c_void_p(1)
    i64 = ctypes.c_int64
    rc = lib.spmm_vendor_spmm_create(i64(4), i64(4), i64(4), None, None, None, None, i64(8), None, 0, None,
                                     ctypes.byref(out))
    assert rc == 1 and b'null CSR' in lib.spmm_last_error() and not out.value
    rc = lib.spmm_vendor_spmm_create(i64(-1), i64(4), i64(0), None, None, None, None, i64(8), None, 0, None,
                                     ctypes.byref(out))
    assert rc == 1 and b'negative' in lib.spmm_last_error()
    dummy = ctypes.c_int32(0)
    rc = lib.spmm_vendor_spmm_create(i64(0), i64(0), i64(0), ctypes.byref(dummy), None, None, None, i64(0),
                                     None, 7, None, ctypes.byref(out))
    assert rc == 1 and b'algorithm' in lib.spmm_last_error()
    assert lib.spmm_vendor_spmm_create(i64(0), i64(0), i64(0), None, None, None, None, i64(0), None, 0, None,
                                       None) == 1
    assert lib.spmm_vendor_spmm_run(None, None) == 1
    assert lib.spmm_vendor_spmm_preprocess(None, None, ctypes.c_size_t(0)) == 1
    assert lib.spmm_vendor_spmm_info(None, None) == 1
    lib.spmm_vendor_spmm_destroy(None)


def _boo_args(x, **kw):
    A = sp.identity(8, dtype=np.float32, format='csr')
    boo = S.csr_to_boo(A, cluster='identity', target_nr=4, target_nc=4)
    t = torch.zeros(1, dtype=torch.int32)
    v = torch.zeros(1, dtype=torch.float32)
    meta = [t] * 8 + [torch.zeros(1, dtype=torch.int16), v, t, t, v, t, t, v]
    return (boo.rows, boo.cols, boo.max_nr, boo.max_nc, boo.max_nnz_blk, *meta, x), kw


@pytest.mark.parametrize('kw, msg', [
    (dict(launch_mode='fast'), "launch_mode must be 'auto' or 'legacy'"),
    (dict(buckets=[0, 1, 2]), 'require auto rowseg and 5-element buckets'),
    (dict(launch_mode='auto', buckets=[0, 1, 2, 3]), 'require auto rowseg and 5-element buckets'),
    (dict(plan_row_ptr=torch.zeros(1, dtype=torch.int32)), 'must be provided together'),
    (dict(), 'X must be a CUDA FP32 tensor'),
])
def test_boo_timed_validation_order(kw, msg):
    args, kw = _boo_args(torch.zeros(8, 4), **kw)
    with pytest.raises(RuntimeError, match=msg):
        S.BOOTimedSpMM(*args, **kw)


def _pbr_args(x):
    t = torch.zeros(1, dtype=torch.int32)
    v = torch.zeros(1, dtype=torch.float32)
    return (8, 8, 8, 8, torch.zeros(1, dtype=torch.int64), t, t, v, t, t, v, x)


@pytest.mark.parametrize('kw, msg', [
    (dict(kernel='fast'), 'unsupported PBR kernel selector: fast'),
    (dict(kernel='nnzflat', diagnostic_raw_store=True), 'available only with kernel=block'),
    (dict(), 'PBRTimedSpMM: X must be a CUDA FP32 tensor'),
])
def test_pbr_timed_validation_order(kw, msg):
    with pytest.raises(RuntimeError, match=msg):
        S.PBRTimedSpMM(*_pbr_args(torch.zeros(8, 4)), **kw)


def test_direct_spmm_requires_cuda_x():
    crow = torch.zeros(9, dtype=torch.int32)
    col = torch.zeros(0, dtype=torch.int32)
    val = torch.zeros(0, dtype=torch.float32)
    with pytest.raises(RuntimeError, match='X must be contiguous CUDA FP32, two-dimensional'):
        S.DirectSpMM(crow, col, val, torch.zeros(8, 4), 'DEFAULT')
