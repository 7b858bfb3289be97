"""The C ABI library loads and exports every function include/spmm_amd.h
declares; its host-only entry points work without a GPU."""

import ctypes
import os
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / 'include' / 'spmm_amd.h'
# SPMM_AMD_LIB: another build of the library (the host-sanitized one of
# `python spmm_amd/build.py san-test`)
LIB = Path(os.environ['SPMM_AMD_LIB']) if os.environ.get('SPMM_AMD_LIB') else ROOT / 'spmm_amd' / 'libspmm_amd.so'


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(spmm_\w+)\s*\(', text,
                                 flags=re.M)))


@pytest.fixture(scope='module')
def lib():
    import torch  # noqa: F401  (one HIP runtime per process, torch's)
    assert LIB.exists(), 'libspmm_amd.so not built'
    return ctypes.CDLL(str(LIB))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for n in ('spmm_boo_matmul', 'spmm_pbr_matmul', 'spmm_csr_naive', 'spmm_boo_stage_create',
              'spmm_boo_stage_sizes', 'spmm_boo_stage_copy', 'spmm_boo_stage_destroy',
              'spmm_boo_workspace_bytes', 'spmm_last_error', 'spmm_version'):
        assert n in names


def test_every_declared_symbol_is_exported(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_version_and_error_path_without_gpu(lib):
    lib.spmm_version.restype = ctypes.c_char_p
    lib.spmm_last_error.restype = ctypes.c_char_p
    assert b'gfx950' in lib.spmm_version()
    # argument checks run before any HIP call
    rc = lib.spmm_boo_matmul(None, 0, None, None, ctypes.c_int64(1), ctypes.c_int64(8), None,
                             ctypes.c_size_t(0), None)
    assert rc == 1 and b'null' in lib.spmm_last_error()
    rc = lib.spmm_pbr_matmul(None, 0, None, None, ctypes.c_int64(1), ctypes.c_int64(8), None)
    assert rc == 1
    n = ctypes.c_int32(-1)
    for fn in (lib.spmm_boo_launch_info, lib.spmm_pbr_launch_info):
        rc = fn(None, 0, None, None, ctypes.c_int64(1), ctypes.c_int64(8), None, 0, ctypes.byref(n))
        assert rc == 1 and b'null' in lib.spmm_last_error()
        rc = fn(None, 0, None, None, ctypes.c_int64(1), ctypes.c_int64(8), None, 4, ctypes.byref(n))
        assert rc == 1 and b'launch info' in lib.spmm_last_error()


def test_stage_create_rejects_bad_arguments_without_gpu(lib):
    lib.spmm_last_error.restype = ctypes.c_char_p
    out = ctypes.c_void_p(0)
    rc = lib.spmm_boo_stage_create(None, 4096, 256, 8, 4, ctypes.c_float(1.5), ctypes.byref(out))
    assert rc == 1 and b'null' in lib.spmm_last_error() and not out.value
    rc = lib.spmm_boo_stage_sizes(None, None)
    assert rc == 1
    lib.spmm_boo_stage_destroy(None)              # a null handle is accepted


def test_pbr_slab_knob_without_gpu(lib):
    lib.spmm_last_error.restype = ctypes.c_char_p
    lib.spmm_pbr_get_slab_bytes.restype = ctypes.c_int64
    assert lib.spmm_pbr_set_slab_bytes(ctypes.c_int64(-1)) == 1 and b'negative' in lib.spmm_last_error()
    assert lib.spmm_pbr_set_slab_bytes(ctypes.c_int64(123 << 20)) == 0
    assert lib.spmm_pbr_get_slab_bytes() == 123 << 20
    assert lib.spmm_pbr_set_slab_bytes(ctypes.c_int64(0)) == 0 and lib.spmm_pbr_get_slab_bytes() == 0
