"""The C ABI library loads and exports every function include/spmm_amd.h
declares; its host-only entry points work without a GPU."""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / 'include' / 'spmm_amd.h'
LIB = ROOT / 'spmm_amd' / 'libspmm_amd.so'


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
    for n in ('spmm_boo_matmul', 'spmm_pbr_matmul', 'spmm_csr_naive', 'spmm_boo_plan_build',
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


def _plan(lib, row_grp_ptr, blk_row_grp, blk_nz_ptr, rem_indptr, max_item_nnz, long_thr):
    i32 = ctypes.POINTER(ctypes.c_int32)
    a = [np.ascontiguousarray(v, dtype=np.int32) for v in (row_grp_ptr, blk_row_grp, blk_nz_ptr, rem_indptr)]
    rows = len(rem_indptr) - 1
    n_rg = len(row_grp_ptr) - 1
    nb = len(blk_row_grp)
    cnt = [ctypes.c_int32(0) for _ in range(4)]
    args = [ctypes.c_int32(rows), ctypes.c_int32(n_rg), ctypes.c_int32(nb)] + \
        [x.ctypes.data_as(i32) for x in a] + [ctypes.c_int32(max_item_nnz), ctypes.c_int32(long_thr)]
    rc = lib.spmm_boo_plan_build(*args, None, None, ctypes.c_int32(0), None,
                                 *[ctypes.byref(c) for c in cnt])
    assert rc == 0
    n_items = cnt[0].value
    items = np.zeros(4 * n_items, np.int32)
    splits = np.zeros(3 * n_items, np.int32)
    longr = np.zeros(rows, np.int32)
    rc = lib.spmm_boo_plan_build(*args, items.ctypes.data_as(i32), splits.ctypes.data_as(i32),
                                 ctypes.c_int32(n_items), longr.ctypes.data_as(i32),
                                 *[ctypes.byref(c) for c in cnt])
    assert rc == 0
    return items.reshape(-1, 4), splits[:3 * cnt[2].value].reshape(-1, 3), cnt[1].value, \
        longr[:cnt[3].value]


def test_plan_build_splits_heavy_groups_and_finds_long_rows(lib):
    # 3 row groups; group 1 holds 4 blocks of 10 nonzeros; group 2 has none.
    row_grp_ptr = [0, 2, 4, 6]
    blk_row_grp = [0, 1, 1, 1, 1]
    blk_nz_ptr = [0, 5, 15, 25, 35, 45]
    rem_indptr = [0, 0, 3, 3, 10, 10, 11]          # row 3 has 7 remainder entries
    items, splits, n_slots, longr = _plan(lib, row_grp_ptr, blk_row_grp, blk_nz_ptr, rem_indptr,
                                          max_item_nnz=20, long_thr=5)
    assert items.tolist() == [[0, 0, 1, -1], [1, 1, 3, -1], [1, 3, 5, 0], [2, 5, 5, -1]]
    assert splits.tolist() == [[1, 0, 1]] and n_slots == 1
    assert longr.tolist() == [3]
    # no split when the limit is generous; every row group gets exactly one owner item
    items, splits, n_slots, _ = _plan(lib, row_grp_ptr, blk_row_grp, blk_nz_ptr, rem_indptr,
                                      max_item_nnz=1000, long_thr=100)
    assert items[:, 3].tolist() == [-1, -1, -1] and n_slots == 0 and splits.size == 0


def test_plan_build_caps_blocks_per_item(lib):
    nb = 150
    items, splits, n_slots, _ = _plan(lib, [0, 32], [0] * nb, list(range(nb + 1)), [0] * 33,
                                      max_item_nnz=10 ** 6, long_thr=10)
    assert (items[:, 2] - items[:, 1]).max() <= 64
    assert items[0, 3] == -1 and n_slots == len(items) - 1


def test_plan_build_rejects_unsorted_blocks(lib):
    lib.spmm_last_error.restype = ctypes.c_char_p
    i32 = ctypes.POINTER(ctypes.c_int32)
    rgp = np.array([0, 1, 2], np.int32)
    brg = np.array([1, 0], np.int32)
    bnz = np.array([0, 1, 2], np.int32)
    n = ctypes.c_int32(0)
    rc = lib.spmm_boo_plan_build(2, 2, 2, rgp.ctypes.data_as(i32), brg.ctypes.data_as(i32),
                                 bnz.ctypes.data_as(i32), None, 100, 10, None, None, 0, None,
                                 ctypes.byref(n), None, None, None)
    assert rc == 1 and b'sorted' in lib.spmm_last_error()
