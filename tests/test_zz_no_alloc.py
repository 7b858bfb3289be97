"""spmm_boo_matmul_noalloc (allocation-free BOO entry point) against
spmm_boo_matmul with a caller workspace, through the C ABI: same staging,
same X, bit-equal Y (the same kernels run; only the workspace's memory
differs), on two calls in a row, the second with a smaller input.  The
stagings are chosen so that the workspace is really used: slices heavier
than the item limit (partial slots added by the fixup pass) and long gather
rows (chunk tasks' partial rows, also in the hot-column launch order).  A
call whose workspace would exceed the scratch is refused before any work is
enqueued."""

import ctypes as C
from pathlib import Path

import numpy as np
import pytest
import scipy.sparse as sp
import torch

import spmm_amd as S
from oracle import oracle as O
from spmm_amd import matrices as M

from test_gpu_abi import BooDesc

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parents[1] / 'spmm_amd' / 'libspmm_amd.so'


@pytest.fixture(scope='module')
def lib():
    L = C.CDLL(str(LIB))
    L.spmm_last_error.restype = C.c_char_p
    L.spmm_boo_workspace_bytes.restype = C.c_size_t
    return L


def _matrix(kind):
    if kind == 'heavy_slices':          # 32-row slices of ~6,500 entries: split into items
        A = sp.random(4096, 2048, density=0.1, format='csr', random_state=np.random.default_rng(7),
                      dtype=np.float32)
    elif kind == 'long_gather_rows':    # power-law rows: long gather rows cut into chunk tasks
        A = M.rmat(13, 16, seed=3)
    else:                               # 2^17 columns: hot-column chunk tasks launched first
        A = M.rmat(17, 8, seed=3)
    return sp.csr_matrix(A, dtype=np.float32)


def _desc(boo):
    return BooDesc(**{f: boo._gpu_meta.desc[f] for f, _ in BooDesc._fields_})


def _run(lib, desc, X, K, batch, noalloc):
    dev = X.device
    rows = desc.rows
    Y = torch.full((batch, rows, K), float('nan'), device=dev)
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    if noalloc:
        rc = lib.spmm_boo_matmul_noalloc(C.byref(desc), 0, C.c_void_p(X.data_ptr()), C.c_void_p(Y.data_ptr()),
                                         C.c_int64(batch), C.c_int64(K), stream)
    else:
        wsb = lib.spmm_boo_workspace_bytes(C.byref(desc), 0, C.c_int64(batch), C.c_int64(K))
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
        rc = lib.spmm_boo_matmul(C.byref(desc), 0, C.c_void_p(X.data_ptr()), C.c_void_p(Y.data_ptr()),
                                 C.c_int64(batch), C.c_int64(K), C.c_void_p(ws.data_ptr()), C.c_size_t(wsb), stream)
    assert rc == 0, lib.spmm_last_error()
    torch.cuda.synchronize()
    return Y


@pytest.mark.parametrize('kind', ['heavy_slices', 'long_gather_rows', 'hot_column_tasks'])
def test_noalloc_matches_workspace_entry_point(lib, kind):
    dev = torch.device('cuda', 0)
    A = _matrix(kind)
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32).to(dev)
    desc = _desc(boo)
    if kind == 'heavy_slices':
        assert desc.n_slots > 0
    else:
        assert desc.n_gtask > 0
    if kind == 'hot_column_tasks':
        assert desc.gtask_order
    # two calls in a row, the second smaller (batch and K)
    for batch, K in ((2, 96), (1, 24)):
        wsb = lib.spmm_boo_workspace_bytes(C.byref(desc), 0, C.c_int64(batch), C.c_int64(K))
        assert 0 < wsb <= 64 << 20
        X = torch.from_numpy(M.dense_x(A.shape[1], K, seed=batch * 100 + K, batch=batch)).to(dev)
        y_ws = _run(lib, desc, X, K, batch, noalloc=False)
        y_na = _run(lib, desc, X, K, batch, noalloc=True)
        assert torch.equal(y_ws, y_na), f'{kind} batch={batch} K={K}: noalloc differs from the workspace call'
        ratio, ok = O.within_bound(y_na.cpu().numpy(), A, X.cpu().numpy(), 1e-5)
        assert ok, f'{kind} batch={batch} K={K}: {ratio:.3e}'


def test_noalloc_refuses_workspace_beyond_its_scratch(lib):
    """A staging whose workspace would exceed 64 MiB: refused with
    SPMM_ENOMEM before anything is launched (the descriptor's arrays are
    never dereferenced, so none are needed)."""
    desc = BooDesc(rows=1, cols=1, n_stream_rows=0, n_crow=1, n_crow_long=1, n_gtask=1 << 20)
    rc = lib.spmm_boo_matmul_noalloc(C.byref(desc), 0, None, None, C.c_int64(1), C.c_int64(64), None)
    assert rc == 4 and b'scratch' in lib.spmm_last_error()
