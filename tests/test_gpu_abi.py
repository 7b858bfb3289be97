"""The C ABI driven the way a foreign binding drives it (ctypes, no pybind):
stage a BOO matrix with spmm_boo_stage_create / _sizes / _copy / _copy_blobs,
move the arrays to the device, fill spmm_boo_desc field by field and call
spmm_boo_matmul; fill spmm_pbr_desc from the PBR arrays and call
spmm_pbr_matmul.  Y is compared with the oracle's fp64 product under the
1e-5 * (|A||X|) bound.  A descriptor that leaves the gather-pass fields unset
must be refused (SPMM_EINVAL), never run with Y rows left unwritten.

This is the recipe INTEGRATION.md gives for the reference-side binding
(bindings/bindings_boo.cu:125-313, bindings/bindings_kernels.cu:91-123 are
the interfaces it replaces)."""

import ctypes as C
from pathlib import Path

import numpy as np
import pytest
import scipy.sparse as sp
import torch

import spmm_amd as S
from oracle import oracle as O
from spmm_amd import matrices as M

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parents[1] / 'spmm_amd' / 'libspmm_amd.so'
P_ = C.c_void_p
I32P = C.POINTER(C.c_int32)


class BooHost(C.Structure):
    _fields_ = [('rows', C.c_int32), ('cols', C.c_int32), ('n_row_groups', C.c_int32),
                ('n_col_groups', C.c_int32), ('num_blocks', C.c_int32), ('dtype', C.c_int),
                ('row_grp_ptr', P_), ('row_ids', P_), ('col_grp_ptr', P_), ('col_ids', P_),
                ('blk_row_grp', P_), ('blk_col_grp', P_), ('blk_nz_ptr', P_), ('blk_shift', P_),
                ('nz_idx', P_), ('nz_val', P_), ('rem_indptr', P_), ('rem_col_ind', P_), ('rem_vals', P_)]


class StageInfo(C.Structure):
    _fields_ = [('n_tiles', C.c_int64), ('n_ent', C.c_int64), ('n_tcols', C.c_int64), ('n_splits', C.c_int64),
                ('n_long', C.c_int64), ('n_crow', C.c_int64), ('n_cnz', C.c_int64), ('n_gtask', C.c_int64),
                ('n_slots', C.c_int32), ('n_waves', C.c_int32), ('group', C.c_int32), ('n_crow_long', C.c_int32),
                ('n_stream_rows', C.c_int32), ('n_blob16', C.c_int64), ('n_gtask_order', C.c_int64)]


class BooDesc(C.Structure):
    _fields_ = [('rows', C.c_int32), ('cols', C.c_int32), ('n_stream_rows', C.c_int32), ('row_ids', P_),
                ('n_tiles', C.c_int32), ('tiles', P_), ('tile_rs', P_), ('ent_val', P_), ('ent_col', P_),
                ('tcols', P_), ('n_waves', C.c_int32), ('group', C.c_int32), ('wave_tiles', P_),
                ('n_slots', C.c_int32), ('n_splits', C.c_int32), ('splits', P_), ('n_long', C.c_int32),
                ('long_rows', P_), ('n_crow', C.c_int32), ('crow_ptr', P_), ('crow_id', P_), ('ccol', P_),
                ('cval', P_), ('n_crow_long', C.c_int32), ('n_gtask', C.c_int32), ('gtask', P_),
                ('gtask_ptr', P_), ('rem_indptr', P_), ('rem_col_ind', P_), ('rem_vals', P_),
                ('n_blob16', C.c_int64), ('blobs', P_), ('blob_first', P_), ('blob_xid', P_),
                ('gtask_order', P_)]


class PbrDesc(C.Structure):
    _fields_ = [('rows', C.c_int64), ('cols', C.c_int64), ('block_rows', C.c_int32), ('block_cols', C.c_int32),
                ('num_blocks', C.c_int64), ('itype', C.c_int), ('codes', P_), ('coords', P_), ('offsets', P_),
                ('data', P_), ('rem_indptr', P_), ('rem_col_ind', P_), ('rem_vals', P_), ('stripe_ptr', P_),
                ('n_long', C.c_int32), ('long_rows', P_), ('long_threshold', C.c_int32)]


@pytest.fixture(scope='module')
def lib():
    L = C.CDLL(str(LIB))
    L.spmm_last_error.restype = C.c_char_p
    L.spmm_boo_workspace_bytes.restype = C.c_size_t
    return L


def _np(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def stage_boo_via_c(lib, boo, dev, keep):
    """The C staging calls, then every array on the device; returns the
    filled descriptor (and keeps the buffers alive in `keep`)."""
    d = boo._d
    i32 = np.int32
    host_arrays = {
        'row_grp_ptr': _np(d['row_grp_ptr'], i32), 'row_ids': _np(d['row_ids'], i32),
        'col_grp_ptr': _np(d['col_grp_ptr'], i32), 'col_ids': _np(d['col_ids'], i32),
        'blk_row_grp': _np(d['blk_row_grp'], i32), 'blk_col_grp': _np(d['blk_col_grp'], i32),
        'blk_nz_ptr': _np(d['blk_nz_ptr'], i32), 'blk_shift': _np(d['blk_shift'], np.uint8),
        'nz_idx': _np(d['nz_idx'], np.uint16), 'nz_val': _np(d['nz_val'], np.float32),
        'rem_indptr': _np(d['rem_indptr'], i32), 'rem_col_ind': _np(d['rem_col_ind'], i32),
        'rem_vals': _np(d['rem_vals'], np.float32),
    }
    keep.append(host_arrays)
    h = BooHost(rows=boo.rows, cols=boo.cols, n_row_groups=boo.num_row_groups(),
                n_col_groups=boo.num_col_groups(), num_blocks=boo.num_blocks(), dtype=0,
                **{k: v.ctypes.data for k, v in host_arrays.items()})
    st = P_()
    rc = lib.spmm_boo_stage_create(C.byref(h), 4096, 256, 256 * 12, 4, C.c_float(1.5), C.byref(st))
    assert rc == 0, lib.spmm_last_error()
    info = StageInfo()
    assert lib.spmm_boo_stage_sizes(st, C.byref(info)) == 0
    n = info
    out = {
        'tiles': np.zeros(n.n_tiles * 8, i32), 'tile_rs': np.zeros(n.n_tiles * 33, np.uint8),
        'ent_val': np.zeros(n.n_ent, np.float32), 'ent_col': np.zeros(n.n_ent, np.uint8),
        'tcols': np.zeros(n.n_tcols, i32), 'splits': np.zeros(n.n_splits * 4, i32),
        'long_rows': np.zeros(n.n_long, i32), 'wave_tiles': np.zeros(n.n_waves + 1, i32),
        'crow_ptr': np.zeros(n.n_crow + 1, i32), 'crow_id': np.zeros(n.n_crow, i32),
        'ccol': np.zeros(n.n_cnz, i32), 'cval': np.zeros(n.n_cnz, np.float32),
        'gtask': np.zeros(n.n_gtask * 2, i32), 'gtask_ptr': np.zeros(n.n_crow_long + 1, i32),
        'blobs': np.zeros(n.n_blob16 * 4, np.uint32),
        'blob_first': np.zeros(n.n_waves * 8 if n.n_blob16 else 0, np.uint32),
        'blob_xid': np.zeros(n.n_tiles * 8 if n.n_blob16 else 0, np.uint32),
        'gtask_order': np.zeros(n.n_gtask_order, i32),
    }
    order = ('tiles', 'tile_rs', 'ent_val', 'ent_col', 'tcols', 'splits', 'long_rows', 'wave_tiles',
             'crow_ptr', 'crow_id', 'ccol', 'cval', 'gtask', 'gtask_ptr')
    rc = lib.spmm_boo_stage_copy(st, *[P_(out[k].ctypes.data) for k in order])
    assert rc == 0, lib.spmm_last_error()
    rc = lib.spmm_boo_stage_copy_blobs(st, P_(out['blobs'].ctypes.data), P_(out['blob_first'].ctypes.data),
                                       P_(out['blob_xid'].ctypes.data))
    assert rc == 0, lib.spmm_last_error()
    rc = lib.spmm_boo_stage_copy_gtask_order(st, P_(out['gtask_order'].ctypes.data))
    assert rc == 0, lib.spmm_last_error()
    lib.spmm_boo_stage_destroy(st)
    dv = {k: torch.from_numpy(v).to(dev) for k, v in out.items()}
    for k in ('row_ids', 'rem_indptr', 'rem_col_ind', 'rem_vals'):
        dv[k] = torch.from_numpy(host_arrays[k]).to(dev)
    keep.append(dv)
    ptr = lambda k: dv[k].data_ptr() if dv[k].numel() else None  # noqa: E731
    desc = BooDesc(rows=boo.rows, cols=boo.cols, n_stream_rows=n.n_stream_rows, row_ids=ptr('row_ids'),
                   n_tiles=n.n_tiles, tiles=ptr('tiles'), tile_rs=ptr('tile_rs'), ent_val=ptr('ent_val'),
                   ent_col=ptr('ent_col'), tcols=ptr('tcols'), n_waves=n.n_waves, group=n.group,
                   wave_tiles=ptr('wave_tiles'), n_slots=n.n_slots, n_splits=n.n_splits, splits=ptr('splits'),
                   n_long=n.n_long, long_rows=ptr('long_rows'), n_crow=n.n_crow, crow_ptr=ptr('crow_ptr'),
                   crow_id=ptr('crow_id'), ccol=ptr('ccol'), cval=ptr('cval'), n_crow_long=n.n_crow_long,
                   n_gtask=n.n_gtask, gtask=ptr('gtask'), gtask_ptr=ptr('gtask_ptr'),
                   rem_indptr=ptr('rem_indptr'), rem_col_ind=ptr('rem_col_ind'), rem_vals=ptr('rem_vals'),
                   n_blob16=n.n_blob16, blobs=ptr('blobs'), blob_first=ptr('blob_first'),
                   blob_xid=ptr('blob_xid'), gtask_order=ptr('gtask_order'))
    return desc, n


def _boo_call(lib, desc, X, Y, K, ws=None, wsb=0):
    stream = torch.cuda.current_stream().cuda_stream
    return lib.spmm_boo_matmul(C.byref(desc), 0, P_(X.data_ptr()), P_(Y.data_ptr()), C.c_int64(1),
                               C.c_int64(K), P_(ws.data_ptr() if ws is not None else None), C.c_size_t(wsb),
                               P_(stream))


@pytest.mark.parametrize('case', ['stencil', 'permuted_half', 'permuted', 'rmat'])
def test_boo_through_raw_c_abi(lib, case):
    """cases: a stencil (tile stream only), a stencil whose second half is
    permuted (tile stream and gather rows), a permuted stencil (gather rows),
    an R-MAT graph (gather rows, chunk tasks with the hot-column launch order
    copied out by spmm_boo_stage_copy_gtask_order)."""
    dev = torch.device('cuda', 0)
    A0 = M.stencil_27pt(16)
    if case == 'stencil':
        A = A0
    elif case == 'rmat':
        A = M.rmat(scale=17, edge_factor=8, seed=3)
    elif case == 'permuted':
        A = M.permuted(A0, seed=2)
    else:
        n = A0.shape[0]
        perm = np.arange(n)
        perm[n // 2:] = n // 2 + np.random.default_rng(4).permutation(n - n // 2)
        A = sp.csr_matrix(A0[perm][:, perm])
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32)
    keep = []
    desc, info = stage_boo_via_c(lib, boo, dev, keep)
    if case == 'stencil':
        assert info.n_crow == 0 and info.n_stream_rows == A.shape[0]
    elif case == 'rmat':
        assert info.n_gtask_order == info.n_gtask > 0 and desc.gtask_order
    elif case == 'permuted':
        assert info.n_crow == A.shape[0]
    else:
        assert 0 < info.n_crow < A.shape[0] and info.n_stream_rows > 0
    for K in (64, 32):
        X = torch.from_numpy(M.dense_x(A.shape[1], K, seed=K)).to(dev)
        Y = torch.full((A.shape[0], K), float('nan'), device=dev)   # unwritten rows would stay NaN
        wsb = lib.spmm_boo_workspace_bytes(C.byref(desc), 0, C.c_int64(1), C.c_int64(K))
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
        rc = _boo_call(lib, desc, X, Y, K, ws, wsb)
        assert rc == 0, lib.spmm_last_error()
        torch.cuda.synchronize()
        y = Y.cpu().numpy()
        assert np.isfinite(y).all()
        ratio, ok = O.within_bound(y, A, X.cpu().numpy(), 1e-5)
        assert ok, f'{case} K={K}: {ratio:.3e}'


def test_boo_incomplete_descriptor_is_refused(lib):
    """The binding INTEGRATION.md once showed left the gather-pass fields
    unset; with gather rows present that descriptor must be refused."""
    dev = torch.device('cuda', 0)
    A = M.permuted(M.stencil_27pt(12), seed=1)
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32)
    keep = []
    desc, info = stage_boo_via_c(lib, boo, dev, keep)
    assert info.n_crow > 0
    X = torch.from_numpy(M.dense_x(A.shape[1], 64)).to(dev)
    Y = torch.zeros((A.shape[0], 64), device=dev)
    bad = BooDesc.from_buffer_copy(desc)
    for f in ('n_crow', 'crow_ptr', 'crow_id', 'ccol', 'cval', 'n_crow_long', 'n_gtask', 'gtask', 'gtask_ptr'):
        setattr(bad, f, 0 if f.startswith('n_') else None)
    rc = _boo_call(lib, bad, X, Y, 64)
    assert rc == 1 and b'gather rows' in lib.spmm_last_error()
    bad2 = BooDesc.from_buffer_copy(desc)
    bad2.n_stream_rows = 0
    if info.n_stream_rows:
        assert _boo_call(lib, bad2, X, Y, 64) == 1
    torch.cuda.synchronize()


@pytest.mark.parametrize('idx', [np.int32, np.int64])
def test_pbr_through_raw_c_abi(lib, idx):
    dev = torch.device('cuda', 0)
    A = M.permuted(M.stencil_27pt(12), seed=5)
    A = sp.csr_matrix(A)
    A.indices, A.indptr = A.indices.astype(idx), A.indptr.astype(idx)   # scipy would narrow them at construction
    pbr = S.csr_to_pbr(A, 8, 8, 4).to(dev)
    d = pbr._gpu_meta.desc
    desc = PbrDesc(**{k: d[k] for k in ('rows', 'cols', 'block_rows', 'block_cols', 'num_blocks', 'itype',
                                         'codes', 'coords', 'offsets', 'data', 'rem_indptr', 'rem_col_ind',
                                         'rem_vals', 'stripe_ptr', 'n_long', 'long_rows', 'long_threshold')})
    assert desc.itype == (1 if idx == np.int64 else 0)
    K = 64
    X = torch.from_numpy(M.dense_x(A.shape[1], K)).to(dev)
    Y = torch.full((A.shape[0], K), float('nan'), device=dev)
    rc = lib.spmm_pbr_matmul(C.byref(desc), 0, P_(X.data_ptr()), P_(Y.data_ptr()), C.c_int64(1), C.c_int64(K),
                             P_(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, lib.spmm_last_error()
    torch.cuda.synchronize()
    ratio, ok = O.within_bound(Y.cpu().numpy(), A, X.cpu().numpy(), 1e-5)
    assert ok, f'{ratio:.3e}'
