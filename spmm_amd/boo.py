"""BOO (blocked COO): build, decode, stage to the GPU, multiply.

API and error behaviour follow ``torch_fast_spdmm/boo.py`` (reference):
``csr_to_boo`` :108-210, ``boo_to_csr`` :213-219, ``.to()`` :54-96,
``boo_matmul`` :230-354, ``boo_info`` / ``boo_arena_bytes`` :361-500.

The arrays are produced by the native builder (``_core.csr_to_boo``), equal to
the reference's ``csr_to_boo`` output.  ``.to('cuda')`` also stages them on the
host into the kernels' schedule (``spmm_boo_stage_create``): 32-row slices cut
into tiles of at most 32 columns, streamed by persistent workgroups that
accumulate each slice in registers and store every output row once, plus a
row-wise gather pass for empty slices and slices whose columns are too
scattered to stage.  So there is no memset of Y and no atomic.
"""

from __future__ import annotations

import enum
import types
from dataclasses import dataclass
from typing import Optional, Tuple

import numpy as np
import scipy.sparse as sp
import torch

from ._native import core
from .clustering import cluster_axes

__all__ = [
    'csr_to_boo', 'boo_to_csr', 'boo_info', 'boo_matmul', 'boo_arena_bytes', 'BOOInfo',
    'BOOMatrix', 'BOOMatrixInt32Float', 'BOOMatrixInt64Float', 'BOOMatrixInt32Double',
    'BOOMatrixInt64Double', 'BooNzOrder', 'BooSmallBlockPolicy',
    'SMALL_BLOCK_POLICIES', 'NZ_ORDERS',
]

SMALL_BLOCK_POLICIES = ('keep', 'merge', 'remainder', 'tail_batch')
NZ_ORDERS = ('rowmajor', 'colmajor')
_POLICY_CODE = {'keep': 0, 'merge': 1, 'remainder': 2, 'tail_batch': 3}
_ORDER_CODE = {'rowmajor': 0, 'colmajor': 1}

# Scheduling knobs of the GPU path (spmm_boo_stage_create in spmm_amd.h).
MAX_ITEM_NNZ = 4096        # a heavier 32-row slice is cut into several work items
LONG_ROW_THRESHOLD = 256   # longer remainder rows go to the split-row pass
WAVES_PER_CU = 16          # persistent waves per compute unit (4 per SIMD at <= 128 VGPRs)
GROUP = 4                  # slices sharing X tiles per workgroup
MIN_COL_REUSE = 1.5        # slices using each column less often go to the gather pass
RECORD_STREAM = False      # hand the kernels the one-DMA-per-step record stream (boo_blob_kernel)


class BooNzOrder(enum.IntEnum):
    ROWMAJOR = 0
    COLMAJOR = 1


class BooSmallBlockPolicy(enum.IntEnum):
    KEEP = 0
    MERGE = 1
    REMAINDER = 2


_ARRAYS = ('row_grp_ptr', 'row_ids', 'col_grp_ptr', 'col_ids', 'blk_row_grp', 'blk_col_grp',
           'blk_nz_ptr', 'blk_shift', 'nz_idx', 'nz_val', 'rem_indptr', 'rem_col_ind',
           'rem_vals', 'tail_row', 'tail_col', 'tail_val')


class BOOMatrix:
    """A built BOO matrix.  Arrays are read-only numpy views; scalars are ints.

    Concrete classes carry the index / value types in their names, as the
    reference's bound classes do (``BOOMatrixInt32Float`` ...).
    """

    index_dtype = None
    scalar_dtype = None

    def __init__(self, d: dict):
        self._d = d
        for k in _ARRAYS:
            d[k].flags.writeable = False
        self._gpu_meta = None

    # -- scalars -------------------------------------------------------------
    rows = property(lambda self: self._d['rows'])
    cols = property(lambda self: self._d['cols'])
    total_nnz = property(lambda self: self._d['total_nnz'])
    max_nr = property(lambda self: self._d['max_nr'])
    max_nc = property(lambda self: self._d['max_nc'])
    max_nnz_blk = property(lambda self: self._d['max_nnz_blk'])
    nz_order = property(lambda self: BooNzOrder(self._d['nz_order']))

    def num_blocks(self):
        return int(self._d['blk_row_grp'].size)

    def num_row_groups(self):
        return int(self._d['row_grp_ptr'].size) - 1

    def num_col_groups(self):
        return int(self._d['col_grp_ptr'].size) - 1

    def compressed_nnz(self):
        return int(self._d['nz_val'].size)

    def remainder_nnz(self):
        return int(self._d['rem_col_ind'].size)

    def tail_nnz(self):
        return int(self._d['tail_val'].size)

    def __repr__(self):
        return (f'BOOMatrix({self.rows}x{self.cols}, blocks={self.num_blocks()}, '
                f'grid={self.num_row_groups()}x{self.num_col_groups()}, max_nr={self.max_nr}, '
                f'max_nc={self.max_nc}, max_nnz_blk={self.max_nnz_blk}, '
                f'compressed_nnz={self.compressed_nnz()}, remainder_nnz={self.remainder_nnz()}, '
                f'tail_nnz={self.tail_nnz()})')

    def to(self, device='cuda'):
        return _boo_to(self, device)


def _array_property(name):
    return property(lambda self: self._d[name])


for _name in _ARRAYS:
    setattr(BOOMatrix, _name, _array_property(_name))


def _make_class(name, idx, val):
    return type(name, (BOOMatrix,), {'index_dtype': idx, 'scalar_dtype': val})


BOOMatrixInt32Float = _make_class('BOOMatrixInt32Float', np.int32, np.float32)
BOOMatrixInt64Float = _make_class('BOOMatrixInt64Float', np.int64, np.float32)
BOOMatrixInt32Double = _make_class('BOOMatrixInt32Double', np.int32, np.float64)
BOOMatrixInt64Double = _make_class('BOOMatrixInt64Double', np.int64, np.float64)
_CLASS = {(np.dtype(c.index_dtype), np.dtype(c.scalar_dtype)): c
          for c in (BOOMatrixInt32Float, BOOMatrixInt64Float, BOOMatrixInt32Double,
                    BOOMatrixInt64Double)}


# ---------------------------------------------------------------------------
# device staging
# ---------------------------------------------------------------------------

def _pinned(arr, device, dtype=None):
    a = np.ascontiguousarray(arr, dtype=dtype)
    if not a.flags.writeable:
        a = a.copy()
    return torch.from_numpy(a).pin_memory().to(device, non_blocking=True)


def _rowmajor_copy(blk_nz_ptr, nz_idx, nz_val):
    """nz_idx/nz_val re-sorted to row-major inside each block (stable)."""
    nb = blk_nz_ptr.size - 1
    blk = np.repeat(np.arange(nb, dtype=np.int64), np.diff(blk_nz_ptr.astype(np.int64)))
    perm = np.argsort(blk * 65536 + nz_idx.astype(np.int64), kind='stable')
    return nz_idx[perm], nz_val[perm]


def _merge_tail(rows, rem_indptr, rem_col_ind, rem_vals, tail_row, tail_col, tail_val):
    """Remainder CSR with the tail_batch COO folded in (rows kept; remainder
    entries first within a row)."""
    rem_rows = np.repeat(np.arange(rows, dtype=np.int64), np.diff(rem_indptr.astype(np.int64)))
    r = np.concatenate([rem_rows, tail_row.astype(np.int64)])
    c = np.concatenate([rem_col_ind.astype(np.int64), tail_col.astype(np.int64)])
    v = np.concatenate([rem_vals, tail_val])
    order = np.argsort(r, kind='stable')
    indptr = np.zeros(rows + 1, dtype=np.int64)
    np.cumsum(np.bincount(r, minlength=rows), out=indptr[1:])
    return indptr, c[order], v[order]


def _kernel_staging(rows, cols, d, rowmajor, row_ids_dev, device, rem_dev=None):
    """The kernel's staging of the BOO arrays ``d`` (the builder's field names,
    host arrays) on ``device``: the tile stream and gather rows
    (``spmm_boo_stage_*``) and the remainder CSR with the tail folded in.
    ``row_ids_dev`` is ``row_ids`` on the device; ``rem_dev`` the remainder CSR
    already there, when there is no tail to fold in.  Returns (stage tensors,
    remainder tensors, launch descriptor)."""
    i32 = np.int32
    if rowmajor:
        k_idx, k_val = d['nz_idx'], d['nz_val']
    else:
        k_idx, k_val = _rowmajor_copy(np.asarray(d['blk_nz_ptr']), np.asarray(d['nz_idx']),
                                      np.asarray(d['nz_val']))
    if np.asarray(d['tail_col']).size:
        k_rem = _merge_tail(rows, d['rem_indptr'], d['rem_col_ind'], d['rem_vals'],
                            d['tail_row'], d['tail_col'], d['tail_val'])
        rem_dev = None
    else:
        k_rem = (d['rem_indptr'], d['rem_col_ind'], d['rem_vals'])
    k_rem_indptr = np.ascontiguousarray(k_rem[0], dtype=i32)
    k_rem_col = np.ascontiguousarray(k_rem[1], dtype=i32)
    k_rem_val = np.ascontiguousarray(k_rem[2])
    n_cu = torch.cuda.get_device_properties(device).multi_processor_count
    host = {
        'rows': rows, 'cols': cols,
        'n_row_groups': int(np.asarray(d['row_grp_ptr']).size) - 1,
        'n_col_groups': int(np.asarray(d['col_grp_ptr']).size) - 1,
        'num_blocks': int(np.asarray(d['blk_row_grp']).size),
        'row_grp_ptr': np.ascontiguousarray(d['row_grp_ptr'], dtype=i32),
        'row_ids': np.ascontiguousarray(d['row_ids'], dtype=i32),
        'col_grp_ptr': np.ascontiguousarray(d['col_grp_ptr'], dtype=i32),
        'col_ids': np.ascontiguousarray(d['col_ids'], dtype=i32),
        'blk_row_grp': np.ascontiguousarray(d['blk_row_grp'], dtype=i32),
        'blk_col_grp': np.ascontiguousarray(d['blk_col_grp'], dtype=i32),
        'blk_nz_ptr': np.ascontiguousarray(d['blk_nz_ptr'], dtype=i32),
        'blk_shift': np.ascontiguousarray(d['blk_shift'], dtype=np.uint8),
        'nz_idx': np.ascontiguousarray(k_idx, dtype=np.uint16),
        'nz_val': np.ascontiguousarray(k_val),
        'rem_indptr': k_rem_indptr, 'rem_col_ind': k_rem_col, 'rem_vals': k_rem_val,
    }
    stage = core.boo_stage(host, MAX_ITEM_NNZ, LONG_ROW_THRESHOLD, max(GROUP, n_cu * WAVES_PER_CU), GROUP,
                           MIN_COL_REUSE)
    names = ['tiles', 'tile_rs', 'ent_val', 'ent_col', 'tcols', 'splits', 'long_rows',
             'wave_tiles', 'crow_ptr', 'crow_id', 'ccol', 'cval', 'gtask', 'gtask_ptr']
    records = RECORD_STREAM and int(stage['n_blob16']) > 0
    if records:
        names += ['blobs', 'blob_first', 'blob_xid']
    ordered = int(stage['n_gtask_order']) > 0   # hot-column chunk tasks first
    if ordered:
        names += ['gtask_order']
    g = types.SimpleNamespace(**{k: _pinned(stage[k], device) for k in names})
    if rem_dev is None:
        rem_dev = (_pinned(k_rem_indptr, device), _pinned(k_rem_col, device), _pinned(k_rem_val, device))
    torch.cuda.synchronize(device)

    p = lambda t: int(t.data_ptr())  # noqa: E731
    desc = {
        'rows': rows, 'cols': cols, 'n_stream_rows': int(stage['n_stream_rows']), 'row_ids': p(row_ids_dev),
        'n_tiles': int(stage['n_tiles']), 'tiles': p(g.tiles),
        'tile_rs': p(g.tile_rs), 'ent_val': p(g.ent_val), 'ent_col': p(g.ent_col),
        'tcols': p(g.tcols), 'n_waves': int(stage['n_waves']), 'group': int(stage['group']),
        'wave_tiles': p(g.wave_tiles),
        'n_slots': int(stage['n_slots']), 'n_splits': int(stage['n_splits']), 'splits': p(g.splits),
        'n_long': int(stage['n_long']), 'long_rows': p(g.long_rows),
        'n_crow': int(stage['n_crow']), 'crow_ptr': p(g.crow_ptr), 'crow_id': p(g.crow_id),
        'ccol': p(g.ccol), 'cval': p(g.cval), 'n_crow_long': int(stage['n_crow_long']),
        'n_gtask': int(stage['n_gtask']), 'gtask': p(g.gtask), 'gtask_ptr': p(g.gtask_ptr),
        'rem_indptr': p(rem_dev[0]), 'rem_col_ind': p(rem_dev[1]), 'rem_vals': p(rem_dev[2]),
        'n_blob16': int(stage['n_blob16']) if records else 0,
        'blobs': p(g.blobs) if records else 0, 'blob_first': p(g.blob_first) if records else 0,
        'blob_xid': p(g.blob_xid) if records else 0,
        'gtask_order': p(g.gtask_order) if ordered else 0,
    }
    return g, rem_dev, desc


def _boo_to(self, device='cuda'):
    device = torch.device('cpu' if device is None else device)
    if device.type not in ('cpu', 'cuda'):
        raise ValueError('BOO supports only CPU and CUDA devices')
    if device.type == 'cuda' and device.index is None:
        device = torch.device('cuda', torch.cuda.current_device())
    target = str(device)
    existing = self._gpu_meta
    current = str(existing.nz_val.device) if existing is not None else 'cpu'
    if current == target:
        return self
    if device.type == 'cpu':
        self._gpu_meta = None
        return self
    if max(self.rows, self.cols, self.total_nnz) > np.iinfo(np.int32).max:
        raise ValueError('BOO CUDA metadata must fit int32')

    d = self._d
    i32 = np.int32
    # Field names and dtypes of the reference's _gpu_meta (boo.py:72-92) ...
    meta = types.SimpleNamespace(
        row_grp_ptr=_pinned(d['row_grp_ptr'], device, i32),
        row_ids=_pinned(d['row_ids'], device, i32),
        col_grp_ptr=_pinned(d['col_grp_ptr'], device, i32),
        col_ids=_pinned(d['col_ids'], device, i32),
        blk_row_grp=_pinned(d['blk_row_grp'], device, i32),
        blk_col_grp=_pinned(d['blk_col_grp'], device, i32),
        blk_nz_ptr=_pinned(d['blk_nz_ptr'], device, i32),
        blk_shift=_pinned(d['blk_shift'], device, np.uint8),
        nz_idx=_pinned(np.ascontiguousarray(d['nz_idx']).view(np.int16), device),
        nz_val=_pinned(d['nz_val'], device),
        rem_indptr=_pinned(d['rem_indptr'], device, i32),
        rem_col_ind=_pinned(d['rem_col_ind'], device, i32),
        rem_vals=_pinned(d['rem_vals'], device),
        tail_row=_pinned(d['tail_row'], device, i32),
        tail_col=_pinned(d['tail_col'], device, i32),
        tail_val=_pinned(d['tail_val'], device),
    )
    # ... plus the kernel's staging (tile stream, gather rows, remainder CSR
    # with the tail folded in) and its launch descriptor.
    rem_dev = None if self.tail_nnz() else (meta.rem_indptr, meta.rem_col_ind, meta.rem_vals)
    meta.stage, (meta.k_rem_indptr, meta.k_rem_col_ind, meta.k_rem_vals), meta.desc = _kernel_staging(
        int(self.rows), int(self.cols), d, self.nz_order == BooNzOrder.ROWMAJOR, meta.row_ids, device,
        rem_dev)
    self._gpu_meta = meta
    return self


# ---------------------------------------------------------------------------
# build / convert
# ---------------------------------------------------------------------------

def _as_scipy_csr(mat):
    if isinstance(mat, torch.Tensor):
        if mat.device.type != 'cpu':
            raise ValueError('Input tensor must be on CPU')
        if mat.layout != torch.sparse_csr or mat.dim() != 2:
            raise ValueError('Input tensor must be a 2D sparse CSR tensor')
        return sp.csr_matrix((mat.values().numpy(), mat.col_indices().numpy(),
                              mat.crow_indices().numpy()), shape=tuple(mat.shape))
    if isinstance(mat, sp.csr_matrix):
        return mat
    raise TypeError(f'Unsupported type {type(mat)}')


def csr_to_boo(mat, cluster: str = 'hem', target_nr: int = 32, target_nc: int = 32,
               max_nr: Optional[int] = None, max_nc: Optional[int] = None,
               max_block_nnz: Optional[int] = None,
               small_block_policy: str = 'remainder', small_block_threshold: int = 4,
               nz_order: str = 'rowmajor', seed: int = 0,
               symmetric: Optional[bool] = None,
               row_labels: Optional[np.ndarray] = None,
               col_labels: Optional[np.ndarray] = None,
               hem_feasible_first: bool = True):
    """Cluster both axes (or take ``row_labels``/``col_labels``) and build BOO.

    Same arguments, validation and errors as the reference's ``csr_to_boo``
    (boo.py:108-210).  The result's class name carries the index and value
    types of the input CSR.
    """
    if small_block_policy not in SMALL_BLOCK_POLICIES:
        raise ValueError(f'small_block_policy must be one of {SMALL_BLOCK_POLICIES}')
    if nz_order not in NZ_ORDERS:
        raise ValueError(f'nz_order must be one of {NZ_ORDERS}')
    for name, value in (('target_nr', target_nr), ('target_nc', target_nc), ('max_nr', max_nr),
                        ('max_nc', max_nc), ('max_block_nnz', max_block_nnz)):
        if value is not None and (not isinstance(value, (int, np.integer)) or value <= 0):
            raise ValueError(f'{name} must be a positive integer')
    if not isinstance(small_block_threshold, (int, np.integer)) or small_block_threshold < 0:
        raise ValueError('small_block_threshold must be a nonnegative integer')
    if (row_labels is None) != (col_labels is None):
        raise ValueError('row_labels and col_labels must be supplied together')

    csr = _as_scipy_csr(mat)
    if csr.dtype not in (np.dtype(np.float32), np.dtype(np.float64)):
        raise TypeError('BOO supports float32/float64 matrix values')
    csr.check_format(full_check=True)

    if max_nr is None:
        max_nr = target_nr
    if max_nc is None:
        max_nc = target_nc
    if row_labels is None or col_labels is None:
        row_labels, col_labels = cluster_axes(
            csr, method=cluster, target_nr=target_nr, target_nc=target_nc, max_nr=max_nr,
            max_nc=max_nc, max_block_nnz=max_block_nnz, seed=seed, symmetric=symmetric,
            feasible_first=hem_feasible_first)

    for name, labels, size in (('row_labels', row_labels, csr.shape[0]),
                               ('col_labels', col_labels, csr.shape[1])):
        labels = np.asarray(labels)
        if labels.ndim != 1 or labels.size != size:
            raise ValueError(f'{name} must be a 1D array matching the matrix dimension')
        if not np.issubdtype(labels.dtype, np.integer):
            raise TypeError(f'{name} must contain integer labels')
        if labels.size and (labels.min() < 0 or labels.max() >= size):
            raise ValueError(f'{name} labels must be in [0, {size})')

    idx_t = np.int64 if csr.indptr.dtype == np.int64 or csr.indices.dtype == np.int64 else np.int32
    d = core.csr_to_boo(
        np.ascontiguousarray(csr.indptr, dtype=idx_t), np.ascontiguousarray(csr.indices, dtype=idx_t),
        np.ascontiguousarray(csr.data), int(csr.shape[0]), int(csr.shape[1]),
        np.ascontiguousarray(row_labels, dtype=np.int32),
        np.ascontiguousarray(col_labels, dtype=np.int32),
        _POLICY_CODE[small_block_policy], int(small_block_threshold), _ORDER_CODE[nz_order])
    return _CLASS[(np.dtype(idx_t), csr.dtype)](d)


def boo_to_csr(boo_mat) -> sp.csr_matrix:
    """Decode to CSR, each row sorted by (column, value) (boo_matrix.cpp:277-333)."""
    idx_t, val_t = boo_mat.index_dtype, boo_mat.scalar_dtype
    indptr = np.zeros(boo_mat.rows + 1, dtype=idx_t)
    indices = np.zeros(boo_mat.total_nnz, dtype=idx_t)
    data = np.zeros(boo_mat.total_nnz, dtype=val_t)
    core.boo_to_csr(boo_mat._d, indptr, indices, data)
    return sp.csr_matrix((data, indices, indptr), shape=(boo_mat.rows, boo_mat.cols))


# ---------------------------------------------------------------------------
# multiply
# ---------------------------------------------------------------------------

_DTYPE_CODE = {torch.float32: 0, torch.float64: 1}


def boo_matmul(boo_mat, x: torch.Tensor, threads: int = 256, p: int = 64,
               csr_mode: int = 0, row_seg: Optional[bool] = None,
               launch_mode: str = 'legacy', execution_plan=None,
               features_per_thread: int = 1,
               nnzflat_impl: Optional[str] = None) -> torch.Tensor:
    """Y = A @ X, dispatching on ``x.device`` (boo.py:230-354).

    The launch knobs (``threads``, ``p``, ``csr_mode``, ``row_seg``,
    ``launch_mode``, ``features_per_thread``, ``nnzflat_impl``) are validated
    exactly as the reference does; the gfx950 kernel derives its own launch
    shape from K, so they do not change the result or the schedule.
    """
    if launch_mode not in ('legacy', 'auto'):
        raise ValueError("launch_mode must be 'legacy' or 'auto'")
    if x.dim() not in (2, 3):
        raise ValueError(f'Expected 2D or 3D input, got {x.dim()}D')
    if x.layout != torch.strided or x.device.type not in ('cpu', 'cuda'):
        raise ValueError('X must be a dense CPU or CUDA tensor')
    if x.size(-2) != boo_mat.cols:
        raise ValueError(f'X has {x.size(-2)} rows, expected {boo_mat.cols}')
    expected = {np.float32: torch.float32, np.float64: torch.float64}[boo_mat.scalar_dtype]
    if x.dtype != expected:
        raise TypeError(f'X dtype must match BOO values ({expected}), got {x.dtype}')
    if execution_plan is not None and not x.is_cuda:
        raise ValueError('BOO execution plans require CUDA inputs')

    x3 = x if x.dim() == 3 else x.unsqueeze(0)
    batch, K = int(x3.size(0)), int(x3.size(2))

    if not x.is_cuda:
        xc = x3.contiguous()
        y = torch.zeros((batch, boo_mat.rows, K), dtype=x.dtype)
        if y.numel():
            core.boo_matmul_cpu(boo_mat._d, xc.numpy(), y.numpy(), batch, K)
        return y.squeeze(0) if x.dim() == 2 else y

    meta = boo_mat._gpu_meta
    if meta is None:
        raise RuntimeError("[boo_matmul] X is on GPU but BOOMatrix is not. Call .to('cuda') first.")
    if meta.nz_val.device != x.device:
        raise ValueError('BOO metadata and X must be on the same CUDA device')
    if threads not in (128, 256, 512):
        raise ValueError('threads must be one of 128, 256, 512')
    if p not in (8, 16, 32, 64, 128):
        raise ValueError('p must be one of 8, 16, 32, 64, 128')
    if csr_mode not in (0, 1, 2):
        raise ValueError('csr_mode must be one of 0, 1, 2')
    if features_per_thread not in (1, 2, 4):
        raise ValueError('features_per_thread must be one of 1, 2, 4')
    if features_per_thread == 4 and x.dtype != torch.float32:
        raise ValueError('features_per_thread=4 requires float32')
    if nnzflat_impl not in (None, 'reference', 'template'):
        raise ValueError("nnzflat_impl must be None, 'reference' or 'template'")
    if row_seg is None:
        row_seg = boo_mat.nz_order == BooNzOrder.ROWMAJOR
    elif row_seg and boo_mat.nz_order != BooNzOrder.ROWMAJOR:
        raise ValueError('row_seg=True requires a matrix built with nz_order="rowmajor"')
    if row_seg:
        if nnzflat_impl is not None:
            raise ValueError('nnzflat_impl applies only to row_seg=False')
    else:
        if features_per_thread == 4:
            raise ValueError('nnzflat (row_seg=False) supports features_per_thread 1 or 2')
        if nnzflat_impl == 'reference' and features_per_thread != 1:
            raise ValueError("nnzflat_impl='reference' is the FPT=1 kernel; use 'template'")
    if execution_plan is not None:
        from .plan import BOOExecutionPlan
        if (not isinstance(execution_plan, BOOExecutionPlan) or execution_plan.matrix is not boo_mat
                or execution_plan.source_meta is not meta):
            raise ValueError('Execution plan does not match this matrix and its current CUDA staging')
        if launch_mode != 'auto' or not row_seg or p != execution_plan.p:
            raise ValueError('Execution plans require launch_mode="auto", row_seg=True and the prepared p')

    with torch.cuda.device(x.device):
        xc = x3.contiguous()
        y = torch.empty((batch, boo_mat.rows, K), dtype=x.dtype, device=x.device)
        if y.numel():
            dt = _DTYPE_CODE[x.dtype]
            ws_bytes = int(core.boo_workspace_bytes(meta.desc, dt, batch, K))
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
            stream = torch.cuda.current_stream(x.device).cuda_stream
            core.boo_matmul_gpu(meta.desc, dt, int(xc.data_ptr()), int(y.data_ptr()), batch, K,
                                int(ws.data_ptr()) if ws is not None else 0, ws_bytes, int(stream))
    return y.squeeze(0) if x.dim() == 2 else y


# ---------------------------------------------------------------------------
# offline metrics
# ---------------------------------------------------------------------------

# gfx950 compute unit limits used by the occupancy estimate.
_LDS_PER_CU = 163840
_MAX_WAVES_PER_CU = 32
_WAVE = 64


@dataclass(frozen=True)
class BOOInfo:
    shape: Tuple[int, int]
    total_nnz: int
    compressed_nnz: int
    remainder_nnz: int
    tail_nnz: int
    compressed_fraction: float
    boo_fraction: float
    num_blocks: int
    num_row_groups: int
    num_col_groups: int
    n_r_mean: float
    n_r_max: int
    n_c_mean: float
    n_c_max: int
    nnz_per_block_mean: float
    nnz_per_block_max: int
    nnz_per_block_hist: dict
    x_loads: int
    y_writes: int
    arithmetic_intensity: float
    scalar_bytes: int
    p: int
    threads: int
    arena_bytes: int
    ctas_per_sm: int
    occupancy_pct: float


def boo_arena_bytes(max_nr: int, max_nc: int, max_nnz_blk: int, p: int, scalar_bytes: int,
                    row_seg: bool = True) -> int:
    """Shared-memory bytes the reference's launcher requests for these global
    maxima (boo.py:412-430); kept for API parity and cross-checking."""
    data = max_nnz_blk * (scalar_bytes + 2)
    if row_seg:
        ids = 4 * (max_nr + max_nc) + 4 * (max_nr + 1)
        tiles = scalar_bytes * p * max_nc
    else:
        ids = 4 * (max_nr + max_nc)
        tiles = scalar_bytes * p * (max_nr + max_nc)
    return data + ids + tiles


def _gfx950_lds_bytes(scalar_bytes: int) -> int:
    """Offline estimate of the LDS per workgroup of the gfx950 tile-stream
    kernel, for a matrix that is not staged on a GPU (a staged one reports
    the runtime's figure, boo_launch_info).  float: the LDS-DMA kernel's
    chunk-major tile, double-buffered, 8 serial-row sums per wave and 136
    entries per wave.  Other types: the register-staged kernel's padded tile
    (row stride 64 features + 32 bytes), the same per-wave arrays and a
    32-entry column table per wave."""
    entry = 8 if scalar_bytes <= 4 else 16    # {uint32 column, value}, aligned
    if scalar_bytes == 4:
        return 2 * 8192 + 8192 + 4 * 136 * entry + 16
    stride = (64 + 32 // scalar_bytes) * scalar_bytes
    return 2 * 32 * stride + 4 * 8 * stride + 4 * 136 * entry + 4 * 32 * 4


def boo_launch_info(boo_mat, features: int, batch: int = 1, x: Optional[torch.Tensor] = None,
                    dtype: Optional[torch.dtype] = None) -> list:
    """The kernels ``boo_matmul(boo_mat, X)`` launches for ``batch`` x
    ``features`` columns, in launch order, each with the runtime's attributes
    of that kernel instance: ``registers_per_thread`` (VGPRs),
    ``local_bytes_per_thread`` (scratch: spills), ``static_shared_bytes``
    (LDS), ``max_threads_per_block`` and ``max_active_blocks_per_cu``
    (resident workgroups per CU at its block size), plus ``grid`` and
    ``threads``.  The multiply's own dispatch runs with every launch recorded
    instead of enqueued, so the list is what the multiply launches.  Replaces
    boo_rowseg_launch_info / boo_nnzflat_launch_info
    (kernels/boo_kernel.cu:710-797, bindings/bindings_boo.cu:421-475).
    ``x`` (optional) supplies the alignment that steers the dispatch;
    ``dtype`` defaults to the matrix's scalar type."""
    meta = boo_mat._gpu_meta
    if meta is None:
        raise RuntimeError("[boo_launch_info] the BOOMatrix is not on a GPU. Call .to('cuda') first.")
    if dtype is None:
        dtype = torch.float32 if np.dtype(boo_mat.scalar_dtype) == np.float32 else torch.float64
    with torch.cuda.device(meta.nz_val.device):
        xp = int(x.data_ptr()) if x is not None else 0
        return core.boo_launch_info(meta.desc, _DTYPE_CODE[dtype], xp, 0, int(batch), int(features))


def boo_info(boo_mat, p: int = 64, threads: int = 256, row_seg: bool = True) -> BOOInfo:
    """Structural summary derived from the built format.  ``arena_bytes`` and
    the occupancy fields describe this library's gfx950 kernel, not the
    reference's CUDA launch: for a matrix staged on a GPU, the runtime's
    figures (LDS, resident workgroups per CU) of the first kernel a multiply
    of ``p`` features launches (boo_launch_info); otherwise an offline
    estimate for the tile-stream kernel (256-lane workgroups of 4 waves,
    LDS-bound count per CU)."""
    scalar_bytes = np.dtype(boo_mat.scalar_dtype).itemsize
    row_grp_ptr = np.asarray(boo_mat.row_grp_ptr, dtype=np.int64)
    col_grp_ptr = np.asarray(boo_mat.col_grp_ptr, dtype=np.int64)
    blk_row_grp = np.asarray(boo_mat.blk_row_grp, dtype=np.int64)
    blk_col_grp = np.asarray(boo_mat.blk_col_grp, dtype=np.int64)
    blk_nz_ptr = np.asarray(boo_mat.blk_nz_ptr, dtype=np.int64)
    rg_size = np.diff(row_grp_ptr)
    cg_size = np.diff(col_grp_ptr)
    nb = int(blk_row_grp.size)
    if nb:
        n_r = rg_size[blk_row_grp]
        n_c = cg_size[blk_col_grp]
        nnz_per_block = np.diff(blk_nz_ptr)
        x_loads = int(n_c.sum())
        y_writes = int(n_r.sum())
        buckets = np.where(nnz_per_block > 0,
                           np.floor(np.log2(np.maximum(nnz_per_block, 1))).astype(int), 0)
        hist = {f'{1 << b}-{(1 << (b + 1)) - 1}': int(cnt)
                for b, cnt in zip(*np.unique(buckets, return_counts=True))}
    else:
        n_r = n_c = nnz_per_block = np.zeros(0, dtype=np.int64)
        x_loads = y_writes = 0
        hist = {}
    compressed = boo_mat.compressed_nnz()
    tail = boo_mat.tail_nnz()
    total = int(boo_mat.total_nnz)
    if boo_mat._gpu_meta is not None and int(boo_mat.rows) > 0 and int(boo_mat.cols) > 0:
        first = boo_launch_info(boo_mat, p)[0]
        arena = int(first['static_shared_bytes'])
        wgs = int(first['max_active_blocks_per_cu'])
        waves = wgs * -(-int(first['threads']) // _WAVE)
    else:
        arena = _gfx950_lds_bytes(scalar_bytes)
        wgs = max(0, min(_LDS_PER_CU // arena, _MAX_WAVES_PER_CU // 4))
        waves = 4 * wgs
    return BOOInfo(
        shape=(int(boo_mat.rows), int(boo_mat.cols)), total_nnz=total, compressed_nnz=compressed,
        remainder_nnz=boo_mat.remainder_nnz(), tail_nnz=tail,
        compressed_fraction=compressed / total if total else 0.0,
        boo_fraction=(compressed + tail) / total if total else 0.0,
        num_blocks=nb, num_row_groups=int(rg_size.size), num_col_groups=int(cg_size.size),
        n_r_mean=float(n_r.mean()) if nb else 0.0, n_r_max=int(n_r.max()) if nb else 0,
        n_c_mean=float(n_c.mean()) if nb else 0.0, n_c_max=int(n_c.max()) if nb else 0,
        nnz_per_block_mean=float(nnz_per_block.mean()) if nb else 0.0,
        nnz_per_block_max=int(nnz_per_block.max()) if nb else 0, nnz_per_block_hist=hist,
        x_loads=x_loads, y_writes=y_writes,
        arithmetic_intensity=compressed / x_loads if x_loads else 0.0,
        scalar_bytes=scalar_bytes, p=p, threads=threads, arena_bytes=arena, ctas_per_sm=wgs,
        occupancy_pct=100.0 * waves / _MAX_WAVES_PER_CU)
