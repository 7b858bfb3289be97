"""PBR (packed block rows): build, decode, stage to the GPU, multiply.

API follows ``torch_fast_spdmm/__init__.py`` (reference): ``csr_to_pbr``
:255-274, ``pbr_to_csr`` :284-290, ``.to()`` :17-40, ``pbr_matmul`` :218-252,
``pbr_batched_matmul_cuda`` :122-153, ``pbr_info`` :314-397.  Arrays come
from the native builder (``_core.csr_to_pbr``), equal to the reference's
``csr_to_pbr`` output including its per-stripe block order.

On the GPU one wave owns one stripe (block row): it decodes each 64-bit block
code in registers (row bits by shift, first value by popcount of the lower
rows, then ctz over the row's bits), accumulates the stripe's rows and their
remainder in registers and stores Y once.
"""

from __future__ import annotations

import enum
import types
from dataclasses import dataclass

import numpy as np
import scipy.sparse as sp
import torch

from ._native import core

__all__ = [
    'csr_to_pbr', 'pbr_to_csr', 'pbr_matmul', 'pbr_batched_matmul_cpu', 'pbr_batched_matmul_cuda',
    'pbr_batched_matmul_chunkcols_cuda', 'pbr_batched_matmul_nnzflat_cuda',
    'pbr_batched_matmul_variant_cuda', 'pbr_info', 'PBRInfo', 'BlockFillStats',
    'BlockStripeStats', 'PBRMatrix', 'PBRMatrixInt32Float', 'PBRMatrixInt64Float',
    'PBRMatrixInt32Double', 'PBRMatrixInt64Double', 'DataOrder',
]

LONG_ROW_THRESHOLD = 256   # longer remainder rows go to the split-row pass
# A PBR matrix whose blocks hold less than this share of its entries (a
# scattered matrix: most entries in the CSR remainder) is multiplied through
# the BOO kernels instead: its whole CSR is staged at .to('cuda') as a BOO
# staging without blocks (32-row slices), whose scattered rows the gather
# pass walks in a Cuthill-McKee order when that keeps their X rows close
# (permuted 27-point 128^3, K=32: the stripe kernel's remainder rounds take
# 1.08 ms in row order).  Block-dominated matrices keep the stripe kernel.
GATHER_MAX_BLOCK_SHARE = 0.25


class DataOrder(enum.IntEnum):
    BLOCK_ROW_MAJOR = 0
    BLOCK_COLUMN_MAJOR = 1
    INTERLEAVED_ROW_MAJOR = 2
    INTERLEAVED_COLUMN_MAJOR = 3


_ARRAYS = ('block_codes', 'block_coords', 'block_offsets', 'block_data', 'remainder_indptr',
           'remainder_col_ind', 'remainder_data')


class PBRMatrix:
    index_dtype = None
    scalar_dtype = None

    def __init__(self, d: dict):
        self._d = d
        for k in _ARRAYS:
            d[k].flags.writeable = False
        self._gpu_meta = None

    rows = property(lambda self: self._d['rows'])
    cols = property(lambda self: self._d['cols'])
    block_rows = property(lambda self: self._d['block_rows'])
    block_cols = property(lambda self: self._d['block_cols'])
    total_nnz = property(lambda self: self._d['total_nnz'])
    data_order = property(lambda self: DataOrder.BLOCK_ROW_MAJOR)

    def accounted_blocks(self):
        return int(self._d['block_codes'].size)

    def compressed_nnz(self):
        return int(self._d['block_data'].size)

    def remainder_nnz(self):
        return int(self._d['remainder_col_ind'].size)

    def __repr__(self):
        return (f'PBRMatrix({self.rows}x{self.cols}, blocks={self.accounted_blocks()}, '
                f'compressed_nnz={self.compressed_nnz()}, remainder_nnz={self.remainder_nnz()}, '
                f'total_nnz={self.total_nnz})')

    def to(self, device='cuda'):
        return _pbr_to(self, device)


for _name in _ARRAYS:
    setattr(PBRMatrix, _name, property(lambda self, _n=_name: self._d[_n]))


def _make_class(name, idx, val):
    return type(name, (PBRMatrix,), {'index_dtype': idx, 'scalar_dtype': val})


PBRMatrixInt32Float = _make_class('PBRMatrixInt32Float', np.int32, np.float32)
PBRMatrixInt64Float = _make_class('PBRMatrixInt64Float', np.int64, np.float32)
PBRMatrixInt32Double = _make_class('PBRMatrixInt32Double', np.int32, np.float64)
PBRMatrixInt64Double = _make_class('PBRMatrixInt64Double', np.int64, np.float64)
_CLASS = {(np.dtype(c.index_dtype), np.dtype(c.scalar_dtype)): c
          for c in (PBRMatrixInt32Float, PBRMatrixInt64Float, PBRMatrixInt32Double,
                    PBRMatrixInt64Double)}


def _pinned(arr, device, dtype=None):
    a = np.ascontiguousarray(arr, dtype=dtype)
    if not a.flags.writeable:       # the builder's arrays are read-only views
        a = a.copy()
    return torch.from_numpy(a).pin_memory().to(device, non_blocking=True)


def _kernel_staging(rows, cols, block_rows, block_cols, coords, rem_indptr, meta, device):
    """The stripe kernel's staging of a PBR matrix whose reference arrays are
    on ``device`` in ``meta`` (codes, coords, offsets, data, rem_*):
    ``stripe_ptr`` (each block row's blocks, which csr_to_pbr emits
    contiguously) and the rows whose remainder is long, from the host copies
    ``coords`` and ``rem_indptr``.  Returns (stripe_ptr, long_rows, desc)."""
    coords = np.asarray(coords)
    nb = coords.size // 2
    n_stripes = (rows + block_rows - 1) // block_rows if rows else 0
    stripe_of = coords.astype(np.int64).reshape(-1, 2)[:, 0] // block_rows
    if nb and np.any(np.diff(stripe_of) < 0):
        raise ValueError('PBR blocks must be grouped by block row')
    stripe_ptr = np.zeros(n_stripes + 1, dtype=np.int64)
    if nb:
        np.cumsum(np.bincount(stripe_of, minlength=n_stripes), out=stripe_ptr[1:])
    if stripe_ptr[-1] > np.iinfo(np.int32).max:
        raise ValueError('PBR block count must fit int32')
    rem_len = np.diff(np.asarray(rem_indptr, dtype=np.int64))
    long_rows = np.flatnonzero(rem_len > LONG_ROW_THRESHOLD).astype(np.int32)
    stripe_t = _pinned(stripe_ptr, device, np.int32)
    long_t = _pinned(long_rows, device, np.int32)
    torch.cuda.synchronize(device)
    p = lambda t: int(t.data_ptr())  # noqa: E731
    desc = {
        'rows': rows, 'cols': cols, 'block_rows': block_rows, 'block_cols': block_cols,
        'num_blocks': nb, 'itype': 1 if coords.dtype == np.int64 else 0,
        'codes': p(meta.codes), 'coords': p(meta.coords), 'offsets': p(meta.offsets),
        'data': p(meta.data), 'rem_indptr': p(meta.rem_indptr),
        'rem_col_ind': p(meta.rem_col_ind), 'rem_vals': p(meta.rem_vals),
        'stripe_ptr': p(stripe_t), 'n_long': int(long_rows.size),
        'long_rows': p(long_t), 'long_threshold': LONG_ROW_THRESHOLD,
    }
    return stripe_t, long_t, desc


def _pbr_to(self, device='cuda'):
    device = torch.device('cpu' if device is None else device)
    if device.type not in ('cpu', 'cuda'):
        raise ValueError('PBR supports only CPU and CUDA devices')
    if device.type == 'cuda' and device.index is None:
        device = torch.device('cuda', torch.cuda.current_device())
    target = str(device)
    existing = self._gpu_meta
    current = str(existing.codes.device) if existing is not None else 'cpu'
    if current == target:
        return self
    if device.type == 'cpu':
        self._gpu_meta = None
        return self

    d = self._d
    # Field names and dtypes of the reference's _gpu_meta (__init__.py:27-35) ...
    meta = types.SimpleNamespace(
        codes=_pinned(d['block_codes'], device, np.int64),
        coords=_pinned(d['block_coords'], device),
        offsets=_pinned(d['block_offsets'], device),
        data=_pinned(d['block_data'], device),
        rem_indptr=_pinned(d['remainder_indptr'], device),
        rem_col_ind=_pinned(d['remainder_col_ind'], device),
        rem_vals=_pinned(d['remainder_data'], device),
    )
    # ... plus the stripe pointer and the long remainder rows.
    meta.stripe_ptr, meta.long_rows, meta.desc = _kernel_staging(
        int(self.rows), int(self.cols), int(self.block_rows), int(self.block_cols),
        d['block_coords'], d['remainder_indptr'], meta, device)
    meta.gather = _gather_staging(self, device) if _scattered(self) else None
    self._gpu_meta = meta
    return self


def _scattered(pbr_mat) -> bool:
    """Most entries in the remainder (see GATHER_MAX_BLOCK_SHARE), and a CSR
    the BOO staging takes (int32 positions and columns)."""
    total = int(pbr_mat.total_nnz)
    return (total > 0 and int(pbr_mat.compressed_nnz()) < GATHER_MAX_BLOCK_SHARE * total
            and total < 2 ** 31 and int(pbr_mat.cols) < 2 ** 31 and int(pbr_mat.rows) < 2 ** 31)


def _gather_staging(pbr_mat, device):
    """The whole matrix as a BOO staging without blocks: every entry in the
    remainder CSR (pbr_to_csr's), identity 32-row slices.  Returns the staged
    tensors and the BOO launch descriptor (``desc``)."""
    from . import boo as _boo
    csr = pbr_to_csr(pbr_mat)
    rows, cols = int(pbr_mat.rows), int(pbr_mat.cols)
    i32 = np.int32
    val_t = np.dtype(pbr_mat.scalar_dtype)
    grp = lambda n: np.r_[np.arange(0, n, 32), n].astype(i32)  # noqa: E731
    d = {
        'row_grp_ptr': grp(rows), 'row_ids': np.arange(rows, dtype=i32),
        'col_grp_ptr': grp(cols), 'col_ids': np.arange(cols, dtype=i32),
        'blk_row_grp': np.zeros(0, i32), 'blk_col_grp': np.zeros(0, i32), 'blk_nz_ptr': np.zeros(1, i32),
        'blk_shift': np.zeros(0, np.uint8), 'nz_idx': np.zeros(0, np.uint16), 'nz_val': np.zeros(0, val_t),
        'rem_indptr': csr.indptr.astype(i32), 'rem_col_ind': csr.indices.astype(i32),
        'rem_vals': np.ascontiguousarray(csr.data, dtype=val_t),
        'tail_row': np.zeros(0, i32), 'tail_col': np.zeros(0, i32), 'tail_val': np.zeros(0, val_t),
    }
    row_ids_dev = torch.arange(rows, dtype=torch.int32, device=device)
    staged, rem_dev, desc = _boo._kernel_staging(rows, cols, d, True, row_ids_dev, device)
    return types.SimpleNamespace(staged=staged, rem=rem_dev, row_ids=row_ids_dev, desc=desc)


# ---------------------------------------------------------------------------
# build / convert
# ---------------------------------------------------------------------------

def _csr_parts(mat):
    if isinstance(mat, torch.Tensor):
        if mat.device.type != 'cpu':
            raise ValueError('Input tensor must be on CPU')
        if mat.layout != torch.sparse_csr or mat.dim() != 2:
            raise ValueError('Input tensor must be a 2D sparse CSR tensor')
        return (mat.crow_indices().numpy(), mat.col_indices().numpy(), mat.values().numpy(),
                int(mat.shape[0]), int(mat.shape[1]))
    if isinstance(mat, sp.csr_matrix):
        return mat.indptr, mat.indices, mat.data, int(mat.shape[0]), int(mat.shape[1])
    raise TypeError(f'Unsupported type {type(mat)}')


def csr_to_pbr(mat, block_rows: int = 8, block_cols: int = 8, min_nnz_per_block: int = 4):
    """Build PBR from a scipy CSR matrix or a CPU torch sparse CSR tensor."""
    indptr, indices, data, rows, cols = _csr_parts(mat)
    idx_t = np.dtype(indptr.dtype)
    if idx_t not in (np.dtype(np.int32), np.dtype(np.int64)) or np.dtype(indices.dtype) != idx_t:
        raise TypeError('PBR needs int32 or int64 CSR indices of one dtype')
    val_t = np.dtype(data.dtype)
    if val_t not in (np.dtype(np.float32), np.dtype(np.float64)):
        raise TypeError('PBR supports float32/float64 matrix values')
    d = core.csr_to_pbr(np.ascontiguousarray(indptr), np.ascontiguousarray(indices),
                        np.ascontiguousarray(data), rows, cols, int(block_rows), int(block_cols),
                        int(min_nnz_per_block))
    return _CLASS[(idx_t, val_t)](d)


def pbr_to_csr(pbr_mat) -> sp.csr_matrix:
    """Decode to CSR, rows sorted by (column, value) (pbr_matrix.cpp:279-331)."""
    idx_t, val_t = pbr_mat.index_dtype, pbr_mat.scalar_dtype
    indptr = np.zeros(pbr_mat.rows + 1, dtype=idx_t)
    indices = np.zeros(pbr_mat.total_nnz, dtype=idx_t)
    data = np.zeros(pbr_mat.total_nnz, dtype=val_t)
    core.pbr_to_csr(pbr_mat._d, indptr, indices, data)
    return sp.csr_matrix((data, indices, indptr), shape=(pbr_mat.rows, pbr_mat.cols))


# ---------------------------------------------------------------------------
# multiply
# ---------------------------------------------------------------------------

_DTYPE_CODE = {torch.float32: 0, torch.float64: 1}


def pbr_batched_matmul_cpu(pbr_mat, x: torch.Tensor) -> torch.Tensor:
    """CPU op: Y[B, rows, K] in the reference's loop order (pbr_matrix.cpp:17-68)."""
    if x.dim() not in (2, 3):
        raise RuntimeError(f'Expected 2D or 3D input, got {x.dim()}D')
    x3 = (x if x.dim() == 3 else x.unsqueeze(0)).contiguous()
    if x3.dtype != torch.from_numpy(np.zeros(0, pbr_mat.scalar_dtype)).dtype:
        raise TypeError(f'X dtype must match PBR values, got {x3.dtype}')
    if x3.size(1) != pbr_mat.cols:
        raise ValueError(f'X has {x3.size(1)} rows, expected {pbr_mat.cols}')
    batch, K = int(x3.size(0)), int(x3.size(2))
    y = torch.zeros((batch, pbr_mat.rows, K), dtype=x3.dtype)
    if y.numel():
        core.pbr_matmul_cpu(pbr_mat._d, x3.numpy(), y.numpy(), batch, K)
    return y


def pbr_batched_matmul_cuda(pbr_mat, x: torch.Tensor, csr_mode: int = 0,
                            smem_size: int = 2048) -> torch.Tensor:
    """GPU op: Y[B, rows, K] (not squeezed), the reference's
    ``pbr_batched_matmul_cuda`` contract.  ``csr_mode`` and ``smem_size`` are
    accepted for parity; the stripe kernel sizes its own LDS tile."""
    meta = pbr_mat._gpu_meta
    if meta is None:
        raise RuntimeError("PBRMatrix is not on GPU. Call .to('cuda') first.")
    if x.dim() not in (2, 3):
        raise ValueError(f'Expected 2D or 3D input, got {x.dim()}D')
    if not x.is_cuda or x.device != meta.codes.device:
        raise ValueError('PBR metadata and X must be on the same CUDA device')
    if x.dtype not in _DTYPE_CODE or x.dtype != meta.data.dtype:
        raise TypeError(f'X dtype must match PBR values ({meta.data.dtype}), got {x.dtype}')
    x3 = x if x.dim() == 3 else x.unsqueeze(0)
    if x3.size(1) != pbr_mat.cols:
        raise ValueError(f'X has {x3.size(1)} rows, expected {pbr_mat.cols}')
    batch, K = int(x3.size(0)), int(x3.size(2))
    with torch.cuda.device(x.device):
        xc = x3.contiguous()
        y = torch.empty((batch, pbr_mat.rows, K), dtype=x.dtype, device=x.device)
        if y.numel():
            stream = torch.cuda.current_stream(x.device).cuda_stream
            dt = _DTYPE_CODE[x.dtype]
            if meta.gather is not None:   # a scattered matrix: the BOO gather pass (GATHER_MAX_BLOCK_SHARE)
                gd = meta.gather.desc
                ws_bytes = int(core.boo_workspace_bytes(gd, dt, batch, K))
                ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
                core.boo_matmul_gpu(gd, dt, int(xc.data_ptr()), int(y.data_ptr()), batch, K,
                                    int(ws.data_ptr()) if ws is not None else 0, ws_bytes, int(stream))
            else:
                core.pbr_matmul_gpu(meta.desc, dt, int(xc.data_ptr()), int(y.data_ptr()), batch, K,
                                    int(stream))
    return y


def set_pbr_slab_bytes(nbytes: int) -> None:
    """Process-wide launch knob (like the reference's set_boo_feat_block):
    when one batch's X is larger than ``nbytes`` (0, the default: never), the
    stripe kernel runs its feature tiles one launch after another at 64
    features (32 for float64), so one tile's X can stay in the last-level
    cache.  Results are the same either way."""
    core.pbr_set_slab_bytes(int(nbytes))


def get_pbr_slab_bytes() -> int:
    return int(core.pbr_get_slab_bytes())


def pbr_launch_info(pbr_mat, features: int, batch: int = 1, x=None) -> list:
    """The kernels ``pbr_matmul(pbr_mat, X)`` launches for ``batch`` x
    ``features`` columns, in launch order, with the runtime's attributes of
    each kernel instance (the same keys as ``boo_launch_info``): the
    multiply's own dispatch, recorded instead of enqueued.  ``x`` (optional)
    supplies the alignment that steers the dispatch."""
    meta = pbr_mat._gpu_meta
    if meta is None:
        raise RuntimeError("PBRMatrix is not on GPU. Call .to('cuda') first.")
    with torch.cuda.device(meta.codes.device):
        xp = int(x.data_ptr()) if x is not None else 0
        if meta.gather is not None:
            return core.boo_launch_info(meta.gather.desc, _DTYPE_CODE[meta.data.dtype], xp, 0, int(batch),
                                        int(features))
        return core.pbr_launch_info(meta.desc, _DTYPE_CODE[meta.data.dtype], xp, 0, int(batch), int(features))


def pbr_batched_matmul_chunkcols_cuda(pbr_mat, x, csr_mode: int = 0, smem_size: int = 2048):
    """The reference's experimental chunkcols variant: same result, served by
    the stripe kernel."""
    return pbr_batched_matmul_cuda(pbr_mat, x, csr_mode, smem_size)


def pbr_batched_matmul_nnzflat_cuda(pbr_mat, x, csr_mode: int = 0, smem_size: int = 2048):
    """The reference's experimental nnzflat variant: same result, served by
    the stripe kernel."""
    return pbr_batched_matmul_cuda(pbr_mat, x, csr_mode, smem_size)


def pbr_batched_matmul_variant_cuda(pbr_mat, x, prefix, csr_mode=0, smem_size=2048):
    if prefix not in ('nnzflat_shared', 'nnzflat_onthefly'):
        raise AttributeError(f'no PBR variant {prefix!r}')
    return pbr_batched_matmul_cuda(pbr_mat, x, csr_mode, smem_size)


def pbr_matmul(pbr_mat, x: torch.Tensor, csr_mode: int = 0, smem_size: int = 2048,
               kernel: str = 'block') -> torch.Tensor:
    """Y = A @ X dispatching on ``x.device`` (__init__.py:218-252)."""
    if x.dim() not in (2, 3):
        raise ValueError(f'Expected 2D or 3D input, got {x.dim()}D')
    if x.is_cuda:
        if pbr_mat._gpu_meta is None:
            raise RuntimeError("[pbr_matmul] X is on GPU but PBRMatrix is not. Call .to('cuda') first.")
        if kernel in ('nnzflat_shared', 'nnzflat_onthefly'):
            y = pbr_batched_matmul_variant_cuda(pbr_mat, x, kernel, csr_mode, smem_size)
        elif kernel == 'chunkcols':
            y = pbr_batched_matmul_chunkcols_cuda(pbr_mat, x, csr_mode, smem_size)
        elif kernel == 'nnzflat':
            y = pbr_batched_matmul_nnzflat_cuda(pbr_mat, x, csr_mode, smem_size)
        else:
            y = pbr_batched_matmul_cuda(pbr_mat, x, csr_mode, smem_size)
    else:
        y = pbr_batched_matmul_cpu(pbr_mat, x)
    return y.squeeze(0) if x.dim() == 2 else y


# ---------------------------------------------------------------------------
# info
# ---------------------------------------------------------------------------

@dataclass(frozen=True)
class BlockFillStats:
    min: int
    max: int
    mean: float
    max_possible: int


@dataclass(frozen=True)
class BlockStripeStats:
    min: int
    max: int
    mean: float


@dataclass(frozen=True)
class PBRInfo:
    shape: tuple
    block_size: tuple
    total_nnz: int
    compressed_nnz: int
    remainder_nnz: int
    compressed_fraction: float
    num_blocks: int
    num_unique_patterns: int
    avg_reuse: float
    block_fill: BlockFillStats
    blocks_per_stripe: BlockStripeStats


def pbr_info(pbr_mat) -> PBRInfo:
    """Structural summary derived from the built arrays (no rebuild)."""
    codes = np.asarray(pbr_mat.block_codes, dtype=np.uint64)
    nb = int(codes.size)
    total = int(pbr_mat.total_nnz)
    comp = pbr_mat.compressed_nnz()
    rem = pbr_mat.remainder_nnz()
    mx = pbr_mat.block_rows * pbr_mat.block_cols
    if nb:
        pop = np.array([bin(int(c)).count('1') for c in codes], dtype=np.int32)
        n_unique = int(np.unique(codes).size)
        rows_abs = np.asarray(pbr_mat.block_coords).reshape(-1, 2)[:, 0]
        _, per_stripe = np.unique(rows_abs // pbr_mat.block_rows, return_counts=True)
        fill = BlockFillStats(int(pop.min()), int(pop.max()), float(pop.mean()), mx)
        stripes = BlockStripeStats(int(per_stripe.min()), int(per_stripe.max()),
                                   float(per_stripe.mean()))
    else:
        n_unique = 0
        fill = BlockFillStats(0, 0, 0.0, mx)
        stripes = BlockStripeStats(0, 0, 0.0)
    return PBRInfo(shape=(pbr_mat.rows, pbr_mat.cols),
                   block_size=(pbr_mat.block_rows, pbr_mat.block_cols), total_nnz=total,
                   compressed_nnz=comp, remainder_nnz=rem,
                   compressed_fraction=comp / total if total > 0 else 0.0, num_blocks=nb,
                   num_unique_patterns=n_unique, avg_reuse=nb / n_unique if n_unique else 0.0,
                   block_fill=fill, blocks_per_stripe=stripes)
