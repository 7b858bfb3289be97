"""C++-timed SpMM harnesses and the vendor SpMM baseline.

The reference's measurement adjuncts, with their constructor arguments,
validation messages and methods (``run``, ``timed_run``, ``output``,
``info``):

* :class:`BOOTimedSpMM` -- ``bindings/bindings_boo_timed.cu:24-315``;
* :class:`PBRTimedSpMM` -- ``bindings/bindings_pbr_timed.cu:24-210``;
* :class:`DirectSpMM` -- ``bindings/bindings_cusparse.cu:21-160`` (a
  persistent vendor SpMM plan; rocSPARSE's generic SpMM here).

Everything a run needs (staging, output, workspace, timer) is made once in
the constructor, outside any measurement.  ``timed_run`` is one native call
that records an event on the construction stream, makes exactly the product
call, records a second event and waits for it, so no Python runs inside the
interval it returns (milliseconds).  ``run`` and ``timed_run`` refuse any
stream but the construction stream, like the reference.

The BOO and PBR harnesses take the reference's device tensors (a
``_gpu_meta``'s fields) and stage this library's kernel schedule from host
copies of them at construction; nothing falls back to a CPU path.
"""

from __future__ import annotations

import numpy as np
import torch

from ._native import core
from . import boo as _boo
from . import pbr as _pbr

__all__ = ['BOOTimedSpMM', 'PBRTimedSpMM', 'DirectSpMM']


def _stream_of(device):
    return torch.cuda.current_stream(device).cuda_stream


class _Timer:
    """An event pair of the C ABI (spmm_timer)."""

    def __init__(self):
        self.handle = int(core.timer_create())

    def __del__(self):
        h, self.handle = getattr(self, 'handle', 0), 0
        if h:
            core.timer_destroy(h)


class BOOTimedSpMM:
    """Y = A X for a BOO matrix given as the reference's CUDA metadata tensors,
    fp32 only (bindings/bindings_boo_timed.cu:139-243).

    ``threads``, ``p``, ``csr_mode``, ``row_seg``, ``nnzflat_*``,
    ``launch_mode``, ``buckets`` and the plan row tables are validated as the
    reference does; the gfx950 kernels derive their own launch shape, so they
    change neither the result nor what is timed.  ``diagnostic_raw_store``
    (the reference's raw-store block kernel, incorrect by construction) has
    no counterpart here and is refused."""

    def __init__(self, rows, cols, max_nr, max_nc, max_nnz_blk,
                 row_grp_ptr, row_ids, col_grp_ptr, col_ids, blk_row_grp, blk_col_grp,
                 blk_nz_ptr, blk_shift, nz_idx, nz_val, rem_indptr, rem_col_ind, rem_vals,
                 tail_row, tail_col, tail_val, x, threads=256, p=64, csr_mode=0, row_seg=True,
                 diagnostic_raw_store=False, nnzflat_fpt=1, nnzflat_reference=True,
                 launch_mode='legacy', buckets=(), plan_row_ptr=None, plan_row_starts=None):
        buckets = list(buckets)
        if launch_mode not in ('auto', 'legacy'):
            raise RuntimeError("launch_mode must be 'auto' or 'legacy'")
        if buckets and not (launch_mode == 'auto' and row_seg and len(buckets) % 5 == 0):
            raise RuntimeError('BOO execution plans require auto rowseg and 5-element buckets')
        if (plan_row_ptr is None) != (plan_row_starts is None):
            raise RuntimeError('BOO plan row tables must be provided together')
        if plan_row_ptr is not None:
            for t in (plan_row_ptr, plan_row_starts):
                if (t.device != x.device or not t.is_contiguous() or t.dtype != torch.int32
                        or t.dim() != 1):
                    raise RuntimeError('BOO plan row tables must be contiguous CUDA int32 vectors')
            if plan_row_ptr.numel() and (plan_row_ptr.numel() != blk_row_grp.numel() + 1
                                         or plan_row_starts.numel() < blk_row_grp.numel()):
                raise RuntimeError('invalid BOO plan row table sizes')
        if not x.is_cuda or x.dtype != torch.float32:
            raise RuntimeError('BOOTimedSpMM: X must be a CUDA FP32 tensor')
        if x.dim() not in (2, 3):
            raise RuntimeError('BOOTimedSpMM: X must be 2D or 3D')
        if threads not in (128, 256, 512):
            raise RuntimeError('BOOTimedSpMM: threads must be 128, 256 or 512')
        if p not in (8, 16, 32, 64, 128):
            raise RuntimeError('BOOTimedSpMM: p must be 8, 16, 32, 64 or 128')
        arrays = dict(row_grp_ptr=row_grp_ptr, row_ids=row_ids, col_grp_ptr=col_grp_ptr, col_ids=col_ids,
                      blk_row_grp=blk_row_grp, blk_col_grp=blk_col_grp, blk_nz_ptr=blk_nz_ptr,
                      blk_shift=blk_shift, nz_idx=nz_idx, nz_val=nz_val, rem_indptr=rem_indptr,
                      rem_col_ind=rem_col_ind, rem_vals=rem_vals, tail_row=tail_row, tail_col=tail_col,
                      tail_val=tail_val)
        for t in arrays.values():
            if t.device != x.device or not t.is_contiguous():
                raise RuntimeError("BOOTimedSpMM: BOO metadata must be contiguous tensors on X's device")
        if nz_val.dtype != torch.float32 or rem_vals.dtype != torch.float32:
            raise RuntimeError('BOOTimedSpMM: nz_val/rem_vals must be fp32 (this harness is fp32 only)')
        if diagnostic_raw_store and not row_seg:
            raise RuntimeError('BOOTimedSpMM: diagnostic_raw_store requires row_seg=True')
        if nnzflat_fpt not in (1, 2):
            raise RuntimeError('BOOTimedSpMM: nnzflat_fpt must be 1 or 2')
        if row_seg and not (nnzflat_fpt == 1 and nnzflat_reference):
            raise RuntimeError('BOOTimedSpMM: nnzflat settings require row_seg=False')
        if nnzflat_fpt != 1 and nnzflat_reference:
            raise RuntimeError('BOOTimedSpMM: nnzflat FPT=2 requires nnzflat_reference=False')
        if diagnostic_raw_store:
            raise RuntimeError('BOOTimedSpMM: diagnostic_raw_store has no gfx950 kernel '
                               '(the stream kernel stores every output row once)')
        if max(rows, cols, int(nz_val.numel()) + int(rem_vals.numel()) + int(tail_val.numel())) \
                > np.iinfo(np.int32).max:
            raise RuntimeError('BOOTimedSpMM: BOO CUDA metadata must fit int32')

        self._device = x.device
        self._squeeze = x.dim() == 2
        self._diag = bool(diagnostic_raw_store)
        self._row_seg = bool(row_seg)
        self._fpt, self._ref = int(nnzflat_fpt), bool(nnzflat_reference)
        with torch.cuda.device(x.device):
            self._stream = _stream_of(x.device)
            self._x3 = (x.unsqueeze(0) if x.dim() == 2 else x).contiguous()
            host = {k: t.cpu().numpy() for k, t in arrays.items()}
            host['nz_idx'] = np.ascontiguousarray(host['nz_idx']).view(np.uint16)
            # sorting by (block, nz_idx) gives row-major order whatever order
            # the nonzeros were built in
            self._stage, self._rem, self._desc = _boo._kernel_staging(
                int(rows), int(cols), host, False, row_ids, x.device)
            self._keep = arrays  # the device tensors the descriptor points into
            batch, K = int(self._x3.size(0)), int(self._x3.size(2))
            self._batch, self._K = batch, K
            self._y = torch.empty((batch, int(rows), K), dtype=torch.float32, device=x.device)
            self._ws_bytes = int(core.boo_workspace_bytes(self._desc, 0, batch, K)) if self._y.numel() else 0
            self._ws = torch.empty(max(self._ws_bytes, 1), dtype=torch.uint8, device=x.device)
            self._timer = _Timer()
            torch.cuda.current_stream(x.device).synchronize()

    def _check_stream(self):
        if _stream_of(self._device) != self._stream:
            raise RuntimeError('BOOTimedSpMM must run on its construction stream')

    def _args(self):
        return (self._desc, 0, int(self._x3.data_ptr()), int(self._y.data_ptr()), self._batch, self._K,
                int(self._ws.data_ptr()), self._ws_bytes, self._stream)

    def run(self):
        with torch.cuda.device(self._device):
            self._check_stream()
            if self._y.numel():
                core.boo_matmul_gpu(*self._args())
        return self.output

    def timed_run(self) -> float:
        with torch.cuda.device(self._device):
            self._check_stream()
            if not self._y.numel():
                return 0.0
            return float(core.boo_matmul_gpu_timed(*self._args(), self._timer.handle))

    @property
    def output(self):
        return self._y.squeeze(0) if self._squeeze else self._y

    def info(self) -> dict:
        return {'diagnostic': self._diag, 'row_seg': self._row_seg, 'nnzflat_fpt': self._fpt,
                'nnzflat_reference': self._ref}


class PBRTimedSpMM:
    """Y = A X for a PBR matrix given as the reference's CUDA metadata
    tensors, int32/fp32 only (bindings/bindings_pbr_timed.cu:90-140).  Every
    ``kernel`` selector is served by the stripe kernel; ``csr_mode`` and
    ``smem_size`` are accepted as the reference does.  ``diagnostic_raw_store``
    has no counterpart here and is refused."""

    _KERNELS = ('block', 'chunkcols', 'nnzflat', 'nnzflat_shared', 'nnzflat_onthefly')

    def __init__(self, cols, rows, block_rows, block_cols, block_codes, block_coords, block_offsets,
                 block_data, rem_indptr, rem_col_ind, rem_vals, x, csr_mode=0, smem_size=2048,
                 diagnostic_raw_store=False, kernel='block'):
        if kernel not in self._KERNELS:
            raise RuntimeError(f'unsupported PBR kernel selector: {kernel}')
        if diagnostic_raw_store and kernel != 'block':
            raise RuntimeError('diagnostic_raw_store is available only with kernel=block')
        if not x.is_cuda or x.dtype != torch.float32:
            raise RuntimeError('PBRTimedSpMM: X must be a CUDA FP32 tensor')
        if x.dim() not in (2, 3):
            raise RuntimeError('PBRTimedSpMM: X must be 2D or 3D')
        x3 = x.unsqueeze(0) if x.dim() == 2 else x
        if not x3.is_contiguous():
            raise RuntimeError('PBRTimedSpMM: X must be contiguous')
        arrays = (block_codes, block_coords, block_offsets, block_data, rem_indptr, rem_col_ind, rem_vals)
        for t in arrays:
            if t.device != x.device or not t.is_contiguous():
                raise RuntimeError("PBRTimedSpMM: PBR metadata must be contiguous tensors on X's device")
        if block_coords.dtype != torch.int32 or block_offsets.dtype != torch.int32:
            raise RuntimeError('PBRTimedSpMM: block_coords/block_offsets must be int32 '
                               '(this harness is int32/fp32 only)')
        if block_data.dtype != torch.float32 or rem_vals.dtype != torch.float32:
            raise RuntimeError('PBRTimedSpMM: block_data/rem_vals must be fp32')
        if diagnostic_raw_store:
            raise RuntimeError('PBRTimedSpMM: diagnostic_raw_store has no gfx950 kernel '
                               '(the stripe kernel stores every output row once)')
        if int(x3.size(1)) != int(cols):
            raise RuntimeError(f'PBRTimedSpMM: X has {int(x3.size(1))} rows, expected {int(cols)}')

        self._device = x.device
        self._squeeze = x.dim() == 2
        with torch.cuda.device(x.device):
            self._stream = _stream_of(x.device)
            self._x3 = x3
            meta = type('PbrMeta', (), {})()
            (meta.codes, meta.coords, meta.offsets, meta.data, meta.rem_indptr, meta.rem_col_ind,
             meta.rem_vals) = arrays
            self._meta = meta
            self._stripe_ptr, self._long_rows, self._desc = _pbr._kernel_staging(
                int(rows), int(cols), int(block_rows), int(block_cols), block_coords.cpu().numpy(),
                rem_indptr.cpu().numpy(), meta, x.device)
            self._batch, self._K = int(x3.size(0)), int(x3.size(2))
            self._y = torch.empty((self._batch, int(rows), self._K), dtype=torch.float32, device=x.device)
            self._timer = _Timer()
            torch.cuda.current_stream(x.device).synchronize()

    def _check_stream(self):
        if _stream_of(self._device) != self._stream:
            raise RuntimeError('PBRTimedSpMM must run on its construction stream')

    def _args(self):
        return (self._desc, 0, int(self._x3.data_ptr()), int(self._y.data_ptr()), self._batch, self._K,
                self._stream)

    def run(self):
        with torch.cuda.device(self._device):
            self._check_stream()
            if self._y.numel():
                core.pbr_matmul_gpu(*self._args())
        return self.output

    def timed_run(self) -> float:
        with torch.cuda.device(self._device):
            self._check_stream()
            if not self._y.numel():
                return 0.0
            return float(core.pbr_matmul_gpu_timed(*self._args(), self._timer.handle))

    @property
    def output(self):
        return self._y.squeeze(0) if self._squeeze else self._y

    def info(self) -> dict:
        return {'diagnostic': False}


# the reference's cuSPARSE names, then rocSPARSE's own (spmm_vendor_alg)
_VENDOR_ALGS = {
    'DEFAULT': 0, 'CSR_ALG1': 1, 'CSR_ALG2': 2, 'CSR_ALG3': 3,
    'default': 0, 'csr': 1, 'csr_row_split': 2, 'csr_nnz_split': 3, 'csr_merge': 3,
    'csr_merge_path': 4,
}


class DirectSpMM:
    """A persistent vendor SpMM plan over an fp32/int32 CSR matrix on X's
    device, beta = 0 (bindings/bindings_cusparse.cu:21-160), on rocSPARSE's
    generic SpMM.  ``algorithm`` takes the reference's names (``DEFAULT``,
    ``CSR_ALG1``-``3``, mapped to rocSPARSE's default, csr, csr_row_split and
    csr_nnz_split) or rocSPARSE's own.  ``run`` returns the persistent output,
    which the next run overwrites."""

    def __init__(self, crow, col, val, x, algorithm='DEFAULT'):
        if not (x.is_cuda and x.dim() == 2 and x.is_contiguous() and x.dtype == torch.float32):
            raise RuntimeError('X must be contiguous CUDA FP32, two-dimensional')
        for t in (crow, col, val):
            if t.device != x.device or t.dim() != 1 or not t.is_contiguous():
                raise RuntimeError("CSR arrays must be contiguous 1D tensors on X's device")
        if crow.dtype != torch.int32 or col.dtype != torch.int32 or val.dtype != torch.float32:
            raise RuntimeError('CSR must use int32 indices and FP32 values')
        if crow.numel() < 1 or col.numel() != val.numel():
            raise RuntimeError('Invalid CSR dimensions')
        if algorithm not in _VENDOR_ALGS:
            raise RuntimeError(f'Unknown SpMM algorithm: {algorithm}')
        self._device = x.device
        self._keep = (crow, col, val, x)
        self._plan = 0
        with torch.cuda.device(x.device):
            self._stream = _stream_of(x.device)
            rows = int(crow.numel()) - 1
            self._y = torch.empty((rows, int(x.size(1))), dtype=torch.float32, device=x.device)
            self._plan = int(core.vendor_create(rows, int(x.size(0)), int(val.numel()), int(crow.data_ptr()),
                                                int(col.data_ptr()), int(val.data_ptr()), int(x.data_ptr()),
                                                int(x.size(1)), int(self._y.data_ptr()),
                                                _VENDOR_ALGS[algorithm], self._stream))
            inf = core.vendor_info(self._plan)
            self._reason = '' if inf['supported'] else 'rocSPARSE: SpMM not implemented at buffer size'
            self._ws = None
            if inf['supported']:
                self._ws = torch.empty(max(int(inf['workspace_bytes']), 1), dtype=torch.uint8, device=x.device)
                core.vendor_preprocess(self._plan, int(self._ws.data_ptr()), int(inf['workspace_bytes']))
            self._timer = _Timer()

    def __del__(self):
        plan, self._plan = getattr(self, '_plan', 0), 0
        if plan:
            core.vendor_destroy(plan)

    def _check(self):
        if self._reason:
            raise RuntimeError(self._reason)
        if _stream_of(self._device) != self._stream:
            raise RuntimeError('DirectSpMM must run on its construction stream')

    def run(self):
        with torch.cuda.device(self._device):
            self._check()
            core.vendor_run(self._plan, self._stream)
        return self._y

    def timed_run(self) -> float:
        with torch.cuda.device(self._device):
            self._check()
            return float(core.vendor_run_timed(self._plan, self._stream, self._timer.handle))

    @property
    def output(self):
        return self._y

    def info(self) -> dict:
        inf = core.vendor_info(self._plan)
        return {'rocsparse_version': inf['version'], 'rocsparse_header_version': inf['header_version'],
                'workspace_bytes': inf['workspace_bytes'], 'preprocess_status': inf['preprocess_status'],
                'supported': inf['supported'], 'unsupported_reason': self._reason}
