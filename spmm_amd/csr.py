"""Naive CSR SpMM baseline on the GPU (``spdmm_csr_naive``).

Semantics of the reference's ``spdmm_csr_naive`` (kernels/csr_kernels.cu:31-53):
a CUDA sparse CSR matrix ``A`` [rows, cols] times a dense ``x`` [cols, K],
float32/float64 values with int32/int64 indices, one thread per output
element summing its row in CSR order, plain stores into a fresh Y.
"""

from __future__ import annotations

import torch

from ._native import core

__all__ = ['spdmm_csr_naive']

_DTYPE_CODE = {torch.float32: 0, torch.float64: 1}
_ITYPE_CODE = {torch.int32: 0, torch.int64: 1}


def spdmm_csr_naive(A: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    if A.layout != torch.sparse_csr or A.dim() != 2:
        raise ValueError('A must be a 2D sparse CSR tensor')
    if not A.is_cuda or not x.is_cuda or A.device != x.device:
        raise ValueError('A and x must be CUDA tensors on the same device')
    if x.dim() != 2 or x.size(0) != A.size(1):
        raise ValueError(f'x must be [{A.size(1)}, K], got {tuple(x.shape)}')
    vals, cols, crow = A.values(), A.col_indices(), A.crow_indices()
    if vals.dtype not in _DTYPE_CODE or x.dtype != vals.dtype:
        raise TypeError(f'A and x must share a float32/float64 dtype, got {vals.dtype}/{x.dtype}')
    if cols.dtype not in _ITYPE_CODE or crow.dtype != cols.dtype:
        raise TypeError('A indices must be int32 or int64')
    rows, K = int(A.size(0)), int(x.size(1))
    with torch.cuda.device(x.device):
        xc = x.contiguous()
        crow, cols, vals = crow.contiguous(), cols.contiguous(), vals.contiguous()
        y = torch.empty((rows, K), dtype=x.dtype, device=x.device)
        if y.numel():
            stream = torch.cuda.current_stream(x.device).cuda_stream
            core.csr_naive_gpu(int(crow.data_ptr()), int(cols.data_ptr()), int(vals.data_ptr()),
                               _ITYPE_CODE[cols.dtype], _DTYPE_CODE[x.dtype], rows, int(A.size(1)),
                               int(xc.data_ptr()), int(y.data_ptr()), K, int(stream))
    return y
