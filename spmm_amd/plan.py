"""Execution plans for ``boo_matmul`` (API of the reference's ``boo_plan.py``).

The reference prepares size-bucketed launches and row-start tables to work
around CUDA's grid-wide dynamic shared memory (torch_fast_spdmm/boo_plan.py:
84-123).  The gfx950 kernel needs neither: its LDS is sized per workgroup and
its work schedule is built once at ``.to('cuda')``.  A plan here therefore
records that staging and is accepted by ``boo_matmul(..., launch_mode='auto',
execution_plan=plan)`` with the same validation as the reference; it adds no
device memory and changes nothing in the launch.
"""

from __future__ import annotations

import time
from dataclasses import dataclass

import torch

__all__ = ['BOOExecutionPlan', 'prepare_boo_cuda']


@dataclass(frozen=True)
class BOOExecutionPlan:
    matrix: object
    source_meta: object
    meta: object
    buckets: tuple
    row_ptr: torch.Tensor
    row_starts: torch.Tensor
    p: int
    bucketed: bool
    precomputed_rows: bool
    build_ms: float
    staging_ms: float
    extra_device_bytes: int


def prepare_boo_cuda(boo, *, bucketed=False, precomputed_rows=False, p=64):
    source = getattr(boo, '_gpu_meta', None)
    if source is None:
        raise ValueError("Call boo.to('cuda') before preparing an execution plan")
    if int(boo.nz_order) != 0:
        raise ValueError('BOO execution plans require rowmajor nonzeros')
    if p not in (8, 16, 32, 64, 128):
        raise ValueError('p must be one of 8, 16, 32, 64, 128')
    start = time.perf_counter()
    count = boo.num_blocks()
    buckets = (0, count, int(boo.max_nr), int(boo.max_nc), int(boo.max_nnz_blk)) if count else ()
    empty = torch.empty(0, dtype=torch.int32, device=source.nz_val.device)
    build_ms = (time.perf_counter() - start) * 1000
    return BOOExecutionPlan(boo, source, source, buckets, empty, empty, p, bool(bucketed),
                            bool(precomputed_rows), build_ms, 0.0, 0)
