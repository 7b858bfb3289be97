"""Parity at BASELINE.json's full sizes for configs 3, 4 and 5.

Configs 1 and 2 are checked in test_gpu_boo.py and test_gpu_pbr_csr.py.
These three are 33-56 M nonzeros; every row of Y is compared with the
oracle's fp64 product, computed in row blocks so the host's memory stays
bounded: |Y - AX| <= 1e-5 (|A||X|) elementwise (the tolerance of the path).
A second call must give bit-equal results (plain stores, no atomics).

The matrices are the bench's own (spmm_amd/matrices.py, seeded).
"""

import functools

import numpy as np
import pytest
import scipy.sparse as sp
import torch

import spmm_amd as S
from spmm_amd import matrices as M

pytestmark = pytest.mark.gpu

TOL = 1e-5
BLOCK = 1 << 17     # rows per block of the fp64 product


@functools.lru_cache(maxsize=1)
def _config(cfg):
    A, spec = M.make_config(cfg)
    x = M.dense_x(A.shape[1], spec['K'])
    return A, spec, x


def _check_full(y, A, x):
    """Every element of y against the fp64 product, block of rows by block."""
    x64 = x.astype(np.float64)
    absx = np.abs(x64)
    # private fp64 copies of A (the caller's arrays are not touched)
    A64 = sp.csr_matrix((A.data.astype(np.float64), A.indices.copy(), A.indptr.copy()), shape=A.shape)
    Aabs = sp.csr_matrix((np.abs(A64.data), A64.indices, A64.indptr), shape=A.shape)
    yh = y.cpu().numpy()
    worst = 0.0
    for r0 in range(0, A.shape[0], BLOCK):
        r1 = min(A.shape[0], r0 + BLOCK)
        ref = A64[r0:r1] @ x64
        bound = Aabs[r0:r1] @ absx
        err = np.abs(yh[r0:r1].astype(np.float64) - ref)
        bad = err > TOL * bound
        if bad.any():
            r, f = np.argwhere(bad)[0]
            raise AssertionError(f'row {r0 + r} feature {f}: |err| {err[r, f]:.3e} > {TOL} x {bound[r, f]:.3e}')
        with np.errstate(divide='ignore', invalid='ignore'):
            q = np.where(bound > 0, err / np.where(bound > 0, bound, 1), 0.0)
        worst = max(worst, float(q.max()) if q.size else 0.0)
    print(f'  every row within the bound; max |err| / (|A||X|) = {worst:.3e}', flush=True)


# generating a config takes up to ~80 s on the host, the fp64 check ~15 s
@pytest.mark.timeout(480)
@pytest.mark.parametrize('cfg,fmt', [(3, 'pbr'), (4, 'boo'), (5, 'boo'), (5, 'pbr')])
def test_full_size_config(cfg, fmt):
    print(f'config {cfg} {fmt}: generating', flush=True)
    A, spec, x_np = _config(cfg)
    print(f'config {cfg} {fmt}: {A.shape} nnz={A.nnz} K={spec["K"]}', flush=True)
    if fmt == 'boo':
        mat = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32).to('cuda')
        run = S.boo_matmul
    else:
        mat = S.csr_to_pbr(A, 8, 8, spec.get('pbr_threshold', 4)).to('cuda')
        run = S.pbr_matmul
    x = torch.from_numpy(x_np).cuda()
    y = run(mat, x)
    torch.cuda.synchronize()
    assert y.shape == (A.shape[0], spec['K']) and y.dtype == torch.float32
    _check_full(y, A, x_np)
    assert torch.equal(run(mat, x), y)
