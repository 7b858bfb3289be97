"""Parity at BASELINE.json's full sizes for configs 3, 4 and 5.

Configs 1 and 2 are checked against the whole fp64 product
(test_gpu_boo.py, test_gpu_pbr_csr.py).  These three are 33-56 M nonzeros,
so the host side keeps to checks that stay cheap at that size:

* 65,536 seeded rows (6-12 % of the rows, spread over the whole matrix)
  against the oracle's fp64 product, elementwise |Y - AX| <= 1e-5 (|A||X|)
  (the tolerance of the path): a wrong value in any sampled row fails;
* a column checksum over every row: sum_r Y[r, f] = ((1^T A) X)_f within
  1e-5 ((1^T |A|) |X|)_f, the sum of the elementwise bounds.  That bound is
  loose at this size: it catches gross errors anywhere (a pass that did not
  run, 1 % of the rows zeroed) but not one wrong row, which the sample is
  for;
* bit-equal results on a second call (plain stores, no atomics).

The matrices are the bench's own (spmm_amd/matrices.py, seeded).
"""

import functools

import numpy as np
import pytest
import torch

import spmm_amd as S
from oracle import oracle as O
from spmm_amd import matrices as M

pytestmark = pytest.mark.gpu

TOL = 1e-5
N_SAMPLE = 65536


@functools.lru_cache(maxsize=1)
def _config(cfg):
    A, spec = M.make_config(cfg)
    x = M.dense_x(A.shape[1], spec['K'])
    return A, spec, x


def _check_full(y, A, x):
    y64 = y.double()
    # column checksum over all rows
    ones = np.ones(A.shape[0])
    colsum = ones @ A                       # 1^T A, fp64 (A is scipy, fp32 values)
    abscolsum = ones @ abs(A)
    ref = torch.from_numpy(colsum.astype(np.float64) @ x.astype(np.float64))
    bound = torch.from_numpy(abscolsum.astype(np.float64) @ np.abs(x).astype(np.float64))
    got = y64.sum(0).cpu()
    assert torch.all((got - ref).abs() <= TOL * bound), \
        f'column checksum: max excess {((got - ref).abs() - TOL * bound).max().item():.3e}'
    # sampled rows against the fp64 product
    rows = np.sort(np.random.default_rng(7).choice(A.shape[0], N_SAMPLE, replace=False))
    ratio, ok = O.within_bound(y[torch.from_numpy(rows).cuda()].cpu().numpy(), A[rows], x, TOL)
    assert ok, f'sampled rows: max |err|/(|A||X|) = {ratio:.3e}'


@pytest.mark.parametrize('cfg,fmt', [(3, 'pbr'), (4, 'boo'), (5, 'boo'), (5, 'pbr')])
def test_full_size_config(cfg, fmt):
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
