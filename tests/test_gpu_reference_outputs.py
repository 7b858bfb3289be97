"""GPU results against the reference's own outputs on the same inputs.

Every committed fixture (tests/golden/*.npz) holds the reference's encoding
of a matrix, an X and the reference CPU op's Y for that X
(boo_batched_matmul_cpu / pbr_batched_matmul_cpu, boo_matrix.cpp:336-396,
pbr_matrix.cpp:17-68, written by tests/golden/make_fixtures.py from the
reference compiled here).  The product builds the same matrix, runs it on
the GPU with that X and must match the reference's Y elementwise within
1e-5 * (|A|.|X|) (float64: 1e-12), the north star's bar for fp32 summation
order.  BOO runs through each of its GPU paths: the LDS-DMA tile stream,
the record-stream kernel and the row-wise gather pass."""

import numpy as np
import pytest
import torch

import spmm_amd as S
import spmm_amd.boo as SB
from conftest import csr_of, fixture_names, load_fixture
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _check(y, fx, A):
    ref = fx['y_cpu'][0].astype(np.float64)
    _, bound = O.spmm_reference(A, fx['x'])
    rel = 1e-5 if fx['x'].dtype == np.float32 else 1e-12
    err = np.abs(np.asarray(y, dtype=np.float64) - ref)
    ok = err <= rel * bound
    assert ok.all(), f'max |y - y_ref| / bound = {np.max(err / np.maximum(bound, 1e-300)):.3e}'


@pytest.mark.parametrize('path', ['tile', 'record', 'gather'])
@pytest.mark.parametrize('name', fixture_names('boo_'))
def test_boo_matches_reference_output(name, path, monkeypatch):
    fx = load_fixture(name)
    pol, thr, order = (int(v) for v in fx['params'])
    monkeypatch.setattr(SB, 'MIN_COL_REUSE', 1e9 if path == 'gather' else (0.0 if path == 'tile' else 1.5))
    monkeypatch.setattr(SB, 'RECORD_STREAM', path == 'record')
    A = csr_of(fx)
    b = S.csr_to_boo(A, row_labels=fx['row_labels'], col_labels=fx['col_labels'],
                     small_block_policy=['keep', 'merge', 'remainder', 'tail_batch'][pol],
                     small_block_threshold=thr, nz_order=['rowmajor', 'colmajor'][order]).to('cuda')
    if path == 'record' and A.dtype == np.float32 and A.shape[0] >= 32:
        d = b._gpu_meta.desc
        assert d['n_blob16'] > 0 or d['n_tiles'] == 0
    y = S.boo_matmul(b, torch.from_numpy(fx['x']).cuda())
    torch.cuda.synchronize()
    _check(y.cpu().numpy(), fx, A)


@pytest.mark.parametrize('name', fixture_names('pbr_'))
def test_pbr_matches_reference_output(name):
    fx = load_fixture(name)
    br, bc, thr = (int(v) for v in fx['params'])
    A = csr_of(fx)
    p = S.csr_to_pbr(A, br, bc, thr).to('cuda')
    y = S.pbr_matmul(p, torch.from_numpy(fx['x']).cuda())
    torch.cuda.synchronize()
    _check(y.cpu().numpy(), fx, A)
