"""Measurement adjuncts on the GPU (bindings/bindings_boo_timed.cu,
bindings/bindings_pbr_timed.cu, bindings/bindings_cusparse.cu): the timed
harnesses give the product's result, time one call, and keep to their
construction stream; the vendor plan's output is within the fp32 bound of the
fp64 product.  Mirrors the reference's tests/torch_fast_spdmm/
test_timed_variants.py (four dense 32x32 diagonal tiles plus an off-diagonal
entry), with a stencil and a tail-policy matrix added."""

import math

import numpy as np
import pytest
import scipy.sparse as sp
import torch

import spmm_amd as S
from oracle import oracle as O
from spmm_amd import matrices as M

pytestmark = pytest.mark.gpu


def _tiles():
    blocks = sp.block_diag([np.ones((32, 32), np.float32) for _ in range(4)], format='lil')
    blocks[0, 96] = 1
    return blocks.tocsr()


def _x(n, K, seed, batch=None):
    shape = (n, K) if batch is None else (batch, n, K)
    return torch.from_numpy(np.random.default_rng(seed).standard_normal(shape, dtype=np.float32)).cuda()


def _boo_timed(boo, x, **kw):
    m = boo._gpu_meta
    return S.BOOTimedSpMM(boo.rows, boo.cols, boo.max_nr, boo.max_nc, boo.max_nnz_blk,
                          m.row_grp_ptr, m.row_ids, m.col_grp_ptr, m.col_ids, m.blk_row_grp,
                          m.blk_col_grp, m.blk_nz_ptr, m.blk_shift, m.nz_idx, m.nz_val,
                          m.rem_indptr, m.rem_col_ind, m.rem_vals, m.tail_row, m.tail_col,
                          m.tail_val, x, **kw)


def _pbr_timed(pbr, x, **kw):
    m = pbr._gpu_meta
    return S.PBRTimedSpMM(pbr.cols, pbr.rows, pbr.block_rows, pbr.block_cols, m.codes, m.coords,
                          m.offsets, m.data, m.rem_indptr, m.rem_col_ind, m.rem_vals, x, **kw)


BOO_CASES = [
    ('tiles', lambda: _tiles(), dict(cluster='hem', small_block_policy='keep')),
    ('stencil', lambda: M.stencil_27pt(8), dict(cluster='identity')),
    ('tail', lambda: M.stencil_27pt(16), dict(cluster='identity', small_block_policy='tail_batch',
                                               small_block_threshold=64)),
    ('colmajor', lambda: M.stencil_27pt(8), dict(cluster='identity', nz_order='colmajor')),
]


@pytest.mark.parametrize('name, make, kw', BOO_CASES, ids=[c[0] for c in BOO_CASES])
@pytest.mark.parametrize('batch', [None, 2])
def test_boo_timed_matches_boo_matmul(name, make, kw, batch):
    A = make()
    boo = S.csr_to_boo(A, target_nr=32, target_nc=32, **kw).to('cuda')
    x = _x(A.shape[1], 64, 2, batch)
    row_seg = boo.nz_order == S.boo.BooNzOrder.ROWMAJOR
    timed = _boo_timed(boo, x, row_seg=row_seg)
    y = timed.run()
    expected = S.boo_matmul(boo, x, row_seg=row_seg)
    assert y.shape == expected.shape
    assert torch.equal(y, expected)   # same kernels, same schedule
    xs = x if batch else x.unsqueeze(0)
    for b in range(xs.size(0)):
        ratio, ok = O.within_bound((y if batch else y.unsqueeze(0))[b].cpu().numpy(), A, xs[b].cpu().numpy(),
                                   1e-5)
        assert ok, ratio
    ms = timed.timed_run()
    assert math.isfinite(ms) and ms > 0
    assert torch.equal(timed.output, expected)
    assert timed.info() == {'diagnostic': False, 'row_seg': row_seg, 'nnzflat_fpt': 1,
                            'nnzflat_reference': True}


def test_boo_timed_stream_and_diagnostic():
    A = M.stencil_27pt(8)
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32).to('cuda')
    x = _x(A.shape[1], 32, 3)
    with pytest.raises(RuntimeError, match='diagnostic_raw_store has no gfx950 kernel'):
        _boo_timed(boo, x, diagnostic_raw_store=True)
    timed = _boo_timed(boo, x)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        with pytest.raises(RuntimeError, match='must run on its construction stream'):
            timed.run()
        with pytest.raises(RuntimeError, match='must run on its construction stream'):
            timed.timed_run()
    torch.cuda.synchronize()
    assert torch.equal(timed.run(), S.boo_matmul(boo, x))


PBR_CASES = [
    ('tiles', lambda: _tiles(), 4),
    ('stencil', lambda: M.stencil_27pt(8), 4),
    ('sparse_blocks', lambda: sp.random(200, 300, density=0.05, format='csr', dtype=np.float32,
                                        random_state=np.random.default_rng(5)), 2),
]


@pytest.mark.parametrize('name, make, thr', PBR_CASES, ids=[c[0] for c in PBR_CASES])
@pytest.mark.parametrize('kernel', ['block', 'nnzflat'])
def test_pbr_timed_matches_pbr_matmul(name, make, thr, kernel):
    A = make()
    pbr = S.csr_to_pbr(A, 8, 8, thr).to('cuda')
    x = _x(A.shape[1], 128, 1)
    timed = _pbr_timed(pbr, x, kernel=kernel)
    y = timed.run()
    expected = S.pbr_matmul(pbr, x, kernel=kernel)
    assert torch.equal(y, expected)
    ratio, ok = O.within_bound(y.cpu().numpy(), A, x.cpu().numpy(), 1e-5)
    assert ok, ratio
    ms = timed.timed_run()
    assert math.isfinite(ms) and ms > 0
    assert timed.info() == {'diagnostic': False}


def _csr_cuda(A):
    A = sp.csr_matrix(A)
    return (torch.from_numpy(A.indptr.astype(np.int32)).cuda(),
            torch.from_numpy(A.indices.astype(np.int32)).cuda(),
            torch.from_numpy(A.data.astype(np.float32)).cuda())


@pytest.mark.parametrize('alg', ['DEFAULT', 'CSR_ALG1', 'CSR_ALG2', 'CSR_ALG3', 'csr_merge_path'])
def test_direct_spmm_vendor_plan(alg):
    A = M.stencil_27pt(8)
    x = _x(A.shape[1], 64, 4)
    crow, col, val = _csr_cuda(A)
    plan = S.DirectSpMM(crow, col, val, x, alg)
    info = plan.info()
    assert set(info) == {'rocsparse_version', 'rocsparse_header_version', 'workspace_bytes',
                         'preprocess_status', 'supported', 'unsupported_reason'}
    if not info['supported']:
        with pytest.raises(RuntimeError, match='not implemented'):
            plan.run()
        return
    assert info['preprocess_status'] == 0
    y = plan.run()
    assert y.data_ptr() == plan.output.data_ptr()
    ratio, ok = O.within_bound(y.cpu().numpy(), A, x.cpu().numpy(), 1e-5)
    assert ok, ratio
    ms = plan.timed_run()
    assert math.isfinite(ms) and ms > 0
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        with pytest.raises(RuntimeError, match='DirectSpMM must run on its construction stream'):
            plan.run()
    torch.cuda.synchronize()


def test_direct_spmm_rejects_bad_csr():
    x = _x(8, 4, 0)
    crow = torch.zeros(9, dtype=torch.int32, device='cuda')
    with pytest.raises(RuntimeError, match='int32 indices and FP32 values'):
        S.DirectSpMM(crow.long(), crow[:0], torch.zeros(0, device='cuda'), x)
    with pytest.raises(RuntimeError, match='Invalid CSR dimensions'):
        S.DirectSpMM(crow, crow[:1], torch.zeros(0, device='cuda'), x)
    with pytest.raises(RuntimeError, match='Unknown SpMM algorithm'):
        S.DirectSpMM(crow, crow[:0], torch.zeros(0, device='cuda'), x, 'CSR_ALG9')
