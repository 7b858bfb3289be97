"""PBR and the naive CSR baseline on the GPU against the oracle's fp64 bound
(tests/torch_fast_spdmm/test_pbr.py, test_csr.py of the reference)."""

import numpy as np
import pytest
import scipy.sparse as sp
import torch

import spmm_amd as S
import spmm_amd.pbr as SP
from conftest import csr_of, fixture_names, load_fixture
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True, params=['auto', 'stripe'])
def pbr_route(request, monkeypatch):
    """Run every PBR case twice: with the default route (a matrix whose
    blocks hold few of its entries runs its CSR through the BOO gather pass)
    and with the stripe kernel forced for every matrix."""
    if request.param == 'stripe':
        if 'pbr' not in request.node.name:
            pytest.skip('the route applies to PBR only')
        monkeypatch.setattr(SP, 'GATHER_MAX_BLOCK_SHARE', 0.0)
    return request.param


def check(y, A, x):
    tol = 1e-5 if y.dtype == torch.float32 else 1e-12
    ratio, ok = O.within_bound(y.detach().cpu().numpy(), A, x.detach().cpu().numpy(), tol)
    assert ok, f'max |err|/(|A||X|) = {ratio:.3e}'


def _mats(n, dtype, seed=0):
    rng = np.random.default_rng(seed)
    eye = sp.eye(n, dtype=dtype, format='csr')
    perm = sp.csr_matrix((np.ones(n, dtype), (np.arange(n), rng.permutation(n))), shape=(n, n))
    dense = sp.random(n, n, density=0.9, format='csr', dtype=dtype, random_state=seed)
    return {'identity': eye, 'permutation': perm, 'low_sparsity': dense}


@pytest.mark.parametrize('kind', ['identity', 'permutation', 'low_sparsity'])
@pytest.mark.parametrize('index_dtype', [np.int32, np.int64])
@pytest.mark.parametrize('data_dtype', [np.float32, np.float64])
@pytest.mark.parametrize('n', [8, 16])
@pytest.mark.parametrize('block_size', [4, 8])
@pytest.mark.parametrize('features', [8, 32])
@pytest.mark.parametrize('min_nnz', [1, 64])
def test_pbr_batched_matmul_direct(kind, index_dtype, data_dtype, n, block_size, features, min_nnz):
    m = _mats(n, data_dtype)[kind]
    m.indptr, m.indices = m.indptr.astype(index_dtype), m.indices.astype(index_dtype)
    p = S.csr_to_pbr(m, block_size, block_size, min_nnz).to('cuda')
    meta = p._gpu_meta
    assert meta.coords.dtype == (torch.int32 if index_dtype == np.int32 else torch.int64)
    assert meta.codes.dtype == torch.int64
    tdt = torch.float32 if data_dtype == np.float32 else torch.float64
    x = torch.randn((1, n, features), dtype=tdt, device='cuda')
    y = S.pbr_batched_matmul_cuda(p, x)
    assert y.shape == (1, n, features)
    check(y, m, x)


@pytest.mark.parametrize('rows', [9, 13, 1001])
@pytest.mark.parametrize('min_nnz', [1, 4, 64])
def test_pbr_partial_last_stripe(rows, min_nnz):
    rng = np.random.default_rng(0)
    mat = sp.random(rows, rows, density=0.3, format='lil', dtype=np.float32, random_state=rng)
    mat[rows - 1, rng.integers(0, rows, size=min(3, rows))] = 1.0
    mat = mat.tocsr()
    mat.sort_indices()
    p = S.csr_to_pbr(mat, 8, 8, min_nnz).to('cuda')
    x = torch.randn((1, rows, 32), device='cuda')
    check(S.pbr_batched_matmul_cuda(p, x), mat, x)


@pytest.mark.parametrize('name', fixture_names('pbr_'))
@pytest.mark.parametrize('K', [1, 5, 64, 100, 256, 300])
def test_pbr_reference_fixtures(name, K):
    """The reference's exact encodings (block order included) through the GPU."""
    fx = load_fixture(name)
    br, bc, thr = (int(v) for v in fx['params'])
    m = csr_of(fx)
    p = S.csr_to_pbr(m, br, bc, thr).to('cuda')
    tdt = torch.float32 if m.dtype == np.float32 else torch.float64
    x = torch.randn((2, m.shape[1], K), dtype=tdt, device='cuda')
    check(S.pbr_matmul(p, x), m, x)


def test_pbr_long_remainder_rows(monkeypatch):
    monkeypatch.setattr(SP, 'LONG_ROW_THRESHOLD', 4)
    A = sp.random(500, 700, density=0.2, format='csr', random_state=3, dtype=np.float32)
    p = S.csr_to_pbr(A, 8, 8, 20).to('cuda')
    assert p._gpu_meta.desc['n_long'] > 0
    for K in (96, 7):
        x = torch.randn(700, K, device='cuda')
        check(S.pbr_matmul(p, x), A, x)


@pytest.mark.parametrize('kernel', ['block', 'chunkcols', 'nnzflat', 'nnzflat_shared', 'nnzflat_onthefly'])
def test_pbr_kernel_names_row_skewed(kernel):
    """row_skewed pattern: one dense row plus one entry per other row."""
    n = 256
    rows = np.r_[np.zeros(n, int), np.arange(1, n)]
    cols = np.r_[np.arange(n), (np.arange(1, n) * 7) % n]
    A = sp.csr_matrix((np.random.default_rng(0).standard_normal(rows.size).astype(np.float32),
                       (rows, cols)), shape=(n, n))
    p = S.csr_to_pbr(A, 8, 8, 1).to('cuda')
    x = torch.randn(n, 64, device='cuda')
    check(S.pbr_matmul(p, x, kernel=kernel), A, x)


def test_pbr_and_boo_agree():
    """test_boo.py:298-310: BOO vs the PBR block kernel on the same matrix."""
    m = sp.random(256, 256, density=0.04, format='csr', random_state=0, dtype=np.float32)
    pbr = S.csr_to_pbr(m, 8, 8, 1).to('cuda')
    boo = S.csr_to_boo(m, cluster='identity', target_nr=16, target_nc=16,
                       small_block_threshold=6).to('cuda')
    x = torch.randn(256, 64, device='cuda')
    torch.testing.assert_close(S.boo_matmul(boo, x), S.pbr_matmul(pbr, x), rtol=1e-5, atol=1e-5)


def test_pbr_config2_full_size():
    from spmm_amd import matrices as M
    A, spec = M.make_config(2)
    p = S.csr_to_pbr(A, 8, 8, 4).to('cuda')
    x = torch.from_numpy(M.dense_x(A.shape[1], spec['K'])).cuda()
    y = S.pbr_matmul(p, x)
    check(y, A, x)
    assert torch.equal(S.pbr_matmul(p, x), y)


def test_pbr_cuda_errors():
    m = sp.random(16, 16, density=0.3, format='csr', random_state=0, dtype=np.float32)
    p = S.csr_to_pbr(m)
    with pytest.raises(RuntimeError, match='to\\(.cuda.\\)'):
        S.pbr_matmul(p, torch.zeros(16, 4, device='cuda'))
    p.to('cuda')
    with pytest.raises(ValueError, match='2D or 3D'):
        S.pbr_matmul(p, torch.zeros(16, device='cuda'))
    q = S.csr_to_pbr(m, 3, 3, 1).to('cuda')
    with pytest.raises(ValueError, match='Unsupported block size'):
        S.pbr_matmul(q, torch.zeros(16, 4, device='cuda'))


# ---------------------------------------------------------------- naive CSR
def _laplacian(n, dtype):
    from spmm_amd import matrices as M
    return M.laplacian_2d(int(np.sqrt(n)), dtype=dtype)


@pytest.mark.parametrize('index_dtype', [torch.int32, torch.int64])
@pytest.mark.parametrize('data_dtype', [torch.float32, torch.float64])
@pytest.mark.parametrize('kind', ['eye', 'laplacian'])
@pytest.mark.parametrize('n', [64, 256])
@pytest.mark.parametrize('features', [16, 32, 64, 128, 256, 512])
def test_csr_naive(index_dtype, data_dtype, kind, n, features):
    npdt = np.float32 if data_dtype == torch.float32 else np.float64
    A = sp.eye(n, dtype=npdt, format='csr') if kind == 'eye' else _laplacian(n, npdt)
    t = torch.sparse_csr_tensor(torch.from_numpy(A.indptr.astype(np.int64)).to(index_dtype),
                                torch.from_numpy(A.indices.astype(np.int64)).to(index_dtype),
                                torch.from_numpy(A.data), size=A.shape).cuda()
    x = torch.randn(n, features, dtype=data_dtype, device='cuda')
    y = S.spdmm_csr_naive(t, x)
    check(y, A, x)
    torch.testing.assert_close(y.cpu(), torch.sparse.mm(t.cpu(), x.cpu()))


@pytest.mark.parametrize('dtype', [np.float32, np.float64])
def test_pbr_scattered_matrix_route(pbr_route, dtype):
    """A permuted 27-point stencil keeps 5 % of its entries in 8x8 blocks: by
    default its whole CSR runs through the BOO gather pass (launch_info names
    those kernels); an unpermuted one, 96 % in blocks, keeps the stripe
    kernel.  Both within the bound, batch 2."""
    from spmm_amd import matrices as M
    K = 32
    for A, scattered in ((M.permuted(M.stencil_27pt(16, dtype=dtype), seed=1), True),
                         (M.stencil_27pt(16, dtype=dtype), False)):
        p = S.csr_to_pbr(A, 8, 8, 4).to('cuda')
        gather = scattered and pbr_route == 'auto'
        assert (p._gpu_meta.gather is not None) == gather
        tdt = torch.float32 if dtype == np.float32 else torch.float64
        x = torch.randn((2, A.shape[1], K), dtype=tdt, device='cuda')
        y = S.pbr_matmul(p, x)
        for b in range(2):
            check(y[b], A, x[b])
        names = [k['kernel'] for k in S.pbr_launch_info(p, K, batch=2, x=x)]
        assert ('pbr_stripe_kernel' in names) == (not gather)
        if gather:
            assert 'boo_rows_kernel' in names
        assert torch.equal(S.pbr_matmul(p, x), y)
