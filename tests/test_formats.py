"""The product's host side against the oracle and the reference's outputs.

Bit-exact: every array of csr_to_boo / csr_to_pbr (PBR including its
in-stripe block order, against fixtures written by the compiled reference),
the decoders, and the CPU SpMM ops (which keep the reference's loop order).
"""

import numpy as np
import pytest
import scipy.sparse as sp
import torch

import spmm_amd as S
from conftest import csr_of, fixture_names, load_fixture
from oracle import oracle as O


def _arrays(obj, fields):
    return {f: np.asarray(getattr(obj, f)) for f in fields}


def _rand_csr(seed, rows, cols, density, dtype=np.float32, itype=np.int32):
    r = np.random.default_rng(seed)
    dense = r.normal(size=(rows, cols))
    dense[r.random((rows, cols)) > density] = 0
    m = sp.csr_matrix(dense.astype(dtype))
    m.indptr, m.indices = m.indptr.astype(itype), m.indices.astype(itype)
    return m


# ---------------------------------------------------------------- BOO builder
@pytest.mark.parametrize('name', fixture_names('boo_'))
def test_csr_to_boo_matches_reference_fixture(name):
    fx = load_fixture(name)
    pol, thr, order = (int(v) for v in fx['params'])
    b = S.csr_to_boo(csr_of(fx), row_labels=fx['row_labels'], col_labels=fx['col_labels'],
                     small_block_policy=['keep', 'merge', 'remainder', 'tail_batch'][pol],
                     small_block_threshold=thr, nz_order=['rowmajor', 'colmajor'][order])
    got = _arrays(b, O.BOO_FIELDS)
    for f in O.BOO_FIELDS:
        assert got[f].dtype == fx[f].dtype and np.array_equal(got[f], fx[f]), f
    assert [b.max_nr, b.max_nc, b.max_nnz_blk] == list(fx['maxima'])
    y = S.boo_matmul(b, torch.from_numpy(fx['x']))
    assert np.array_equal(y.numpy(), fx['y_cpu'][0])      # CPU op, bit for bit


@pytest.mark.parametrize('seed', range(8))
@pytest.mark.parametrize('policy', ['keep', 'remainder', 'tail_batch'])
@pytest.mark.parametrize('order', ['rowmajor', 'colmajor'])
def test_csr_to_boo_matches_oracle(seed, policy, order):
    dt = [np.float32, np.float64][seed % 2]
    it = [np.int32, np.int64][(seed // 2) % 2]
    r = np.random.default_rng(seed)
    rows, cols = int(r.integers(1, 150)), int(r.integers(1, 150))
    m = _rand_csr(seed, rows, cols, 0.05 + 0.03 * seed, dt, it)
    rl = r.integers(0, max(1, rows // 9), size=rows)
    cl = r.integers(0, max(1, cols // 11), size=cols)
    b = S.csr_to_boo(m, row_labels=rl, col_labels=cl, small_block_policy=policy,
                     small_block_threshold=int(r.integers(0, 6)) if policy != 'keep' else 4,
                     nz_order=order)
    thr = None
    # rebuild the oracle with the same threshold the product used
    pol = {'keep': 0, 'remainder': 2, 'tail_batch': 3}[policy]
    o = None
    for t in range(0, 6):
        cand = O.boo_build(m.indptr, m.indices, m.data, rows, cols, rl, cl, pol, t,
                           0 if order == 'rowmajor' else 1)
        if np.array_equal(cand['blk_nz_ptr'], np.asarray(b.blk_nz_ptr)):
            o, thr = cand, t
            break
    assert o is not None
    got = _arrays(b, O.BOO_FIELDS)
    for f in O.BOO_FIELDS:
        assert got[f].dtype == o[f].dtype and np.array_equal(got[f], o[f]), (f, thr)
    assert type(b).__name__ == f'BOOMatrixInt{np.dtype(it).itemsize * 8}' + \
        ('Float' if dt == np.float32 else 'Double')
    # decode and CPU op
    np.testing.assert_array_equal(S.boo_to_csr(b).toarray(), m.toarray())
    x = np.random.default_rng(seed + 50).standard_normal((2, cols, 7)).astype(dt)
    assert np.array_equal(S.boo_matmul(b, torch.from_numpy(x)).numpy(), O.boo_cpu_matmul(o, x))


def test_csr_to_boo_identity_full_config2():
    """Config 2 at full size: product arrays == oracle arrays."""
    from spmm_amd import matrices as M
    A = M.stencil_27pt(64)
    b = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32)
    rl = O.identity_labels(A.shape[0], 32)
    o = O.boo_build(A.indptr, A.indices, A.data, A.shape[0], A.shape[1], rl, rl, 2, 4, 0)
    got = _arrays(b, O.BOO_FIELDS)
    for f in O.BOO_FIELDS:
        assert np.array_equal(got[f], o[f]), f


def test_csr_to_boo_live_reference(ref_core):
    """Product == compiled reference on the 3-D stencil (smaller grid)."""
    from spmm_amd import matrices as M
    A = M.stencil_27pt(24)
    rl = O.identity_labels(A.shape[0], 32)
    for pol in (0, 2, 3):
        b = S.csr_to_boo(A, row_labels=rl, col_labels=rl,
                         small_block_policy=['keep', 'merge', 'remainder', 'tail_batch'][pol])
        r = ref_core.csr_to_boo(A.indptr, A.indices, A.data, A.shape[0], A.shape[1], rl, rl, pol, 4, 0)
        for f in O.BOO_FIELDS:
            assert np.array_equal(np.asarray(getattr(b, f)), np.asarray(getattr(r, f))), (pol, f)


def test_torch_csr_input_and_errors():
    m, rl, cl = _seven_by_eleven()
    t = torch.sparse_csr_tensor(torch.from_numpy(m.indptr), torch.from_numpy(m.indices),
                                torch.from_numpy(m.data), size=m.shape)
    b = S.csr_to_boo(t, row_labels=rl, col_labels=cl)
    np.testing.assert_array_equal(S.boo_to_csr(b).toarray(), m.toarray())
    with pytest.raises(TypeError, match='float32/float64'):
        S.csr_to_boo(m.astype(np.int32))
    with pytest.raises(ValueError, match='sparse CSR'):
        S.csr_to_boo(torch.zeros(7, 11))
    broken = m.copy()
    broken.indices[0] = 11
    with pytest.raises(ValueError):
        S.csr_to_boo(broken)
    with pytest.raises(Exception, match='merge'):
        S.csr_to_boo(m, row_labels=rl, col_labels=cl, small_block_policy='merge')


def _seven_by_eleven():
    ent = [(0, 0, 2), (0, 2, -1), (2, 6, 3), (2, 0, 1), (0, 1, 4), (1, 1, 2), (1, 4, -3),
           (4, 7, 1), (4, 9, 2), (4, 3, -2), (3, 5, 1)]
    r, c, v = zip(*ent)
    m = sp.csr_matrix((np.array(v, dtype=np.float32), (r, c)), shape=(7, 11))
    return m, np.array([0, 1, 0, 2, 1, 0, 2]), np.array([0, 1, 0, 2, 1, 2, 0, 1, 2, 1, 2])


@pytest.mark.parametrize('kwargs', [{'target_nr': 0}, {'max_nc': -1}, {'max_block_nnz': 0},
                                    {'small_block_threshold': -1}, {'nz_order': 'unknown'},
                                    {'small_block_policy': 'unknown'}])
def test_invalid_builder_parameters(kwargs):
    with pytest.raises(ValueError):
        S.csr_to_boo(_seven_by_eleven()[0], **kwargs)


@pytest.mark.parametrize('case', ['missing', 'length', 'rank', 'negative', 'too_large', 'float'])
def test_invalid_labels(case):
    m, rl, cl = _seven_by_eleven()
    if case == 'missing':
        cl = None
    elif case == 'length':
        rl = rl[:-1]
    elif case == 'rank':
        rl = rl.reshape(1, -1)
    elif case == 'negative':
        rl[0] = -1
    elif case == 'too_large':
        rl[0] = 2 ** 40
    else:
        rl = rl.astype(float) + 0.5
    with pytest.raises((ValueError, TypeError), match='labels'):
        S.csr_to_boo(m, row_labels=rl, col_labels=cl)


@pytest.mark.parametrize('shape', [(0, 0), (0, 5), (5, 0), (5, 7)])
@pytest.mark.parametrize('policy', ['keep', 'remainder', 'tail_batch'])
def test_empty_matrix_cpu(shape, policy):
    m = sp.csr_matrix(shape, dtype=np.float32)
    b = S.csr_to_boo(m, cluster='identity', small_block_policy=policy)
    assert b.num_blocks() == b.total_nnz == 0
    np.testing.assert_array_equal(S.boo_to_csr(b).toarray(), m.toarray())
    x = torch.randn(2, shape[1], 9)
    assert torch.equal(S.boo_matmul(b, x), torch.zeros(2, shape[0], 9))


def test_invalid_x_contract_cpu():
    m, rl, cl = _seven_by_eleven()
    b = S.csr_to_boo(m, row_labels=rl, col_labels=cl)
    for shape in [(11,), (1, 1, 11, 3)]:
        with pytest.raises(ValueError, match='2D or 3D'):
            S.boo_matmul(b, torch.zeros(shape))
    with pytest.raises(ValueError, match='rows'):
        S.boo_matmul(b, torch.zeros(10, 3))
    for dtype in (torch.float64, torch.float16, torch.int32, torch.complex64):
        with pytest.raises(TypeError, match='dtype'):
            S.boo_matmul(b, torch.zeros(11, 3, dtype=dtype))
    with pytest.raises(ValueError, match='dense'):
        S.boo_matmul(b, torch.zeros(11, 3).to_sparse())
    with pytest.raises(ValueError, match='launch_mode'):
        S.boo_matmul(b, torch.zeros(11, 3), launch_mode='bogus')


@pytest.mark.parametrize('layout', ['transpose', 'slice', 'expand', 'batch_transpose'])
def test_noncontiguous_x_cpu(layout):
    m, rl, cl = _seven_by_eleven()
    b = S.csr_to_boo(m, row_labels=rl, col_labels=cl, small_block_policy='remainder')
    g = torch.Generator().manual_seed(123)
    if layout == 'transpose':
        x = torch.randn(13, 11, generator=g).T
    elif layout == 'slice':
        x = torch.randn(11, 26, generator=g)[:, 1::2]
    elif layout == 'expand':
        x = torch.randn(11, 1, generator=g).expand(11, 13)
    else:
        x = torch.randn(3, 13, 11, generator=g).transpose(1, 2)
    saved = x.clone()
    ratio, ok = O.within_bound(S.boo_matmul(b, x).numpy(), m, x.numpy())
    assert ok, ratio
    assert torch.equal(x, saved)


def test_unsorted_duplicates_and_explicit_zeros_cpu():
    """test_boo_edges.py:251-259."""
    m = sp.csr_matrix((np.array([2., -2., 0., 3., 4.]), np.array([3, 3, 1, 0, 2]),
                       np.array([0, 4, 5, 5])), shape=(3, 5))
    assert not m.has_canonical_format
    for order in ('rowmajor', 'colmajor'):
        b = S.csr_to_boo(m, row_labels=np.zeros(3, int), col_labels=np.zeros(5, int),
                         small_block_policy='keep', nz_order=order)
        np.testing.assert_array_equal(S.boo_to_csr(b).toarray(), m.toarray())
        x = torch.randn(5, 17, dtype=torch.float64)
        np.testing.assert_allclose(S.boo_matmul(b, x).numpy(), m.toarray() @ x.numpy(), rtol=1e-10)


def test_boo_info_fields():
    m = sp.random(256, 256, density=0.05, format='csr', random_state=0, dtype=np.float32)
    b = S.csr_to_boo(m, cluster='identity', target_nr=16, target_nc=16, small_block_policy='keep')
    info = S.boo_info(b)
    assert info.compressed_fraction == 1.0 and info.boo_fraction == 1.0
    assert info.num_blocks == b.num_blocks() and info.x_loads >= info.num_blocks
    assert S.boo_arena_bytes(32, 32, 94, 64, 4) == 94 * 6 + 4 * 64 + 4 * 33 + 4 * 64 * 32


def test_clustering_identity_and_symmetric_copy():
    from spmm_amd.clustering import cluster_axes
    m = sp.random(100, 100, density=0.05, format='csr', random_state=0)
    m = (m + m.T).tocsr()
    rl, cl = cluster_axes(m, 'identity', 32, 32)
    assert np.array_equal(rl, O.identity_labels(100, 32)) and np.array_equal(cl, rl)
    r2 = sp.random(50, 70, density=0.1, format='csr', random_state=1)
    rl, cl = cluster_axes(r2, 'identity', 16, 32)
    assert np.array_equal(rl, O.identity_labels(50, 16))
    assert np.array_equal(cl, O.identity_labels(70, 32))
    for method, pkg in (('graclus', 'torch-cluster'), ('metis', 'pymetis')):
        with pytest.raises(ImportError, match=pkg):
            cluster_axes(m, method, 32, 32)
    with pytest.raises(ValueError):
        cluster_axes(m, 'bogus', 32, 32)


# ---------------------------------------------------------------- PBR builder
@pytest.mark.parametrize('name', fixture_names('pbr_'))
def test_csr_to_pbr_matches_reference_fixture_exactly(name):
    """All seven arrays, in the reference's block order (its hash map's)."""
    fx = load_fixture(name)
    br, bc, thr = (int(v) for v in fx['params'])
    p = S.csr_to_pbr(csr_of(fx), block_rows=br, block_cols=bc, min_nnz_per_block=thr)
    got = _arrays(p, O.PBR_FIELDS)
    for f in O.PBR_FIELDS:
        assert got[f].dtype == fx[f].dtype and np.array_equal(got[f], fx[f]), f
    y = S.pbr_batched_matmul_cpu(p, torch.from_numpy(fx['x']))
    assert np.array_equal(y.numpy(), fx['y_cpu'])
    r = S.pbr_to_csr(p)
    m = csr_of(fx)
    np.testing.assert_array_equal(r.indptr, m.indptr)
    np.testing.assert_array_equal(r.indices, m.indices)


@pytest.mark.parametrize('seed', range(6))
@pytest.mark.parametrize('bs', [2, 4, 8])
def test_csr_to_pbr_matches_oracle(seed, bs):
    dt = [np.float32, np.float64][seed % 2]
    it = [np.int32, np.int64][(seed // 2) % 2]
    r = np.random.default_rng(seed)
    n = int(r.integers(1, 200))
    m = _rand_csr(seed, n, int(r.integers(1, 200)), 0.08, dt, it)
    thr = int(r.integers(1, 8))
    p = S.csr_to_pbr(m, bs, bs, thr)
    o = O.pbr_build(m.indptr, m.indices, m.data, m.shape[0], m.shape[1], bs, bs, thr)
    canon = O.pbr_canonical(dict(rows=m.shape[0], cols=m.shape[1], block_rows=bs, block_cols=bs,
                                 **_arrays(p, O.PBR_FIELDS)))
    for f in O.PBR_FIELDS:
        assert canon[f].dtype == o[f].dtype and np.array_equal(canon[f], o[f]), f
    assert type(p).__name__ == f'PBRMatrixInt{np.dtype(it).itemsize * 8}' + \
        ('Float' if dt == np.float32 else 'Double')


def test_csr_to_pbr_live_reference(ref_core):
    """Raw order included, on a matrix with many block columns per stripe."""
    from spmm_amd import matrices as M
    A = M.permuted(M.stencil_27pt(16), seed=3)
    for bs, thr in ((8, 4), (4, 2), (2, 1)):
        p = S.csr_to_pbr(A, bs, bs, thr)
        r = ref_core.csr_to_pbr(A.indptr, A.indices, A.data, A.shape[0], A.shape[1], bs, bs, thr)
        for f in O.PBR_FIELDS:
            assert np.array_equal(np.asarray(getattr(p, f)), np.asarray(getattr(r, f))), (bs, f)


@pytest.mark.parametrize('rows', [1, 9, 13, 17, 1001])
@pytest.mark.parametrize('block_size', [4, 8])
@pytest.mark.parametrize('min_nnz', [1, 4, 64])
def test_pbr_roundtrip_partial_last_stripe(rows, block_size, min_nnz):
    """test_pbr.py:208-228."""
    rng = np.random.default_rng(0)
    mat = sp.random(rows, rows, density=0.3, format='lil', dtype=np.float32, random_state=rng)
    mat[rows - 1, rng.integers(0, rows, size=min(3, rows))] = 1.0
    mat = mat.tocsr()
    mat.sort_indices()
    p = S.csr_to_pbr(mat, block_size, block_size, min_nnz)
    r = S.pbr_to_csr(p)
    np.testing.assert_array_equal(r.indptr, mat.indptr)
    np.testing.assert_array_equal(r.indices, mat.indices)
    np.testing.assert_allclose(r.data, mat.data)


def test_pbr_config2_closed_form_counts():
    from spmm_amd import matrices as M
    A = M.stencil_27pt(64)
    p = S.csr_to_pbr(A, 8, 8, 4)
    assert (p.accounted_blocks(), p.compressed_nnz(), p.remainder_nnz()) == \
        (8 * 190 ** 2, 22 * 8 * 190 ** 2, 190 ** 3 - 22 * 8 * 190 ** 2)
    info = S.pbr_info(p)
    assert info.block_fill.min == info.block_fill.max == 22


def test_pbr_input_contract():
    with pytest.raises(TypeError):
        S.csr_to_pbr(np.eye(4))
    with pytest.raises(ValueError, match='CPU'):
        if not torch.cuda.is_available():
            raise ValueError('Input tensor must be on CPU')
        S.csr_to_pbr(torch.eye(4).to_sparse_csr().cuda())
    m = sp.random(10, 10, density=0.3, format='csr', random_state=0, dtype=np.float32)
    with pytest.raises(ValueError):
        S.csr_to_pbr(m, 8, 8, 300)
