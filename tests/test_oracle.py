"""Pin the CPU oracle (oracle/oracle.py) before trusting it.

Each check is independent of the oracle's own formulas: the reference's
written-out worked example and test counts, closed forms derived from the
stencil geometry, the compiled reference (when built), and dense fp64
products.
"""

import numpy as np
import pytest
import scipy.sparse as sp

from conftest import csr_of, fixture_names, load_fixture
from oracle import oracle as O
from spmm_amd import matrices as M


# ---------------------------------------------------------------- labels
def test_identity_labels_closed_form():
    lab = O.identity_labels(100, 32)
    assert lab.dtype == np.int32
    assert np.array_equal(lab, np.r_[np.zeros(32), np.ones(32), np.full(32, 2), np.full(4, 3)])
    assert O.identity_labels(0, 32).size == 0


# ---------------------------------------------------------------- BOO
def _worked_example():
    """docs/reference/BOO_FORMAT.md:102-131, values a..g = 1..7."""
    a, b, c, d, e, f, g = 1., 2., 3., 4., 5., 6., 7.
    ent = [(0, 0, a), (0, 3, b), (1, 1, e), (2, 0, c), (3, 4, f), (4, 5, d), (5, 3, g)]
    r, cc, v = zip(*ent)
    m = sp.csr_matrix((np.array(v, np.float32), (r, cc)), shape=(6, 6))
    rl = np.array([0, 1, 0, 1, 0, 1], np.int32)       # RG0={0,2,4}, RG1={1,3,5}
    cl = np.array([0, 1, 1, 0, 1, 1], np.int32)       # CG0={0,3}, CG1={1,2,4,5}
    return m, rl, cl


def test_boo_worked_example_every_array():
    m, rl, cl = _worked_example()
    o = O.boo_build(m.indptr, m.indices, m.data, 6, 6, rl, cl, policy=0)
    assert list(o['row_grp_ptr']) == [0, 3, 6]
    assert list(o['row_ids']) == [0, 2, 4, 1, 3, 5]
    assert list(o['col_grp_ptr']) == [0, 2, 6]
    assert list(o['col_ids']) == [0, 3, 1, 2, 4, 5]
    assert list(o['blk_row_grp']) == [0, 0, 1, 1]
    assert list(o['blk_col_grp']) == [0, 1, 0, 1]
    assert list(o['blk_nz_ptr']) == [0, 3, 4, 5, 7]
    assert list(o['nz_idx']) == [0, 1, 2, 11, 5, 0, 6]
    assert list(o['nz_val']) == [1., 2., 3., 4., 7., 5., 6.]   # a,b,c, d, g, e,f
    assert list(o['blk_shift']) == [1, 2, 1, 2]
    assert (o['max_nr'], o['max_nc'], o['max_nnz_blk']) == (3, 4, 3)
    assert o['rem_col_ind'].size == 0 and o['tail_val'].size == 0


def _example_7x11(dtype=np.float32, itype=np.int32):
    """tests/torch_fast_spdmm/test_boo_edges.py:21-31."""
    ent = [(0, 0, 2), (0, 2, -1), (2, 6, 3), (2, 0, 1), (0, 1, 4), (1, 1, 2), (1, 4, -3),
           (4, 7, 1), (4, 9, 2), (4, 3, -2), (3, 5, 1)]
    r, c, v = zip(*ent)
    m = sp.csr_matrix((np.array(v, dtype=dtype), (r, c)), shape=(7, 11))
    m.indptr, m.indices = m.indptr.astype(itype), m.indices.astype(itype)
    return (m, np.array([0, 1, 0, 2, 1, 0, 2], np.int32),
            np.array([0, 1, 0, 2, 1, 2, 0, 1, 2, 1, 2], np.int32))


@pytest.mark.parametrize('policy,comp,rem,tail', [(0, 11, 0, 0), (2, 8, 3, 0), (3, 8, 0, 3)])
@pytest.mark.parametrize('order', [0, 1])
def test_boo_7x11_counts_and_roundtrip(policy, comp, rem, tail, order):
    """test_boo_edges.py:53-70: keep -> 11 compressed; remainder(4) -> 8 + 3."""
    m, rl, cl = _example_7x11(np.float64, np.int64)
    o = O.boo_build(m.indptr, m.indices, m.data, 7, 11, rl, cl, policy, 4, order)
    assert o['nz_val'].size == comp and o['rem_vals'].size == rem and o['tail_val'].size == tail
    assert o['row_grp_ptr'].dtype == np.int64 and o['nz_val'].dtype == np.float64
    np.testing.assert_array_equal(O.boo_decode(o).toarray(), m.toarray())
    for ptr, length in (('row_grp_ptr', 7), ('col_grp_ptr', 11), ('blk_nz_ptr', comp),
                        ('rem_indptr', rem)):
        assert o[ptr][0] == 0 and o[ptr][-1] == length and np.all(np.diff(o[ptr]) >= 0)


def test_boo_uint16_endpoint_and_overflow():
    """test_boo_edges.py:186-196 (last coordinate 65535) and :223-227 (one
    more row must be rejected)."""
    m = sp.csr_matrix((np.array([2, -3, 4], np.float64), ([0, 128, 255], [0, 1, 255])),
                      shape=(256, 256))
    z = np.zeros(256, np.int32)
    o = O.boo_build(m.indptr, m.indices, m.data, 256, 256, z, z, policy=0)
    assert o['nz_idx'].max() == 65535 and list(o['blk_shift']) == [8]
    m2 = sp.csr_matrix(([1.0], ([256], [255])), shape=(257, 256), dtype=np.float32)
    with pytest.raises(ValueError, match='uint16'):
        O.boo_build(m2.indptr, m2.indices, m2.data, 257, 256, np.zeros(257, np.int32),
                    np.zeros(256, np.int32), policy=0)


@pytest.mark.parametrize('order', [0, 1])
def test_boo_invariants_random(order):
    """Format invariants of test_boo.py:130-191 on a random square matrix."""
    m = sp.random(256, 256, density=0.05, format='csr', random_state=0, dtype=np.float32)
    rl = O.identity_labels(256, 16)
    o = O.boo_build(m.indptr, m.indices, m.data, 256, 256, rl, rl, 2, 4, order)
    assert np.array_equal(np.sort(o['row_ids']), np.arange(256))
    rgp, nzp, sh = o['row_grp_ptr'], o['blk_nz_ptr'], o['blk_shift'].astype(np.int64)
    for b in range(o['blk_row_grp'].size):
        blk = o['nz_idx'][nzp[b]:nzp[b + 1]].astype(np.int64)
        n_r = rgp[o['blk_row_grp'][b] + 1] - rgp[o['blk_row_grp'][b]]
        assert np.all((blk >> sh[b]) < n_r)
        key = blk if order == 0 else (((blk & ((1 << sh[b]) - 1)) << 32) | (blk >> sh[b]))
        assert np.all(np.diff(key) > 0)
    assert o['nz_val'].size + o['rem_vals'].size == m.nnz


def _stencil_counts():
    from spmm_amd import matrices as M
    return M


def test_config_closed_form_counts():
    """Closed forms from the stencil geometry (not from the builder):
    27-pt 64^3: nnz = 190^3; identity 32: a kept block per (row half-line,
    neighbouring line) = 2*190^2, each the 32x32 tridiagonal band with 94
    entries; the cross-half entries (one per block row edge) spill.  8x8 PBR
    (threshold 4): 8 band blocks of 22 entries per line pair; corners spill.
    2-D 5-pt 256^2: per 32-row group, 1 band block (94) and 1-2 identity
    blocks (32) from the neighbouring grid lines."""
    M = _stencil_counts()
    A = M.stencil_27pt(64)
    assert A.nnz == 190 ** 3
    rl = O.identity_labels(A.shape[0], 32)
    o = O.boo_build(A.indptr, A.indices, A.data, A.shape[0], A.shape[1], rl, rl, 2, 4, 0)
    nb = 2 * 190 ** 2
    assert o['blk_row_grp'].size == nb
    assert np.all(np.diff(o['blk_nz_ptr']) == 94)
    assert o['nz_val'].size == 94 * nb and o['rem_vals'].size == 190 ** 3 - 94 * nb
    assert (o['max_nr'], o['max_nc'], o['max_nnz_blk']) == (32, 32, 94)
    p = O.pbr_build(A.indptr, A.indices, A.data, A.shape[0], A.shape[1], 8, 8, 4)
    assert p['block_codes'].size == 8 * 190 ** 2
    assert p['block_data'].size == 22 * 8 * 190 ** 2
    assert p['remainder_data'].size == 190 ** 3 - 22 * 8 * 190 ** 2

    L = M.laplacian_2d(256)
    assert L.nnz == 5 * 65536 - 4 * 256
    rl = O.identity_labels(65536, 32)
    o = O.boo_build(L.indptr, L.indices, L.data, 65536, 65536, rl, rl, 2, 4, 0)
    per_half = 256 + 2 * 255          # band blocks + neighbour-line identity blocks
    assert o['blk_row_grp'].size == 8 * per_half
    assert o['nz_val'].size == 8 * (256 * 94 + 510 * 32)
    assert o['rem_vals'].size == L.nnz - 8 * (256 * 94 + 510 * 32)


# ---------------------------------------------------------------- vs compiled reference fixtures
@pytest.mark.parametrize('name', fixture_names('boo_'))
def test_boo_oracle_matches_reference_fixture(name):
    fx = load_fixture(name)
    pol, thr, order = (int(v) for v in fx['params'])
    rows, cols = (int(v) for v in fx['shape'])
    o = O.boo_build(fx['indptr'], fx['indices'], fx['data'], rows, cols, fx['row_labels'],
                    fx['col_labels'], pol, thr, order)
    for f in O.BOO_FIELDS:
        assert o[f].dtype == fx[f].dtype and np.array_equal(o[f], fx[f]), f
    assert [o['max_nr'], o['max_nc'], o['max_nnz_blk']] == list(fx['maxima'])
    y = O.boo_cpu_matmul(o, fx['x'])
    assert y.dtype == fx['y_cpu'].dtype and np.array_equal(y, fx['y_cpu'][0])   # bit for bit


@pytest.mark.parametrize('name', fixture_names('pbr_'))
def test_pbr_oracle_matches_reference_fixture(name):
    fx = load_fixture(name)
    br, bc, thr = (int(v) for v in fx['params'])
    rows, cols = (int(v) for v in fx['shape'])
    o = O.pbr_build(fx['indptr'], fx['indices'], fx['data'], rows, cols, br, bc, thr)
    ref = dict(rows=rows, cols=cols, block_rows=br, block_cols=bc,
               **{f: fx[f] for f in O.PBR_FIELDS})
    canon = O.pbr_canonical(ref)
    for f in O.PBR_FIELDS:
        assert o[f].dtype == canon[f].dtype and np.array_equal(o[f], canon[f]), f
    # the CPU op consumes blocks in the reference's own order: bit for bit
    assert np.array_equal(O.pbr_cpu_matmul(ref, fx['x'])[0], fx['y_cpu'][0])
    np.testing.assert_array_equal(O.pbr_decode(ref).toarray(), csr_of(fx).toarray())


# ---------------------------------------------------------------- vs compiled reference (live)
@pytest.mark.parametrize('seed', range(6))
def test_oracle_matches_compiled_reference(ref_core, seed):
    r = np.random.default_rng(100 + seed)
    rows, cols = int(r.integers(1, 90)), int(r.integers(1, 90))
    dt = [np.float32, np.float64][seed % 2]
    it = [np.int32, np.int64][(seed // 2) % 2]
    dense = r.normal(size=(rows, cols))
    dense[r.random((rows, cols)) > 0.2] = 0
    m = sp.csr_matrix(dense.astype(dt))
    m.indptr, m.indices = m.indptr.astype(it), m.indices.astype(it)
    rl = r.integers(0, max(1, rows // 6), size=rows).astype(np.int32)
    cl = r.integers(0, max(1, cols // 6), size=cols).astype(np.int32)
    for pol in (0, 2, 3):
        for order in (0, 1):
            o = O.boo_build(m.indptr, m.indices, m.data, rows, cols, rl, cl, pol, 4, order)
            b = ref_core.csr_to_boo(m.indptr, m.indices, m.data, rows, cols, rl, cl, pol, 4, order)
            for f in O.BOO_FIELDS:
                assert np.array_equal(o[f], np.asarray(getattr(b, f))), (pol, order, f)
    for bs in (2, 4, 8):
        o = O.pbr_build(m.indptr, m.indices, m.data, rows, cols, bs, bs, 3)
        p = ref_core.csr_to_pbr(m.indptr, m.indices, m.data, rows, cols, bs, bs, 3)
        canon = O.pbr_canonical(dict(rows=rows, cols=cols, block_rows=bs, block_cols=bs,
                                     **{f: np.asarray(getattr(p, f)) for f in O.PBR_FIELDS}))
        for f in O.PBR_FIELDS:
            assert np.array_equal(o[f], canon[f]), (bs, f)


# ---------------------------------------------------------------- numerics
def test_cpu_matmul_oracle_vs_dense_fp64():
    """test_boo.py:241-254: the CPU loop order in fp64 agrees with the dense
    product to rtol 1e-10."""
    m = sp.random(200, 200, density=0.05, format='csr', random_state=1, dtype=np.float64)
    rl = O.identity_labels(200, 16)
    x = np.random.default_rng(3).standard_normal((200, 24))
    o = O.boo_build(m.indptr, m.indices, m.data, 200, 200, rl, rl, 2, 4, 0)
    np.testing.assert_allclose(O.boo_cpu_matmul(o, x), m.toarray() @ x, rtol=1e-10, atol=1e-10)
    p = O.pbr_build(m.indptr, m.indices, m.data, 200, 200, 8, 8, 4)
    np.testing.assert_allclose(O.pbr_cpu_matmul(p, x)[0], m.toarray() @ x, rtol=1e-10, atol=1e-10)


def test_within_bound_detects_a_planted_error():
    m = sp.random(50, 40, density=0.2, format='csr', random_state=2, dtype=np.float32)
    x = np.random.default_rng(4).standard_normal((40, 8)).astype(np.float32)
    y = (m.astype(np.float64) @ x.astype(np.float64)).astype(np.float32)
    ratio, ok = O.within_bound(y, m, x)
    assert ok and ratio < 1e-6
    y[3, 2] += 1e-3 * (abs(m) @ abs(x))[3, 2] + 1e-3
    assert not O.within_bound(y, m, x)[1]


def test_reference_product_leaves_unsorted_input_untouched():
    """A CSR whose rows are not sorted (P A P^T with fancy indexing) must
    come out of spmm_reference unchanged, and the product must equal the
    dense product every time (scipy canonicalises matrices in place, and a
    dtype-converting csr_matrix(...) shares the caller's index arrays)."""
    A0 = M.stencil_27pt(10)
    n = A0.shape[0]
    perm = np.random.default_rng(4).permutation(n)
    A = sp.csr_matrix(A0[perm][:, perm])
    assert not A.has_sorted_indices
    before = (A.indptr.copy(), A.indices.copy(), A.data.copy())
    x = M.dense_x(n, 32, seed=3)
    dense = A.toarray().astype(np.float64) @ x.astype(np.float64)
    for _ in range(3):
        ref, bound = O.spmm_reference(A, x)
        assert np.abs(ref - dense).max() < 1e-12
        assert np.all(bound >= np.abs(ref))
        for a, b in zip(before, (A.indptr, A.indices, A.data)):
            assert np.array_equal(a, b)


def test_builders_leave_unsorted_input_untouched():
    import spmm_amd as S
    A0 = M.stencil_27pt(8)
    n = A0.shape[0]
    perm = np.random.default_rng(1).permutation(n)
    A = sp.csr_matrix(A0[perm][:, perm])
    assert not A.has_sorted_indices
    before = (A.indptr.copy(), A.indices.copy(), A.data.copy())
    S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32)
    S.csr_to_pbr(A, 8, 8, 4)
    for a, b in zip(before, (A.indptr, A.indices, A.data)):
        assert np.array_equal(a, b)
