"""HEM clustering (spmm_amd/clustering.py) against the oracle's loop
restatement (oracle/oracle.py hem_*), the reference's own known answers and
the published SplitMix64 vectors.  CPU only."""

import numpy as np
import pytest
import scipy.sparse as sp

import spmm_amd as S
from spmm_amd import clustering as C
from oracle import oracle as O

G64 = 0x9E3779B97F4A7C15


def _pat(A):
    return C._pattern(A)


def test_mix64_is_splitmix64():
    # SplitMix64 seeded with 0 outputs mix64(k * golden) for k = 1, 2, ...
    want = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4]
    for k, w in enumerate(want, start=1):
        z = (k * G64) % (1 << 64)
        assert O._mix64_int(z) == w
        assert int(C._mix64(np.array([z], dtype=np.uint64))[0]) == w


def test_pair_hash_symmetric_and_equal_to_oracle():
    rng = np.random.default_rng(0)
    a = rng.integers(0, 1 << 40, 500)
    b = rng.integers(0, 1 << 40, 500)
    h = C._pair_hash(a, b)
    assert np.array_equal(h, C._pair_hash(b, a)) and np.all(h >= 0)
    assert [int(x) for x in h] == [O.hem_pair_hash(int(x), int(y)) for x, y in zip(a, b)]


@pytest.mark.parametrize('cap_kind', ['size', 'nnz'])
def test_mutual_max_reference_known_answer(cap_kind):
    # tests/torch_fast_spdmm/test_boo_optimization.py:15-29 of the reference:
    # A-B is strongest but over the cap; A-C and B-D are feasible.
    W = np.array([[0, 10, 9, 0], [10, 0, 0, 8], [9, 0, 0, 0], [0, 8, 0, 0]])
    costs = np.array([30, 30, 2, 2])
    kw = dict(max_size=32 if cap_kind == 'size' else None, max_nnz=32 if cap_kind == 'nnz' else None)
    act = np.ones(4, dtype=bool)
    left, right = C._mutual_max_pairs(sp.csr_matrix(W), act, costs, costs, **kw, feasible_first=False)
    assert len(left) == 0
    left, right = C._mutual_max_pairs(sp.csr_matrix(W), act, costs, costs, **kw, feasible_first=True)
    assert set(zip(left.tolist(), right.tolist())) == {(0, 2), (1, 3)}
    edges = {(i, j): int(W[i, j]) for i in range(4) for j in range(4) if W[i, j]}
    assert O.hem_mutual_max(edges, 4, [True] * 4, costs, costs, **kw) == []
    assert O.hem_mutual_max(edges, 4, [True] * 4, costs, costs, **kw,
                            feasible_first=True) == [(0, 2), (1, 3)]


@pytest.mark.parametrize('shape,density', [((30, 30), 0.15), ((25, 40), 0.2), ((60, 45), 0.08)])
def test_oracle_similarity_is_shared_column_count(shape, density):
    A = sp.random(*shape, density=density, format='csr', random_state=1)
    P = (_pat(A).toarray() > 0).astype(np.int64)
    dense = P @ P.T
    np.fill_diagonal(dense, 0)
    got = O.hem_similarity(_pat(A), hub_degree=10 ** 9, topk=None)
    want = {(i, j): int(dense[i, j]) for i, j in zip(*np.nonzero(dense))}
    assert got == want


@pytest.mark.parametrize('seed', range(6))
@pytest.mark.parametrize('hub,topk', [(10 ** 9, None), (4, None), (10 ** 9, 3), (5, 2)])
def test_similarity_graph_matches_oracle(seed, hub, topk):
    rng = np.random.default_rng(seed)
    n, m = int(rng.integers(2, 50)), int(rng.integers(2, 60))
    A = sp.random(n, m, density=float(rng.uniform(0.05, 0.3)), format='csr', random_state=seed)
    W = C._similarity_graph(_pat(A), hub, topk, chunk_rows=7)
    got = {(int(i), int(j)): int(w) for i, j, w in zip(*sp.find(W)[:2], sp.find(W)[2])}
    assert got == O.hem_similarity(_pat(A), hub, topk)
    assert (W != W.T).nnz == 0


@pytest.mark.parametrize('seed', range(8))
@pytest.mark.parametrize('feasible_first', [False, True])
def test_mutual_max_matches_oracle(seed, feasible_first):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(5, 60))
    A = sp.random(n, 40, density=0.2, format='csr', random_state=seed)
    W = C._similarity_graph(_pat(A), 10 ** 9, 8)
    edges = O.hem_similarity(_pat(A), 10 ** 9, 8)
    active = rng.random(n) < 0.8
    size = rng.integers(1, 5, n)
    nnz = rng.integers(1, 20, n)
    for caps in [dict(), dict(max_size=5), dict(max_nnz=20), dict(max_size=6, max_nnz=25)]:
        left, right = C._mutual_max_pairs(W, active.copy(), size, nnz, caps.get('max_size'),
                                          caps.get('max_nnz'), feasible_first)
        want = O.hem_mutual_max(edges, n, list(active), size, nnz, feasible_first=feasible_first, **caps)
        assert sorted(zip(left.tolist(), right.tolist())) == want


@pytest.mark.parametrize('seed', range(6))
@pytest.mark.parametrize('target', [4, 8, 16])
@pytest.mark.parametrize('feasible_first', [False, True])
def test_hem_labels_match_oracle(seed, target, feasible_first):
    rng = np.random.default_rng(seed)
    n, m = int(rng.integers(10, 90)), int(rng.integers(10, 90))
    A = sp.random(n, m, density=float(rng.uniform(0.04, 0.2)), format='csr', random_state=seed)
    pat = _pat(A)
    for caps in [dict(max_size=target), dict(max_size=target, max_nnz=3 * target), dict()]:
        got = C._hem_labels(pat, target, caps.get('max_size'), caps.get('max_nnz'), 1024, 32,
                            feasible_first=feasible_first)
        want = O.hem_labels(pat, target, caps.get('max_size'), caps.get('max_nnz'),
                            feasible_first=feasible_first)
        assert np.array_equal(got, want)


def test_hem_hub_pruning_and_topk_reach_the_labels():
    # small hub degree and top-k change the graph, and the labels follow it
    A = sp.random(70, 50, density=0.2, format='csr', random_state=3)
    pat = _pat(A)
    for hub, topk in [(6, 32), (1024, 2)]:
        assert np.array_equal(C._hem_labels(pat, 8, 8, None, hub, topk),
                              O.hem_labels(pat, 8, 8, None, hub_degree=hub, topk=topk))


@pytest.mark.parametrize('shape', [(97, 97), (73, 89)])
@pytest.mark.parametrize('target', [(8, 8), (16, 8), (8, 16)])
def test_hem_clustering_roundtrip_caps_and_determinism(shape, target):
    # tests/torch_fast_spdmm/test_boo_optimization.py:32-42 of the reference
    mat = sp.random(*shape, density=0.12, format='csr', dtype=np.float32, random_state=7)
    kw = dict(target_nr=target[0], target_nc=target[1], hem_feasible_first=True)
    first, second = S.csr_to_boo(mat, **kw), S.csr_to_boo(mat, **kw)
    assert (S.boo_to_csr(first) != mat).nnz == 0
    for name in ('row_grp_ptr', 'row_ids', 'col_grp_ptr', 'col_ids', 'nz_idx', 'nz_val'):
        np.testing.assert_array_equal(getattr(first, name), getattr(second, name))
    assert max(np.diff(first.row_grp_ptr), default=0) <= target[0]
    assert max(np.diff(first.col_grp_ptr), default=0) <= target[1]


def _square(n=256, density=0.05, seed=0, dtype=np.float32):
    rng = np.random.default_rng(seed)
    mat = sp.random(n, n, density=density, format='csr', random_state=seed)
    mat.data = rng.standard_normal(mat.nnz)
    return mat.astype(dtype)


@pytest.mark.parametrize('policy,threshold', [('keep', 0), ('remainder', 4), ('tail_batch', 4)])
@pytest.mark.parametrize('order', ['rowmajor', 'colmajor'])
def test_hem_boo_roundtrip_and_cpu_product(policy, threshold, order):
    # test_boo.py:104-116 and :193-205 of the reference, cluster='hem'
    mat = _square()
    boo = S.csr_to_boo(mat, cluster='hem', target_nr=16, target_nc=16, small_block_policy=policy,
                       small_block_threshold=threshold, nz_order=order)
    assert (S.boo_to_csr(boo) != mat).nnz == 0
    again = S.csr_to_boo(mat, cluster='hem', target_nr=16, target_nc=16, small_block_policy=policy,
                         small_block_threshold=threshold, nz_order=order)
    for f in O.BOO_FIELDS:
        assert np.array_equal(np.asarray(getattr(boo, f)), np.asarray(getattr(again, f))), f
    import torch
    x = torch.randn(256, 7, generator=torch.Generator().manual_seed(0))
    y = S.boo_matmul(boo, x).numpy()              # CPU X: the reference's CPU op order
    np.testing.assert_allclose(y, mat.astype(np.float64) @ x.numpy().astype(np.float64),
                               rtol=1e-4, atol=1e-4)


def test_hem_tail_batch_leaves_a_tail():
    # test_boo.py:218-231 of the reference: this matrix has a tail under HEM 16
    boo = S.csr_to_boo(_square(n=512, density=0.02), cluster='hem', target_nr=16, target_nc=16,
                       small_block_policy='tail_batch', small_block_threshold=4)
    assert boo.remainder_nnz() == 0 and boo.tail_nnz() > 0
    info = S.boo_info(boo)
    assert info.compressed_fraction < 1.0 and info.boo_fraction == 1.0


def test_hem_hierarchy_records_every_level():
    A = _square(n=128, density=0.06)
    levels = []
    labels = C.cluster_axis(A, 'hem', target=16, max_size=16, hem_hierarchy=levels)
    assert np.array_equal(levels[0], np.arange(128)) and len(levels) >= 3
    assert np.array_equal(levels[-1], C._hem_labels(C._pattern(A), 16, 16, None, 1024, 32))
    assert labels.dtype == np.int32 and np.bincount(labels).max() <= 16
    with pytest.raises(ValueError, match='hem_hierarchy'):
        C.cluster_axis(A, 'identity', hem_hierarchy=[])


@pytest.mark.parametrize('n', [0, 1, 19])
def test_hem_empty_similarity_graph(n):
    # test_clustering_backends.py:52-57 of the reference, with hem
    labels = C.cluster_axis(sp.eye(n, format='csr'), method='hem', target=8, max_size=8)
    assert len(labels) == n
    if n:
        assert np.bincount(labels).max() <= 8


def test_hem_is_the_default_and_groups_the_banded_matrix():
    a = sp.diags([np.ones(511), np.ones(512), np.ones(511)], [-1, 0, 1], shape=(512, 512),
                 format='csr', dtype=np.float32)
    rows, cols = C.cluster_axes(a, target_nr=16, target_nc=16, max_nr=16, max_nc=16)
    assert np.array_equal(rows, cols) and np.bincount(rows).max() <= 16
    # neighbours share columns, so groups are far fewer than the rows
    assert rows.max() + 1 < 512 // 4
    boo = S.csr_to_boo(a)                               # default cluster='hem'
    assert (S.boo_to_csr(boo) != a).nnz == 0


def _golden_cases():
    from pathlib import Path
    import ast
    path = Path(__file__).resolve().parent / 'golden' / 'hem_labels.npz'
    z = np.load(path)
    names = sorted({k.split('__')[0] for k in z.files})
    out = []
    for nm in names:
        shape = tuple(int(v) for v in z[f'{nm}__shape'])
        indptr, indices = z[f'{nm}__indptr'], z[f'{nm}__indices']
        A = sp.csr_matrix((np.ones(indices.size), indices, indptr), shape=shape)
        kw = ast.literal_eval(str(z[f'{nm}__kw']))
        axes = (z[f'{nm}__axes_rows'], z[f'{nm}__axes_cols']) if f'{nm}__axes_rows' in z.files else None
        out.append((nm, A, kw, z[f'{nm}__labels'], axes))
    return out


GOLDEN = _golden_cases()


@pytest.mark.parametrize('case', GOLDEN, ids=[c[0] for c in GOLDEN])
def test_hem_labels_equal_reference_vectors(case):
    """Labels written by the reference's own clustering.py
    (tests/golden/make_hem_fixtures.py): the product and the oracle both."""
    name, A, kw, want, axes = case
    got = C.cluster_axis(A, **kw)
    assert got.dtype == np.int32 and np.array_equal(got, want)
    raw = O.hem_labels(C._pattern(A), kw['target'], kw.get('max_size'), kw.get('max_nnz'),
                       hub_degree=kw.get('hub_degree', 1024), topk=kw.get('topk', 32),
                       feasible_first=kw['feasible_first'])
    capped = C._enforce_caps(raw, np.diff(C._pattern(A).indptr), kw.get('max_size'), kw.get('max_nnz'))
    assert np.array_equal(C._relabel_consecutive(capped), want)
    if axes is not None:
        r, c = C.cluster_axes(A, 'hem', kw['target'], kw['target'], kw.get('max_size'),
                              kw.get('max_size'), feasible_first=kw['feasible_first'])
        assert np.array_equal(r, axes[0]) and np.array_equal(c, axes[1])


def test_size_cap_without_the_member_loop():
    """_enforce_caps with only a size cap runs without the per-member loop;
    it must give the loop's labels (the loop runs when an nnz cap is given:
    an nnz cap nothing reaches makes it the size-cap loop)."""
    from spmm_amd import clustering as C
    rng = np.random.default_rng(0)
    for trial in range(200):
        n = int(rng.integers(0, 300))
        lab = rng.integers(0, max(1, int(rng.integers(1, 40))), n)
        if trial % 3 == 0:
            lab = np.sort(lab)
        nnz = rng.integers(0, 10, n)
        cap = int(rng.integers(1, 12))
        assert np.array_equal(C._enforce_caps(lab, nnz, cap, None), C._enforce_caps(lab, nnz, cap, 10 ** 12))
