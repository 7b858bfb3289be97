"""BOO on the GPU against the oracle's fp64 product and error bound.

Bar: |Y - A X| <= 1e-5 * (|A|.|X|) elementwise for float32 (1e-12 for
float64), against the fp64 product of the ORIGINAL CSR -- never a decoder of
the format under test.  Cases follow the reference's GPU contract
(tests/torch_fast_spdmm/test_boo_edges.py, test_boo.py).
"""

import numpy as np
import pytest
import scipy.sparse as sp
import torch

import spmm_amd as S
import spmm_amd.boo as SB
from oracle import oracle as O

pytestmark = pytest.mark.gpu

POLICIES = ['keep', 'remainder', 'tail_batch']
ORDERS = ['rowmajor', 'colmajor']


@pytest.fixture(autouse=True, params=['tile', 'gather'])
def path(request, monkeypatch):
    """Run every case twice: with every slice in the tile stream, and with
    every slice light enough sent to the row-wise gather pass."""
    monkeypatch.setattr(SB, 'MIN_COL_REUSE', 0.0 if request.param == 'tile' else 1e9)
    return request.param


def _tol(dtype):
    return 1e-5 if dtype in (torch.float32, np.float32) else 1e-12


def check(y, A, x):
    assert y.is_cuda
    ratio, ok = O.within_bound(y.detach().cpu().numpy(), A, x.detach().cpu().numpy(), _tol(y.dtype))
    assert ok, f'max |err|/(|A||X|) = {ratio:.3e}'


def _example(dtype=np.float32, index_dtype=np.int32):
    ent = [(0, 0, 2), (0, 2, -1), (2, 6, 3), (2, 0, 1), (0, 1, 4), (1, 1, 2), (1, 4, -3),
           (4, 7, 1), (4, 9, 2), (4, 3, -2), (3, 5, 1)]
    r, c, v = zip(*ent)
    m = sp.csr_matrix((np.array(v, dtype=dtype), (r, c)), shape=(7, 11))
    m.indptr, m.indices = m.indptr.astype(index_dtype), m.indices.astype(index_dtype)
    return m, np.array([0, 1, 0, 2, 1, 0, 2]), np.array([0, 1, 0, 2, 1, 2, 0, 1, 2, 1, 2])


def _x(shape, dtype=torch.float32, seed=123):
    return torch.randn(shape, dtype=dtype, generator=torch.Generator().manual_seed(seed))


def _build(m, rl, cl, policy='keep', order='rowmajor', threshold=4):
    return S.csr_to_boo(m, row_labels=rl, col_labels=cl, small_block_policy=policy,
                        small_block_threshold=threshold, nz_order=order)


@pytest.mark.parametrize('order', ORDERS)
@pytest.mark.parametrize('features', [1, 7, 8, 9, 31, 32, 33, 63, 64, 65, 127, 128, 129, 511, 512, 513, 1025])
@pytest.mark.parametrize('dtype', [torch.float32, torch.float64])
def test_feature_boundaries(order, features, dtype):
    m, rl, cl = _example(np.float32 if dtype == torch.float32 else np.float64)
    boo = _build(m, rl, cl, order=order).to('cuda')
    x = _x((2, 11, features), dtype).cuda()
    check(S.boo_matmul(boo, x), m, x)


@pytest.mark.parametrize('threads', [128, 256, 512])
@pytest.mark.parametrize('p', [8, 16, 32, 64, 128])
def test_launch_knobs_accepted(threads, p):
    m, rl, cl = _example()
    boo = _build(m, rl, cl).to('cuda')
    x = _x((11, 257)).cuda()
    check(S.boo_matmul(boo, x, threads=threads, p=p), m, x)


@pytest.mark.parametrize('order', ORDERS)
@pytest.mark.parametrize('policy,threshold', [('remainder', 4), ('tail_batch', 4), ('remainder', 100),
                                              ('tail_batch', 100)])
def test_mixed_and_all_spilled(order, policy, threshold):
    m, rl, cl = _example()
    boo = _build(m, rl, cl, policy, order, threshold).to('cuda')
    assert boo.compressed_nnz() == (8 if threshold == 4 else 0)
    for csr_mode in (0, 2):
        x = _x((2, 11, 65)).cuda()
        check(S.boo_matmul(boo, x, csr_mode=csr_mode), m, x)


@pytest.mark.parametrize('shape', [(0, 0), (0, 5), (5, 0), (5, 7)])
@pytest.mark.parametrize('policy', POLICIES)
def test_empty_matrix(shape, policy):
    m = sp.csr_matrix(shape, dtype=np.float32)
    boo = S.csr_to_boo(m, cluster='identity', small_block_policy=policy).to('cuda')
    x = _x((2, shape[1], 9)).cuda()
    y = S.boo_matmul(boo, x)
    assert y.shape == (2, shape[0], 9) and torch.count_nonzero(y).item() == 0


@pytest.mark.parametrize('x_shape', [(11, 0), (0, 11, 9), (2, 11, 0)])
@pytest.mark.parametrize('policy', POLICIES)
def test_empty_dense_dimensions(x_shape, policy):
    m, rl, cl = _example()
    boo = _build(m, rl, cl, policy).to('cuda')
    y = S.boo_matmul(boo, _x(x_shape).cuda())
    assert y.shape == (x_shape[:-2] + (7, x_shape[-1]))


@pytest.mark.parametrize('order', ORDERS)
@pytest.mark.parametrize('shape', [(1, 1), (1, 17), (19, 1)])
def test_singleton_axes(order, shape):
    m = sp.csr_matrix(np.arange(1, np.prod(shape) + 1, dtype=np.float32).reshape(shape))
    boo = _build(m, np.zeros(shape[0], int), np.zeros(shape[1], int), order=order).to('cuda')
    x = _x((shape[1], 33)).cuda()
    check(S.boo_matmul(boo, x), m, x)


@pytest.mark.parametrize('dtype', [torch.float32, torch.float64])
def test_int64_host_indices(dtype):
    m, rl, cl = _example(np.float32 if dtype == torch.float32 else np.float64, np.int64)
    boo = _build(m, rl, cl, 'tail_batch').to('cuda')
    assert 'Int64' in type(boo).__name__
    x = _x((2, 11, 33), dtype).cuda()
    check(S.boo_matmul(boo, x), m, x)


@pytest.mark.parametrize('order', ORDERS)
def test_many_blocks_accumulate_into_same_rows(order):
    """257 blocks of ones into 3 rows: exact integers, no lost update."""
    m = sp.csr_matrix(np.ones((3, 257), dtype=np.float32))
    boo = _build(m, np.zeros(3, int), np.arange(257), order=order).to('cuda')
    assert boo.num_blocks() == 257
    x = torch.ones(257, 17, device='cuda')
    for _ in range(3):
        got = S.boo_matmul(boo, x)
        assert torch.equal(got.cpu(), torch.full((3, 17), 257.))


@pytest.mark.parametrize('layout', ['transpose', 'slice', 'expand', 'batch_transpose'])
def test_noncontiguous_x(layout):
    m, rl, cl = _example()
    boo = _build(m, rl, cl, 'remainder').to('cuda')
    if layout == 'transpose':
        x = _x((13, 11)).cuda().T
    elif layout == 'slice':
        x = _x((11, 26)).cuda()[:, 1::2]
    elif layout == 'expand':
        x = _x((11, 1)).cuda().expand(11, 13)
    else:
        x = _x((3, 13, 11)).cuda().transpose(1, 2)
    saved = x.clone()
    check(S.boo_matmul(boo, x), m, x)
    assert torch.equal(x, saved)


@pytest.mark.parametrize('order', ORDERS)
def test_uint16_high_bit_and_last_coordinate(order):
    mat = sp.csr_matrix((np.array([2, -3, 4], np.float64), ([0, 128, 255], [0, 1, 255])),
                        shape=(256, 256))
    z = np.zeros(256, dtype=np.int32)
    boo = _build(mat, z, z, order=order).to('cuda')
    assert max(boo.nz_idx) == 65535
    x = _x((256, 9), torch.float64).cuda()
    check(S.boo_matmul(boo, x, p=8, threads=128), mat, x)


@pytest.mark.parametrize('order', ORDERS)
def test_large_blocks_beyond_lds_tiles(order):
    """A 32x64 dense block (2048 entries, 64 columns) and a 256x256 dense
    block: both exceed the LDS tile and the staged-nonzero cap."""
    for shape in ((32, 64), (256, 256)):
        mat = sp.csr_matrix(np.ones(shape, dtype=np.float64))
        boo = _build(mat, np.zeros(shape[0], int), np.zeros(shape[1], int), order=order).to('cuda')
        x = _x((2, shape[1], 129), torch.float64).cuda()
        check(S.boo_matmul(boo, x), mat, x)


@pytest.mark.parametrize('seed', range(12))
def test_seeded_randomized_product(seed):
    rng = np.random.default_rng(seed)
    rows, cols = int(rng.integers(2, 40)), int(rng.integers(2, 50))
    dtype = np.float32 if seed % 2 else np.float64
    tdt = torch.float32 if seed % 2 else torch.float64
    dense = rng.normal(size=(rows, cols))
    dense[rng.random((rows, cols)) > (0.05 + 0.07 * seed)] = 0
    mat = sp.csr_matrix(dense.astype(dtype))
    rl = rng.integers(0, min(rows, 5), size=rows)
    cl = rng.integers(0, min(cols, 6), size=cols)
    features = [1, 17, 65, 129, 513, 1025][seed % 6]
    for order in ORDERS:
        boo = _build(mat, rl, cl, POLICIES[seed % 3], order).to('cuda')
        x = _x((2, cols, features), tdt, seed).cuda()
        check(S.boo_matmul(boo, x, threads=[128, 256, 512][seed % 3]), mat, x)


@pytest.mark.parametrize('seed', range(6))
def test_random_square_identity_and_targets(seed):
    """Identity tiles of 8/16/32 over random sparse squares (test_boo.py:261-277)."""
    rng = np.random.default_rng(seed)
    n = 256 + 37 * seed
    mat = sp.random(n, n, density=0.05, format='csr', random_state=seed, dtype=np.float32)
    mat.data = rng.standard_normal(mat.nnz).astype(np.float32)
    for target in (8, 16, 32):
        boo = S.csr_to_boo(mat, cluster='identity', target_nr=target, target_nc=target).to('cuda')
        for K in (32, 64, 100, 128):
            x = _x((n, K), seed=seed).cuda()
            check(S.boo_matmul(boo, x), mat, x)


@pytest.mark.parametrize('order', ORDERS)
def test_unsorted_duplicates_and_explicit_zeros(order):
    mat = sp.csr_matrix((np.array([2., -2., 0., 3., 4.]), np.array([3, 3, 1, 0, 2]),
                         np.array([0, 4, 5, 5])), shape=(3, 5))
    boo = _build(mat, np.zeros(3, int), np.zeros(5, int), order=order).to('cuda')
    x = _x((5, 17), torch.float64).cuda()
    check(S.boo_matmul(boo, x), mat, x)


@pytest.mark.parametrize('policy', POLICIES)
def test_nondefault_stream_producer_consumer(policy):
    m, rl, cl = _example()
    boo = _build(m, rl, cl, policy).to('cuda')
    stream = torch.cuda.Stream()
    base = _x((13, 11))
    outputs = []
    with torch.cuda.stream(stream):
        for i in range(8):
            x = (base.to('cuda') + i).T
            outputs.append(S.boo_matmul(boo, x) * 2 + 1)
    stream.synchronize()
    for i, got in enumerate(outputs):
        expected = torch.from_numpy(m.toarray()).double() @ (base.double() + i).T
        torch.testing.assert_close(got.cpu().double(), expected * 2 + 1, rtol=3e-5, atol=3e-5)


def test_device_staging_is_idempotent_and_reversible():
    m, rl, cl = _example()
    boo = _build(m, rl, cl).to('cuda')
    meta = boo._gpu_meta
    assert boo.to('cuda') is boo and boo._gpu_meta is meta
    assert meta.nz_idx.dtype == torch.int16 and meta.blk_shift.dtype == torch.uint8
    assert meta.row_ids.dtype == torch.int32
    boo.to('cpu')
    with pytest.raises(RuntimeError, match='not'):
        S.boo_matmul(boo, _x((11, 17)).cuda())
    x = _x((11, 17)).cuda()
    check(S.boo_matmul(boo.to('cuda'), x), m, x)


def test_invalid_x_contract_cuda():
    m, rl, cl = _example()
    boo = _build(m, rl, cl).to('cuda')
    for shape in [(11,), (1, 1, 11, 3)]:
        with pytest.raises(ValueError, match='2D or 3D'):
            S.boo_matmul(boo, torch.zeros(shape, device='cuda'))
    with pytest.raises(ValueError, match='rows'):
        S.boo_matmul(boo, torch.zeros(10, 3, device='cuda'))
    for dtype in (torch.float64, torch.float16, torch.int32):
        with pytest.raises(TypeError, match='dtype'):
            S.boo_matmul(boo, torch.zeros(11, 3, dtype=dtype, device='cuda'))


@pytest.mark.parametrize('kwargs', [{'p': 0}, {'p': 4}, {'p': 12}, {'p': 256}, {'threads': 0},
                                    {'threads': 192}, {'threads': 1024}, {'csr_mode': 3}])
def test_invalid_launch_parameters(kwargs):
    m, rl, cl = _example()
    boo = _build(m, rl, cl).to('cuda')
    with pytest.raises(ValueError):
        S.boo_matmul(boo, _x((11, 17)).cuda(), **kwargs)


def test_rowseg_rejects_column_major():
    m, rl, cl = _example()
    boo = _build(m, rl, cl, order='colmajor').to('cuda')
    with pytest.raises(ValueError, match='rowmajor'):
        S.boo_matmul(boo, _x((11, 17)).cuda(), row_seg=True)


def test_execution_plan_contract():
    m, rl, cl = _example()
    boo = _build(m, rl, cl).to('cuda')
    plan = S.prepare_boo_cuda(boo)
    x = _x((11, 17)).cuda()
    check(S.boo_matmul(boo, x, launch_mode='auto', execution_plan=plan), m, x)
    with pytest.raises(ValueError):
        S.boo_matmul(boo, x, execution_plan=plan)          # legacy launch mode


def test_split_row_groups_and_long_remainder_rows(monkeypatch, path):
    """Heavy row groups cut into several items (partial sums + fixup pass) and
    long remainder rows (split-row pass), forced with small thresholds."""
    monkeypatch.setattr(SB, 'MAX_ITEM_NNZ', 64)
    monkeypatch.setattr(SB, 'LONG_ROW_THRESHOLD', 8)
    rng = np.random.default_rng(5)
    # ~10 random entries per 32x32 tile (spilled at threshold 40); row 7 dense
    # (its tiles reach ~42 and are kept: a row group of ~900 block entries,
    # split at 64); row 300 on every 2nd column (~26 per tile: spilled, so a
    # ~360-entry remainder row).
    A = sp.random(500, 700, density=0.01, format='csr', random_state=3, dtype=np.float32)
    extra = sp.lil_matrix((500, 700), dtype=np.float32)
    extra[7, :] = 1.0
    extra[300, ::2] = -2.0
    A = (A + extra.tocsr()).tocsr()
    A.data = rng.standard_normal(A.nnz).astype(np.float32)
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32,
                       small_block_threshold=40).to('cuda')
    d = boo._gpu_meta.desc
    if path == 'tile':
        assert d['n_splits'] > 0 and d['n_long'] > 0
    else:   # the same rows as chunked gather rows
        assert d['n_gtask'] >= d['n_crow_long'] > 0
    for K in (64, 5, 128):
        x = _x((3, 700, K)).cuda()
        check(S.boo_matmul(boo, x), A, x)


def test_skewed_gather_rows_as_chunk_tasks(path):
    """Power-law-like gather rows at the default thresholds: the rows of 40-200
    entries among rows of ~3 go to chunk tasks (the stage's skewed rule)."""
    rng = np.random.default_rng(11)
    A = sp.random(2000, 20000, density=0.00015, format='lil', random_state=4, dtype=np.float32)
    for r in rng.choice(2000, 60, replace=False):
        A[r, rng.choice(20000, int(rng.integers(40, 200)), replace=False)] = 1.0
    A = A.tocsr()
    A.data = rng.standard_normal(A.nnz).astype(np.float32)
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32).to('cuda')
    d = boo._gpu_meta.desc
    if path == 'gather':
        assert d['n_crow_long'] == int((np.diff(A.indptr) > 32).sum()) >= 60 and d['n_gtask'] >= d['n_crow_long']
    for K in (32, 128, 5):
        x = _x((2, 20000, K)).cuda()
        check(S.boo_matmul(boo, x), A, x)


@pytest.mark.parametrize('cfg', [1, 2])
def test_benchmark_configs_full_size(cfg):
    from spmm_amd import matrices as M
    A, spec = M.make_config(cfg)
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32).to('cuda')
    x = torch.from_numpy(M.dense_x(A.shape[1], spec['K'])).cuda()
    y = S.boo_matmul(boo, x)
    check(y, A, x)
    # size-independent: linearity in X and determinism (no atomics)
    x2 = torch.from_numpy(M.dense_x(A.shape[1], spec['K'], seed=1)).cuda()
    assert torch.equal(S.boo_matmul(boo, x), y)
    lin = S.boo_matmul(boo, x + x2) - y - S.boo_matmul(boo, x2)
    bound = torch.from_numpy(abs(A) @ (np.abs(x.cpu().numpy()) + np.abs(x2.cpu().numpy()))).cuda()
    assert torch.all(lin.abs() <= 3e-5 * bound)


@pytest.mark.parametrize('K', [1, 5, 32, 64, 128, 256, 300])
@pytest.mark.parametrize('dtype', [torch.float32, torch.float64])
def test_scattered_columns_take_the_gather_pass(K, dtype, monkeypatch):
    from spmm_amd import matrices as M
    monkeypatch.setattr(SB, 'MIN_COL_REUSE', 1.5)      # the default
    np_dtype = np.float32 if dtype == torch.float32 else np.float64
    A = M.permuted(M.stencil_27pt(16, dtype=np_dtype), seed=1)
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32).to('cuda')
    assert boo._gpu_meta.desc['n_crow'] > 0.9 * A.shape[0]
    x = _x((2, A.shape[1], K), dtype).cuda()
    check(S.boo_matmul(boo, x), A, x)


@pytest.mark.parametrize('which', ['rmat', 'permuted_stencil'])
def test_scaled_down_power_law_and_permuted_configs(which, monkeypatch):
    """Configs 4 and 5 at reduced size: heavy slices split into items, long
    remainder rows, scattered slices in the gather pass, all at once."""
    from spmm_amd import matrices as M
    monkeypatch.setattr(SB, 'MIN_COL_REUSE', 1.5)
    if which == 'rmat':
        A, K = M.rmat(14, 16), 128
    else:
        A, K = M.permuted(M.stencil_27pt(32)), 32
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32).to('cuda')
    d = boo._gpu_meta.desc
    assert d['n_crow'] > 0
    x = torch.from_numpy(M.dense_x(A.shape[1], K)).cuda()
    y = S.boo_matmul(boo, x)
    check(y, A, x)
    assert torch.equal(S.boo_matmul(boo, x), y)


def _permuted_path(n, seed=3):
    T = sp.diags([-np.ones(n - 1), 2 * np.ones(n), -np.ones(n - 1)], [-1, 0, 1], format='csr',
                 dtype=np.float32)
    p = np.random.default_rng(seed).permutation(n)
    return T[p][:, p].tocsr()


def _permuted_laplacian_2d(m, seed=4):
    I = sp.identity(m, format='csr', dtype=np.float32)
    L1 = sp.diags([-np.ones(m - 1), 2 * np.ones(m), -np.ones(m - 1)], [-1, 0, 1], format='csr',
                  dtype=np.float32)
    L = (sp.kron(L1, I) + sp.kron(I, L1)).tocsr()
    p = np.random.default_rng(seed).permutation(L.shape[0])
    return L[p][:, p].tocsr()


@pytest.mark.parametrize('which', ['path_200000', 'laplacian_2d_448'])
@pytest.mark.parametrize('K', [16, 64])
def test_reordered_gather_rows(which, K, monkeypatch):
    """Gather rows walked in breadth-first (Cuthill-McKee) order, not row
    order: the stage reorders them when that keeps the X rows they read close.
    The whole Y against the fp64 product, and a second call bit-equal."""
    monkeypatch.setattr(SB, 'MIN_COL_REUSE', 1.5)
    A = _permuted_path(200_000) if which == 'path_200000' else _permuted_laplacian_2d(448)
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32).to('cuda')
    d = boo._gpu_meta.desc
    n_short = d['n_crow'] - d['n_crow_long']
    assert n_short > 0.9 * A.shape[0]
    cid = boo._gpu_meta.stage.crow_id[:n_short].cpu().numpy()
    assert not np.all(np.diff(cid) > 0), 'the stage kept row order: the reorder did not fire'
    x = _x((1, A.shape[1], K)).cuda()
    y = S.boo_matmul(boo, x)
    check(y, A, x)
    assert torch.equal(S.boo_matmul(boo, x), y)


@pytest.mark.parametrize('K', [4, 32, 130])
def test_long_gather_rows_in_chunks(K, monkeypatch):
    monkeypatch.setattr(SB, 'MIN_COL_REUSE', 1.5)
    rng = np.random.default_rng(5)
    A = sp.random(600, 5000, density=0.002, format='lil', random_state=3, dtype=np.float32)
    for r, n in ((7, 3000), (300, 1500), (599, 300)):
        A[r, rng.choice(5000, n, replace=False)] = rng.standard_normal(n).astype(np.float32)
    A = A.tocsr()
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32).to('cuda')
    d = boo._gpu_meta.desc
    assert d['n_crow_long'] == 3 and d['n_gtask'] == 6
    x = _x((2, 5000, K)).cuda()
    y = S.boo_matmul(boo, x)
    check(y, A, x)
    assert torch.equal(S.boo_matmul(boo, x), y)


@pytest.mark.parametrize('target', [8, 16, 32])
@pytest.mark.parametrize('shape', [(256, 256), (192, 320)])
def test_hem_clustered_product(target, shape):
    """The reference's default clustering (cluster='hem'): non-trivial row and
    column permutations inside every group."""
    rng = np.random.default_rng(0)
    A = sp.random(*shape, density=0.05, format='csr', random_state=0, dtype=np.float32)
    A.data = rng.standard_normal(A.nnz).astype(np.float32)
    boo = S.csr_to_boo(A, target_nr=target, target_nc=target).to('cuda')
    x = _x((2, shape[1], 33)).cuda()
    check(S.boo_matmul(boo, x), A, x)


def test_hot_column_tasks_first(path):
    """A power-law graph's long gather rows: the chunk tasks over their most
    used columns are launched first (gtask_order).  The product is within the
    bound, and the same staging run in task order gives the same Y bit for
    bit: each row's partial rows are added in task order either way."""
    from spmm_amd import matrices as M
    from spmm_amd._native import core
    A = M.rmat(scale=17, edge_factor=8, seed=3)
    K, B = 64, 2
    x = torch.from_numpy(np.random.default_rng(1).standard_normal((B, A.shape[1], K)).astype(np.float32)).cuda()
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32).to('cuda')
    y = S.boo_matmul(boo, x)
    for b in range(B):
        check(y[b], A, x[b])
    desc = boo._gpu_meta.desc
    if path == 'gather':
        assert desc['gtask_order'] != 0
    if desc['gtask_order']:
        plain = dict(desc, gtask_order=0)
        y2 = torch.empty_like(y)
        wsb = int(core.boo_workspace_bytes(plain, 0, B, K))
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device='cuda')
        core.boo_matmul_gpu(plain, 0, int(x.data_ptr()), int(y2.data_ptr()), B, K, int(ws.data_ptr()), wsb,
                            int(torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        assert torch.equal(y, y2)


def test_hot_split_edge_rows(path):
    """Long rows all in hot columns, all in cold ones, both, and one longer
    than a chunk task on both sides (tests/test_boo_stage.py's matrix): within
    the bound, and bit-equal to the same staging run in task order."""
    from test_boo_stage import _hot_edge_matrix
    from spmm_amd._native import core
    A = _hot_edge_matrix()
    K = 64
    x = torch.from_numpy(np.random.default_rng(2).standard_normal((A.shape[1], K)).astype(np.float32)).cuda()
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32).to('cuda')
    y = S.boo_matmul(boo, x)
    check(y, A, x)
    desc = boo._gpu_meta.desc
    if path == 'gather':
        assert desc['gtask_order'] != 0
    if desc['gtask_order']:
        plain = dict(desc, gtask_order=0)
        y2 = torch.empty_like(y)
        wsb = int(core.boo_workspace_bytes(plain, 0, 1, K))
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device='cuda')
        core.boo_matmul_gpu(plain, 0, int(x.data_ptr()), int(y2.data_ptr()), 1, K, int(ws.data_ptr()), wsb,
                            int(torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        assert torch.equal(y, y2)
