"""Host staging of BOO into the kernel's tile stream (spmm_boo_stage_* in
include/spmm_amd.h): every nonzero of the matrix lands in exactly one tile (or
in a long remainder row), tiles respect their size limits, items and waves
partition the stream.  CPU only."""

import numpy as np
import pytest
import scipy.sparse as sp

import spmm_amd as S
from spmm_amd import _core
from spmm_amd import boo as SB
from spmm_amd import matrices as M


def _host(boo):
    d = boo._d
    i32 = np.int32
    nz_idx, nz_val = d['nz_idx'], d['nz_val']
    if boo.nz_order != SB.BooNzOrder.ROWMAJOR:
        nz_idx, nz_val = SB._rowmajor_copy(d['blk_nz_ptr'], nz_idx, nz_val)
    if boo.tail_nnz():
        rem = SB._merge_tail(boo.rows, d['rem_indptr'], d['rem_col_ind'], d['rem_vals'],
                             d['tail_row'], d['tail_col'], d['tail_val'])
    else:
        rem = (d['rem_indptr'], d['rem_col_ind'], d['rem_vals'])
    c = lambda a, t=i32: np.ascontiguousarray(a, dtype=t)  # noqa: E731
    return {
        'rows': int(boo.rows), 'cols': int(boo.cols), 'n_row_groups': boo.num_row_groups(),
        'n_col_groups': boo.num_col_groups(), 'num_blocks': boo.num_blocks(),
        'row_grp_ptr': c(d['row_grp_ptr']), 'row_ids': c(d['row_ids']),
        'col_grp_ptr': c(d['col_grp_ptr']), 'col_ids': c(d['col_ids']),
        'blk_row_grp': c(d['blk_row_grp']), 'blk_col_grp': c(d['blk_col_grp']),
        'blk_nz_ptr': c(d['blk_nz_ptr']), 'blk_shift': c(d['blk_shift'], np.uint8),
        'nz_idx': c(nz_idx, np.uint16), 'nz_val': np.ascontiguousarray(nz_val),
        'rem_indptr': c(rem[0]), 'rem_col_ind': c(rem[1]), 'rem_vals': np.ascontiguousarray(rem[2]),
    }


def decode(host, st):
    """COO (row, col, val) of everything the stream and the long rows hold."""
    tiles = st['tiles'].reshape(-1, 8)
    rs = st['tile_rs'].reshape(-1, 33)
    R, C, V = [], [], []
    for t, (eo, w1, co, ro, _slot, _, _, _) in enumerate(tiles):
        assert eo % 2 == 0
        nnz, nc, nr = w1 & 0xff, (w1 >> 8) & 0xff, (w1 >> 16) & 0xff
        assert 0 <= nnz <= 128 and 0 <= nc <= 32 and 0 <= nr <= 32
        assert nr > 0 or nnz == 0                      # nr = 0: a padding wave of a workgroup
        r = rs[t]
        assert r[0] == 0 and r[-1] == nnz and np.all(np.diff(r.astype(int)) >= 0)
        assert np.all(r[nr:] == nnz)                   # rows past the slice hold nothing
        lr = np.repeat(np.arange(32), np.diff(r.astype(int)))
        lc = st['ent_col'][eo:eo + nnz].astype(int)
        assert np.all(lc < nc)
        R.append(host['row_ids'][ro + lr])
        C.append(st['tcols'][co + lc])
        V.append(st['ent_val'][eo:eo + nnz])
    cp = st['crow_ptr']
    assert cp[0] == 0 and np.all(np.diff(cp) >= 0) and cp[-1] == len(st['ccol']) == len(st['cval'])
    R.append(np.repeat(st['crow_id'], np.diff(cp)))
    C.append(st['ccol'])
    V.append(st['cval'])
    ip, ci, cv = host['rem_indptr'], host['rem_col_ind'], host['rem_vals']
    for row in st['long_rows']:
        R.append(np.full(ip[row + 1] - ip[row], row))
        C.append(ci[ip[row]:ip[row + 1]])
        V.append(cv[ip[row]:ip[row + 1]])
    return np.concatenate(R), np.concatenate(C), np.concatenate(V)


def check_stream(A, boo, max_item_nnz=4096, long_thr=256, n_waves=64, group=1, min_reuse=0.0):
    host = _host(boo)
    st = _core.boo_stage(host, max_item_nnz, long_thr, n_waves, group, min_reuse)
    r, c, v = decode(host, st)
    # every stored value exactly once (explicit zeros included)
    got = sp.coo_matrix((np.ones_like(v, dtype=np.int64), (r, c)), shape=A.shape).tocsr()
    want = sp.csr_matrix((np.ones(A.nnz, np.int64), A.indices, A.indptr), shape=A.shape)
    assert (got != want).nnz == 0
    B = sp.coo_matrix((v, (r, c)), shape=A.shape).tocsr()
    D = (B - A).tocsr()
    D.eliminate_zeros()
    assert D.nnz == 0                                  # and each with its own value
    # items / waves
    tiles = st['tiles'].reshape(-1, 8)
    last = (tiles[:, 1] >> 24) & 1
    # every Y row is stored exactly once: by the last tile of its slice's
    # first item, or by the gather pass
    owner = tiles[(last == 1) & (tiles[:, 4] == -1)]
    stored = [host['row_ids'][ro:ro + ((w1 >> 16) & 0xff)] for _, w1, _, ro, *_ in owner]
    stored = np.concatenate(stored + [st['crow_id']])
    assert np.array_equal(np.sort(stored), np.arange(A.shape[0]))
    wt = st['wave_tiles']
    if len(tiles) == 0:
        assert st['n_waves'] == 0 and list(wt) == [0]
        return st
    assert wt[0] == 0 and wt[-1] == len(tiles) and np.all(np.diff(wt) > 0)
    assert st['n_waves'] == len(wt) - 1 <= max(n_waves, group) and st['n_waves'] % group == 0
    # waves hold whole items: a wave's stream splits at its storing tiles into
    # runs whose tiles with entries all belong to one slice, and after its
    # last storing tile come only tiles without entries (a member of a long
    # group stores at its own last tile with entries)
    nnz_t = tiles[:, 1] & 0xff
    for w in range(len(wt) - 1):
        idx = np.arange(wt[w], wt[w + 1])
        stores = idx[last[idx] == 1]
        assert len(stores) > 0
        assert np.all(nnz_t[stores[-1] + 1:wt[w + 1]] == 0)
        a = wt[w]
        for e in stores:
            run = np.arange(a, e + 1)
            busy = run[nnz_t[run] > 0]
            assert len(set(tiles[busy, 3].tolist())) <= 1
            a = e + 1
    # the waves of a workgroup walk equal-length streams over the same X tiles
    lens = np.diff(wt).reshape(-1, group)
    assert np.all(lens == lens[:, :1])
    for g0 in range(0, len(wt) - 1, group):
        base = tiles[wt[g0]:wt[g0 + 1]]
        for v in range(1, group):
            other = tiles[wt[g0 + v]:wt[g0 + v + 1]]
            assert np.array_equal(other[:, 2], base[:, 2])                       # same column chunk
            assert np.array_equal((other[:, 1] >> 8) & 0xff, (base[:, 1] >> 8) & 0xff)
    slots = tiles[:, 4]
    assert np.all(slots[last == 1] >= -1)
    sl = st['splits'].reshape(-1, 4)
    assert st['n_slots'] == (sl[:, 3] - sl[:, 2]).sum() if len(sl) else st['n_slots'] == 0
    lens = np.diff(host['rem_indptr'])
    check_long(st, host, long_thr, set(np.nonzero(lens > long_thr)[0].tolist()))
    return st


def gather_threshold(st, long_thr):
    """The gather pass's long-row threshold: long_thr, or at most 32 when the
    gather rows' lengths have a standard deviation above their mean."""
    lens = np.diff(st['crow_ptr']).astype(np.float64)
    if len(lens) and lens.var() > lens.mean() ** 2:
        return min(long_thr, 32)
    return long_thr


def check_long(st, host, long_thr, long_rem):
    """Long remainder rows: listed for the split-row pass if their slice is
    in the tile stream, else whole rows of the gather pass.  Gather rows longer
    than the gather threshold come last, cut into contiguous chunk tasks."""
    listed = set(st['long_rows'].tolist())
    gathered = set(st['crow_id'].tolist())
    assert listed <= long_rem and long_rem <= listed | gathered and not (listed & gathered)
    cp, n_long = st['crow_ptr'], st['n_crow_long']
    n_short = len(st['crow_id']) - n_long
    thr = gather_threshold(st, long_thr)
    assert np.all(np.diff(cp)[:n_short] <= thr) and np.all(np.diff(cp)[n_short:] > thr)
    gt, gp = st['gtask'].reshape(-1, 2), st['gtask_ptr']
    assert len(gp) == n_long + 1 and gp[0] == 0 and gp[-1] == len(gt)
    for i in range(n_long):
        t = gt[gp[i]:gp[i + 1]]
        assert t[0, 0] == cp[n_short + i] and t[-1, 1] == cp[n_short + i + 1]
        assert np.all(t[1:, 0] == t[:-1, 1]) and np.all(t[:, 1] - t[:, 0] <= 1024) and np.all(t[:, 1] > t[:, 0])


@pytest.mark.parametrize('policy', ['keep', 'remainder', 'tail_batch'])
@pytest.mark.parametrize('order', ['rowmajor', 'colmajor'])
@pytest.mark.parametrize('group', [1, 2, 4])
@pytest.mark.parametrize('min_reuse', [0.0, 1.5])
def test_stream_covers_every_entry(policy, order, group, min_reuse):
    A = sp.random(300, 260, density=0.05, format='lil', random_state=7, dtype=np.float32)
    A[:40] = 0.0                        # a few empty slices
    A = A.tocsr()
    A.eliminate_zeros()
    boo = S.csr_to_boo(A, cluster='random', target_nr=16, target_nc=24, small_block_policy=policy,
                       nz_order=order, seed=3)
    check_stream(A, boo, group=group, min_reuse=min_reuse)


@pytest.mark.parametrize('nr,nc', [(32, 32), (64, 64), (8, 100), (100, 8)])
@pytest.mark.parametrize('group', [1, 4])
def test_stream_cuts_wide_and_tall_groups(nr, nc, group):
    A = sp.random(400, 500, density=0.08, format='csr', random_state=1, dtype=np.float64)
    boo = S.csr_to_boo(A, cluster='identity', target_nr=nr, target_nc=nc)
    st = check_stream(A, boo, group=group)
    assert st['ent_val'].dtype == np.float64


def test_stream_dense_block_is_cut_between_rows():
    A = sp.csr_matrix(np.arange(1, 32 * 32 + 1, dtype=np.float32).reshape(32, 32))
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32)
    st = check_stream(A, boo)
    tiles = st['tiles'].reshape(-1, 8)
    # 96 entries per tile at most: 3 whole rows of 32, the last tile 2 rows
    assert len(tiles) == 11 and np.all(tiles[:-1, 1] & 0xff == 96) and tiles[-1, 1] & 0xff == 64


def test_stream_cuts_inside_a_row_longer_than_a_tile():
    """Duplicate entries can give one row of one block more entries than a
    tile holds; the row is cut inside, its parts in consecutive tiles of the
    same item, and no tile exceeds 96 entries."""
    n_dup = 250
    rows = np.r_[np.zeros(n_dup, int), np.arange(1, 40)]
    cols = np.r_[np.full(n_dup, 3), np.arange(1, 40) % 37]
    vals = np.arange(1, rows.size + 1, dtype=np.float32)
    order = np.lexsort((cols, rows))      # CSR built directly: the duplicates stay separate entries
    A = sp.csr_matrix((vals[order], cols[order], np.r_[0, np.cumsum(np.bincount(rows, minlength=40))]),
                      shape=(40, 40))
    assert A.nnz == rows.size
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32)
    for group in (1, 4):
        st = check_stream(A, boo, group=group)
        nnz = st['tiles'].reshape(-1, 8)[:, 1] & 0xff
        assert nnz.max() <= 96 and nnz.sum() >= n_dup


def test_stream_splits_heavy_items_and_long_rows():
    A = sp.random(200, 3000, density=0.0005, format='lil', random_state=2, dtype=np.float32)
    A[5, :] = 0.0
    A[5, ::37] = 1.0                   # one entry per 32-column block: all remainder
    A = A.tocsr()
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32)
    for group in (1, 4):
        st = check_stream(A, boo, max_item_nnz=10, long_thr=40, group=group)
        assert st['n_slots'] > 0 and len(st['long_rows']) > 0


def test_stream_empty_rows_get_a_tile():
    A = sp.csr_matrix((70, 50), dtype=np.float32)
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32)
    host = _host(boo)
    st = _core.boo_stage(host, 4096, 256, 8, 1)
    tiles = st['tiles'].reshape(-1, 8)
    assert len(tiles) == 3 and np.all(tiles[:, 1] & 0xff == 0)   # 70 rows -> 3 slices
    assert len(st['crow_id']) == 0


def test_gather_pass_takes_empty_and_scattered_slices():
    # empty slices: rows with no entries, stored as zeros by the gather pass
    A = sp.csr_matrix((70, 50), dtype=np.float32)
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32)
    st = check_stream(A, boo, min_reuse=1.5)
    assert len(st['tiles']) == 0 and sorted(st['crow_id']) == list(range(70))
    assert np.all(np.diff(st['crow_ptr']) == 0)
    # a permuted stencil: every slice's columns are scattered (each used ~once)
    Ap = M.permuted(M.stencil_27pt(16), seed=1)
    boo = S.csr_to_boo(Ap, cluster='identity', target_nr=32, target_nc=32)
    st = check_stream(Ap, boo, min_reuse=1.5, group=4)
    assert len(st['crow_id']) > 0.9 * Ap.shape[0]
    # the same matrix unpermuted keeps its slices in the tile stream
    As = M.stencil_27pt(8)
    boo = S.csr_to_boo(As, cluster='identity', target_nr=32, target_nc=32)
    st = check_stream(As, boo, min_reuse=1.5, group=4)
    assert len(st['crow_id']) == 0


def test_stream_config2_counts():
    A, _ = M.make_config(2)
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32)
    host = _host(boo)
    st = _core.boo_stage(host, 4096, 256, 2048, 1)
    tiles = st['tiles'].reshape(-1, 8)
    nnz = tiles[:, 1] & 0xff
    assert nnz.sum() == A.nnz and len(st['long_rows']) == 0
    # 72,200 block tiles + one remainder tile per row group (8,192)
    assert len(tiles) == 72200 + 8192
    assert 2000 <= st['n_waves'] <= 2048 and st['n_slots'] == 0
    # grouped by 4: the 27-point stencil's row groups share column groups, so
    # a group of 4 loads far fewer X tiles than 4 separate row groups
    st4 = _core.boo_stage(host, 4096, 256, 4096, 4, 1.5)
    assert len(st4['crow_id']) == 0         # reuse ~2.9 per column: all slices stay tiles
    t4 = st4['tiles'].reshape(-1, 8)
    assert (t4[:, 1] & 0xff).sum() == A.nnz
    steps = len(t4) // 4
    assert steps < 0.55 * len(tiles)
    # each XCD (an eighth of the workgroups, in launch order) gets a share of
    # near-equal cost, dealt round-robin: every workgroup holds two groups
    # of at most ~26 steps
    lens = np.diff(st4['wave_tiles'])[::4]
    per = (len(lens) + 7) // 8
    xcd = np.array([lens[i:i + per].sum() for i in range(0, len(lens), per)])
    assert xcd.max() <= 1.03 * xcd.mean() and lens.max() <= 52


def test_stream_rejects_unsorted_blocks():
    A = sp.random(64, 64, density=0.2, format='csr', random_state=0, dtype=np.float32)
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32)
    host = _host(boo)
    host['blk_row_grp'] = host['blk_row_grp'][::-1].copy()
    with pytest.raises(ValueError, match='sorted'):
        _core.boo_stage(host, 4096, 256, 8)


def test_stream_rejects_bad_group():
    A = sp.random(64, 64, density=0.2, format='csr', random_state=0, dtype=np.float32)
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32)
    host = _host(boo)
    for g in (0, 3, 8):
        with pytest.raises(ValueError, match='group'):
            _core.boo_stage(host, 4096, 256, 8, g)


def test_gather_pass_long_rows_are_chunked():
    # scattered columns everywhere, a few rows far longer than the threshold
    rng = np.random.default_rng(5)
    A = sp.random(600, 5000, density=0.002, format='lil', random_state=3, dtype=np.float32)
    for r, n in ((7, 3000), (300, 1500), (599, 300)):
        A[r, rng.choice(5000, n, replace=False)] = 1.0
    A = A.tocsr()
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32)
    st = check_stream(A, boo, long_thr=256, min_reuse=1.5, group=4)
    assert st['n_crow_long'] == 3 and len(st['gtask']) // 2 == 3 + 2 + 1


def test_gather_pass_skewed_rows_chunk_earlier():
    # power-law-like rows (a few of 40-200 entries among rows of ~3): the rows
    # above 32 entries become chunk tasks although the threshold is 256
    rng = np.random.default_rng(11)
    A = sp.random(2000, 20000, density=0.00015, format='lil', random_state=4, dtype=np.float32)
    mid = rng.choice(2000, 60, replace=False)
    for r in mid:
        A[r, rng.choice(20000, int(rng.integers(40, 200)), replace=False)] = 1.0
    A = A.tocsr()
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32)
    st = check_stream(A, boo, long_thr=256, min_reuse=1.5, group=4)
    lens = np.diff(st['crow_ptr'])
    assert lens.var() > lens.mean() ** 2
    assert st['n_crow_long'] == int((np.diff(A.indptr) > 32).sum()) >= 60
    # even rows of 48 entries: the threshold stays at 256, nothing is chunked
    n, d = 3000, 48
    cols = np.stack([rng.choice(20000, d, replace=False) for _ in range(n)]).ravel().astype(np.int32)
    E = sp.csr_matrix((np.ones(n * d, np.float32), cols, np.arange(0, n * d + 1, d)), shape=(n, 20000))
    boo = S.csr_to_boo(E, cluster='identity', target_nr=32, target_nc=32)
    st = check_stream(E, boo, long_thr=256, min_reuse=1.5, group=4)
    assert len(st['crow_id']) == n and st['n_crow_long'] == 0


def _hot_columns(ccol, n_cols, n_hot):
    """The n_hot most used columns of ccol (ties: lower column first), as a mask."""
    cnt = np.bincount(ccol, minlength=n_cols)
    order = np.lexsort((np.arange(n_cols), -cnt))
    mask = np.zeros(n_cols, bool)
    mask[order[:n_hot]] = True
    return mask


def test_gather_pass_hot_columns_first():
    # R-MAT 2^17: the long gather rows' entries in their 16,384 most used
    # columns become tasks of their own, every one launched before the rest
    A = M.rmat(scale=17, edge_factor=8, seed=3)
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32)
    st = check_stream(A, boo, long_thr=256, min_reuse=1.5, group=4)
    gt = st['gtask'].reshape(-1, 2)
    go = st['gtask_order']
    n_long = st['n_crow_long']
    assert n_long > 1000 and len(go) == len(gt)
    assert np.array_equal(np.sort(go), np.arange(len(gt)))          # a permutation of the tasks
    cp = st['crow_ptr']
    first = cp[len(cp) - 1 - n_long]                                  # the long rows' first entry
    hot = _hot_columns(st['ccol'][first:], A.shape[1], 16384)
    kind = np.array([int(hot[st['ccol'][a:b]].all()) - int((~hot[st['ccol'][a:b]]).all()) for a, b in gt])
    assert np.all(kind != 0)                                          # each task all hot (1) or all cold (-1)
    n_hot = int((kind == 1).sum())
    assert 0 < n_hot < len(gt)
    assert np.all(kind[go[:n_hot]] == 1) and np.all(kind[go[n_hot:]] == -1)
    # inside a row: its hot tasks, then its cold ones, each part in column order
    gp = st['gtask_ptr']
    for i in range(0, n_long, 97):
        k = kind[gp[i]:gp[i + 1]]
        assert np.all(np.diff(k) <= 0)
        a, b = gt[gp[i], 0], gt[gp[i + 1] - 1, 1]
        h = hot[st['ccol'][a:b]]
        assert np.all(np.diff(h.astype(int)) <= 0)
    # the same shape with columns used evenly: no split, tasks in task order
    rng = np.random.default_rng(2)
    n = A.shape[0]
    lens = np.diff(A.indptr)
    cols = np.concatenate([rng.choice(n, int(m), replace=False) for m in lens]).astype(np.int32)
    E = sp.csr_matrix((np.ones(len(cols), np.float32), cols, A.indptr), shape=A.shape)
    E.sort_indices()
    st = check_stream(E, S.csr_to_boo(E, cluster='identity', target_nr=32, target_nc=32), long_thr=256,
                      min_reuse=1.5, group=4)
    assert st['n_crow_long'] > 1000 and len(st['gtask_order']) == 0


def _hot_edge_matrix(seed=0):
    """40,000 x 262,144.  Long rows: 400 over 100 hot columns each (windows
    that cover columns 0-16,383 at least twice), 400 over 50 cold ones, 400
    over 40 hot and 30 cold, and row 3 over 1,500 hot and 900 cold (longer
    than a chunk task on both sides); cold columns (from 131,072 up) are each
    used once, so the 16,384 most used columns are exactly 0-16,383.  The
    other rows hold 3 hot entries."""
    rng = np.random.default_rng(seed)
    n, cols, H = 40000, 1 << 18, 16384
    cold = iter(range(1 << 17, 1 << 18))
    win = iter(range(0, 10 ** 9, 100))
    rows, cc = [], []
    for r in range(n):
        if r == 3:
            c = np.concatenate([rng.choice(H, 1500, replace=False), [next(cold) for _ in range(900)]])
        elif r % 100 == 0:
            w = next(win)
            c = (w + np.arange(100)) % H
        elif r % 100 == 1:
            c = np.array([next(cold) for _ in range(50)])
        elif r % 100 == 2:
            c = np.concatenate([rng.choice(H, 40, replace=False), [next(cold) for _ in range(30)]])
        else:
            c = rng.choice(H, 3, replace=False)
        rows.append(np.full(len(c), r))
        cc.append(np.asarray(c))
    r = np.concatenate(rows)
    c = np.concatenate(cc)
    v = rng.standard_normal(len(r)).astype(np.float32)
    A = sp.csr_matrix((v, (r, c)), shape=(n, cols))
    A.sum_duplicates()
    A.sort_indices()
    return A


def test_gather_pass_hot_split_edge_rows():
    # long rows all in hot columns, all in cold ones, both, and one longer than
    # a chunk task: every task one kind, each row's hot tasks first, the rows'
    # entries unchanged (check_stream), all hot tasks launched first
    A = _hot_edge_matrix()
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32)
    st = check_stream(A, boo, long_thr=256, min_reuse=1.5, group=4)
    gt = st['gtask'].reshape(-1, 2)
    go = st['gtask_order']
    n_long = st['n_crow_long']
    assert n_long == 1201 and len(go) == len(gt)
    cp = st['crow_ptr']
    first = cp[len(cp) - 1 - n_long]
    hot = _hot_columns(st['ccol'][first:], A.shape[1], 16384)
    assert np.array_equal(np.nonzero(hot)[0], np.arange(16384))
    kind = np.array([int(hot[st['ccol'][a:b]].all()) - int((~hot[st['ccol'][a:b]]).all()) for a, b in gt])
    assert np.all(kind != 0)
    n_hot = int((kind == 1).sum())
    assert np.all(kind[go[:n_hot]] == 1) and np.all(kind[go[n_hot:]] == -1)
    gp = st['gtask_ptr']
    row_of = st['crow_id'][len(st['crow_id']) - n_long:]
    kinds = {}
    for i in range(n_long):
        k = kind[gp[i]:gp[i + 1]]
        assert np.all(np.diff(k) <= 0)
        kinds[int(row_of[i]) % 100 if row_of[i] != 3 else 'big'] = (int((k == 1).sum()), int((k == -1).sum()))
    assert kinds[0] == (1, 0) and kinds[1] == (0, 1) and kinds[2] == (1, 1)
    assert kinds['big'][0] >= 2 and kinds['big'][1] >= 1        # cut into chunks on both sides


def test_gather_rows_reordered_when_it_keeps_x_rows_close():
    # A randomly permuted path graph (tridiagonal, 200,000 rows): in row order
    # the rows naming any X row lie ~67,000 rows apart, beyond the staging's
    # 8,192-row window; breadth-first order puts them next to each other, so
    # the short gather rows are walked along the path: almost every row is a
    # graph neighbour of the row before it.
    n = 200_000
    T = sp.diags([-np.ones(n - 1), 2 * np.ones(n), -np.ones(n - 1)], [-1, 0, 1], format='csr',
                 dtype=np.float32)
    p = np.random.default_rng(3).permutation(n)
    A = T[p][:, p].tocsr()
    st = _stage_sparse_checked(A)
    cid = st['crow_id'][:len(st['crow_id']) - st['n_crow_long']]
    assert len(cid) == n and not np.all(np.diff(cid) > 0)
    Ac = A.tocoo()
    edges = Ac.row.astype(np.int64) * n + Ac.col
    adjacent = np.isin(cid[:-1].astype(np.int64) * n + cid[1:], edges)
    assert adjacent.mean() > 0.99
    # uniformly random columns: no order keeps X rows closer, row order stays
    rng = np.random.default_rng(5)
    R = sp.csr_matrix((rng.standard_normal(3 * n).astype(np.float32),
                       (np.repeat(np.arange(n), 3), rng.integers(0, n, 3 * n))), shape=(n, n))
    R.sum_duplicates()
    st = _stage_sparse_checked(R)
    cid = st['crow_id'][:len(st['crow_id']) - st['n_crow_long']]
    assert len(cid) > 0.9 * n and np.all(np.diff(cid) > 0)


def _stage_sparse_checked(A):
    """Stage A (identity 32x32, the GPU path's knobs) and check, without
    densifying, that the stream and gather pass hold A's values exactly."""
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32)
    host = _host(boo)
    st = _core.boo_stage(host, SB.MAX_ITEM_NNZ, SB.LONG_ROW_THRESHOLD, 4096, 4, SB.MIN_COL_REUSE)
    r, c, v = decode(host, st)
    B = sp.coo_matrix((v.astype(np.float64), (r, c)), shape=A.shape).tocsr()
    assert B.nnz == A.nnz and abs(B - A.astype(np.float64)).max() == 0
    assert np.array_equal(np.sort(st['crow_id']), np.unique(st['crow_id']))
    return st


# ---------------------------------------------------------------------------
# record stream (float, group 4): one DMA-able record per wave and step
# ---------------------------------------------------------------------------

def decode_records(st):
    """Walk each wave's records by their own look-ahead links (records 0-3
    from the wave's first words, record k >= 4 from record k - 4's link) and
    return, per wave, the decoded records (dicts).  Independent of the
    kernel: follows the byte layout the staging documents."""
    blobs = st['blobs'].view(np.uint8)
    first = st['blob_first'].reshape(-1, 8)
    out = []
    for w in range(st['n_waves']):
        f = first[w]
        recs = []
        for k in range(int(f[5])):
            if k < 4:
                o, nv = int(f[k]), (int(f[4]) >> (8 * k)) & 0xff
            else:
                o, nv = recs[k - 4]['next_off'], recs[k - 4]['next_nvec']
            rec = blobs[o * 16:(o + nv) * 16]
            h = rec[:16].view(np.uint32)
            w0 = int(h[0])
            d = {'nnz': w0 & 0xff, 'nr': (w0 >> 8) & 63, 'nc': (w0 >> 14) & 63, 'flags': (w0 >> 20) & 15,
                 'slot': int(np.int32(h[1])), 'next_off': int(h[2]), 'next_nvec': w0 >> 24,
                 'rbase': int(h[3]), 'off': o, 'nvec': nv}
            p = 16
            if d['nnz']:
                d['rs'] = rec[p:p + 32].copy()
                p += 32
            nnz = d['nnz']
            d['col'] = rec[p:p + nnz].copy()
            p += (nnz + 3) & ~3
            d['val'] = rec[p:p + 4 * nnz].view(np.float32).copy()
            p += 4 * nnz
            assert (p + 15) // 16 == nv          # the record is exactly its 16-byte count
            recs.append(d)
        out.append(recs)
    return out


@pytest.mark.parametrize('case', ['stencil', 'permuted', 'rmat', 'heavy', 'hem'])
def test_record_stream_matches_tiles(case):
    """The record stream holds exactly the tiles of the tile stream: per wave
    and step its entries, row starts and the slice's rows (first row when
    consecutive, else its offset into row_ids); the X-id stream names the X
    rows each wave stages (2 of the 8 DMA instructions of the step's
    32-column tile); each record's look-ahead link names the record 4 steps
    later (the last one for the stream's final records)."""
    if case == 'stencil':
        A = M.stencil_27pt(16)
    elif case in ('permuted', 'hem'):
        A = M.permuted(M.stencil_27pt(12), seed=3)
    elif case == 'rmat':
        A = M.rmat(12, 8, seed=1)
    else:   # heavy slices: split items with partial slots
        rng = np.random.default_rng(5)
        A = sp.random(96, 96, density=0.9, random_state=rng, format='csr', dtype=np.float32)
    A = sp.csr_matrix(A, dtype=np.float32)
    boo = S.csr_to_boo(A, cluster='hem' if case == 'hem' else 'identity', target_nr=32, target_nc=32)
    host = _host(boo)
    st = _core.boo_stage(host, 512 if case == 'heavy' else 4096, 256, 64, 4, 0.0 if case == 'hem' else 1.5)
    if st['n_waves'] == 0:
        assert st['n_blob16'] == 0
        return
    assert st['n_blob16'] == len(st['blobs']) // 4 > 0
    tiles = st['tiles'].reshape(-1, 8)
    trs = st['tile_rs'].reshape(-1, 33)
    xid = st['blob_xid'].reshape(-1, 8)
    assert len(xid) == len(tiles)
    wt = st['wave_tiles']
    recs = decode_records(st)
    first = st['blob_first'].reshape(-1, 8)
    n_noncontig = 0
    for w in range(st['n_waves']):
        m = w % 4
        t0, t1 = wt[w], wt[w + 1]
        assert len(recs[w]) == t1 - t0 and first[w][6] == t0
        for k, t in enumerate(range(t0, t1)):
            d = recs[w][k]
            eo, w1, co, ro, slot = (int(x) for x in tiles[t][:5])
            nnz, nc, nr, fl = w1 & 0xff, (w1 >> 8) & 0xff, (w1 >> 16) & 0xff, (w1 >> 24) & 0xff
            assert (d['nnz'], d['nr'], d['slot']) == (nnz, nr, slot)
            assert d['flags'] & 1 == fl & 1 and (d['flags'] >> 1) & 1 == (fl >> 1) & 1
            if nnz:
                assert np.array_equal(d['rs'].astype(int), trs[t][:32].astype(int))
            assert np.array_equal(d['col'], st['ent_col'][eo:eo + nnz])
            assert np.array_equal(d['val'], st['ent_val'][eo:eo + nnz])
            # the X rows this wave stages: column 2m + (j >> 2) + 8 (j & 3)
            cols = [min(2 * m + (j >> 2) + 8 * (j & 3), max(nc - 1, 0)) for j in range(8)]
            want = [st['tcols'][co + c] if nc else 0 for c in cols]
            assert list(xid[t]) == want
            rows = host['row_ids'][ro:ro + nr]
            if d['flags'] & 4:
                assert nr > 0 and np.array_equal(rows, d['rbase'] + np.arange(nr))
            else:
                n_noncontig += nr > 0
                assert d['rbase'] == ro
    if case == 'hem':
        assert n_noncontig > 0          # HEM slices' rows are scattered: the row_ids path is staged
    # the 4-step links: past the stream's end they name its last record (the
    # kernel prefetches it again and never uses it); every record lies inside
    # the stream
    blobs16 = len(st['blobs']) // 4
    for w in range(st['n_waves']):
        n = len(recs[w])
        for k in range(n):
            assert recs[w][k]['off'] + recs[w][k]['nvec'] <= blobs16
            nx = recs[w][min(k + 4, n - 1)]
            assert (recs[w][k]['next_off'], recs[w][k]['next_nvec']) == (nx['off'], nx['nvec'])
        for k in range(4):
            assert int(first[w][k]) == recs[w][min(k, n - 1)]['off']


def test_record_stream_absent_for_double_and_small_groups():
    A = sp.csr_matrix(M.stencil_27pt(8), dtype=np.float64)
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32)
    st = _core.boo_stage(_host(boo), 4096, 256, 64, 4, 1.5)
    assert st['n_blob16'] == 0 and len(st['blobs']) == 0
    A32 = sp.csr_matrix(A, dtype=np.float32)
    boo = S.csr_to_boo(A32, cluster='identity', target_nr=32, target_nc=32)
    st = _core.boo_stage(_host(boo), 4096, 256, 64, 1, 1.5)
    assert st['n_blob16'] == 0


def test_stage_rejects_out_of_range_columns():
    """Column ids and remainder columns out of [0, cols), and a decreasing
    remainder row pointer, are errors of the staging call (SPMM_EINVAL ->
    ValueError), never an out-of-range host access."""
    n = 2000
    A = sp.diags([np.ones(n - 1), 2 * np.ones(n), np.ones(n - 1)], [-1, 0, 1], format='csr', dtype=np.float32)
    A = M.permuted(A, seed=1)
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32)
    good = _host(boo)
    _core.boo_stage(good, 4096, 256, 64, 4, 1.5)                 # the unmodified input stages
    assert good['rem_col_ind'].size > 0
    for key, idx, val in (('rem_col_ind', 0, -2 ** 30), ('rem_col_ind', -1, n), ('col_ids', 3, n + 7),
                          ('col_ids', 0, -1)):
        h = dict(good)
        h[key] = good[key].copy()
        h[key][idx] = val
        with pytest.raises(ValueError, match='out of range'):
            _core.boo_stage(h, 4096, 256, 64, 4, 1.5)
    h = dict(good)
    h['rem_indptr'] = good['rem_indptr'].copy()
    r = int(np.nonzero(np.diff(h['rem_indptr']) > 0)[0][0])
    h['rem_indptr'][r + 1] = h['rem_indptr'][r] - 1
    with pytest.raises(ValueError, match='nondecreasing|start'):
        _core.boo_stage(h, 4096, 256, 64, 4, 1.5)
