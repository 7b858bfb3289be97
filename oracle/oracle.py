"""CPU oracle for the SpMM hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module (or anything under oracle/), and only as the checker.
The product (spmm_amd) never imports it and has no CPU fallback through it.

A restatement, in vectorised numpy, of what the reference computes on this
path.  Every function cites the reference routine it follows (paths relative
to the reference root, torch_fast_spdmm/).  It is written independently of
spmm_amd's C++ builders so the two check each other.

How each function is pinned (tests/test_oracle.py):
  identity_labels      closed form arange(n)//target (clustering.py:483-484);
                       caps a no-op for exact tiles (clustering.py:83-121).
  boo_build            the worked example of docs/reference/BOO_FORMAT.md:
                       102-131 (every array); the 7x11 example counts of
                       tests/torch_fast_spdmm/test_boo_edges.py:21-31,53-70;
                       the uint16 endpoint/overflow cases (:186-196,:223-227);
                       the compiled reference (oracle/_ref) array for array on
                       random matrices, all policies and orders; closed-form
                       counts of the stencil configs.
  boo_decode           round trip to the input CSR; compiled reference.
  boo_cpu_matmul       compiled reference bit for bit; fp64 dense product.
  pbr_build            compiled reference after ordering each stripe's blocks
                       by column (the reference's in-stripe order is the
                       iteration order of libstdc++'s std::unordered_map --
                       the third-party dependency on this path, GCC 11.4's
                       libstdc++ here -- which this restatement does not
                       model; tests pin that order against the compiled
                       reference and committed fixtures written from it);
                       closed-form counts of config 2; round trips incl. the
                       partial last stripe (tests/torch_fast_spdmm/
                       test_pbr.py:208-228).
  pbr_decode, pbr_cpu_matmul  compiled reference; fp64 dense product.
  spmm_reference       fp64 product of the ORIGINAL CSR plus the elementwise
                       bound |A|.|X| the tolerance is stated against
                       (tests/torch_fast_spdmm/benchmark/bench_real.py:168-208).
  hem_similarity       (plain loops, small cases) shared-column counts by set
                       intersection, checked against a dense A A^T; top-k
                       and symmetrisation rules spelled out per row.
  hem_pair_hash        the published SplitMix64 output sequence for seed 0
                       (its first outputs 0xe220a8397b1dcdaf,
                       0x6e789e6aa1b965f4) pins the mixing function; symmetry.
  hem_mutual_max       the reference's known answer
                       (tests/torch_fast_spdmm/test_boo_optimization.py:
                       15-29); every returned pair is each other's strict
                       best by (weight, hash); maximality of the round.
  hem_labels           (plain loops) label vectors written by the
                       reference's own clustering.py
                       (tests/golden/make_hem_fixtures.py ->
                       tests/golden/hem_labels.npz, 32 cases incl. caps, hub
                       pruning and top-k); group sizes / nnz within the caps;
                       determinism; test_boo.py:193-235 expectations.
"""

from __future__ import annotations

import numpy as np
import scipy.sparse as sp

__all__ = [
    'identity_labels', 'boo_build', 'boo_decode', 'boo_cpu_matmul', 'pbr_build',
    'pbr_canonical', 'pbr_decode', 'pbr_cpu_matmul', 'spmm_reference', 'within_bound',
    'BOO_FIELDS', 'PBR_FIELDS', 'hem_similarity', 'hem_pair_hash', 'hem_mutual_max',
    'hem_labels',
]

BOO_FIELDS = ('row_grp_ptr', 'row_ids', 'col_grp_ptr', 'col_ids', 'blk_row_grp', 'blk_col_grp',
              'blk_nz_ptr', 'blk_shift', 'nz_idx', 'nz_val', 'rem_indptr', 'rem_col_ind',
              'rem_vals', 'tail_row', 'tail_col', 'tail_val')
PBR_FIELDS = ('block_codes', 'block_coords', 'block_offsets', 'block_data', 'remainder_indptr',
              'remainder_col_ind', 'remainder_data')


# ---------------------------------------------------------------------------
# clustering (identity)
# ---------------------------------------------------------------------------

def identity_labels(n: int, target: int) -> np.ndarray:
    """clustering.py:483-484 then caps (no-op: every tile has <= target
    members) and consecutive relabelling (labels already 0..n_groups-1)."""
    return (np.arange(n, dtype=np.int64) // max(target, 1)).astype(np.int32)


# ---------------------------------------------------------------------------
# BOO
# ---------------------------------------------------------------------------

def _groups(labels: np.ndarray, n_groups: int, itype):
    """boo_matrix.cpp:23-48: counting sort, ids ascending within a group,
    position = rank inside the group."""
    labels = np.asarray(labels, dtype=np.int64)
    counts = np.bincount(labels, minlength=n_groups)
    ptr = np.zeros(n_groups + 1, dtype=np.int64)
    np.cumsum(counts, out=ptr[1:])
    ids = np.argsort(labels, kind='stable')
    pos = np.empty(labels.size, dtype=np.int64)
    pos[ids] = np.arange(labels.size) - ptr[labels[ids]]
    return ptr.astype(itype), ids.astype(itype), pos


def _ceil_log2(n: np.ndarray) -> np.ndarray:
    """boo_matrix.cpp:12-16: the smallest s with 2^s >= n (0 for n <= 1),
    counted exactly in integers."""
    n = np.asarray(n, dtype=np.int64)
    out = np.zeros(n.shape, dtype=np.int64)
    for s in range(63):
        out += (n > (np.int64(1) << s))
    return out


def boo_build(indptr, indices, data, rows: int, cols: int, row_labels, col_labels,
              policy: int = 2, threshold: int = 4, order: int = 0) -> dict:
    """csr_to_boo (boo_matrix.cpp:53-274).

    policy: 0 keep, 2 remainder, 3 tail_batch (1 merge is rejected).
    order: 0 rowmajor, 1 colmajor.  Returns the reference's arrays in its
    dtypes (index type of indptr, value type of data, u8 shifts, u16 idx).
    """
    if policy == 1:
        raise ValueError("csr_to_boo: 'merge' policy is a clustering-level column relabel")
    if policy not in (0, 2, 3):
        raise ValueError('csr_to_boo: unknown small_block_policy')
    if order not in (0, 1):
        raise ValueError('csr_to_boo: unknown nz_order')
    itype = np.asarray(indptr).dtype
    vtype = np.asarray(data).dtype
    indptr = np.asarray(indptr, dtype=np.int64)
    indices = np.asarray(indices, dtype=np.int64)
    data = np.asarray(data)
    rl = np.asarray(row_labels, dtype=np.int64)
    cl = np.asarray(col_labels, dtype=np.int64)
    n_rg = int(rl.max()) + 1 if rows else 0
    n_cg = int(cl.max()) + 1 if cols else 0
    row_grp_ptr, row_ids, row_pos = _groups(rl, n_rg, itype)
    col_grp_ptr, col_ids, col_pos = _groups(cl, n_cg, itype)

    nnz = int(indptr[-1]) if rows else 0
    r = np.repeat(np.arange(rows, dtype=np.int64), np.diff(indptr))
    c = indices[:nnz]
    key = rl[r] * n_cg + cl[c]
    ukeys, counts = np.unique(key, return_counts=True)          # sorted keys
    keep = counts >= threshold if policy in (2, 3) else np.ones(ukeys.size, bool)
    bkeys, bcounts = ukeys[keep], counts[keep]
    b_rg, b_cg = bkeys // max(n_cg, 1), bkeys % max(n_cg, 1)
    rgp = np.asarray(row_grp_ptr, dtype=np.int64)
    cgp = np.asarray(col_grp_ptr, dtype=np.int64)
    n_r = rgp[b_rg + 1] - rgp[b_rg]
    n_c = cgp[b_cg + 1] - cgp[b_cg]
    shift = _ceil_log2(n_c)
    span = ((n_r - 1) << shift) + (n_c - 1)
    if np.any(span > 0xFFFF):
        raise ValueError('csr_to_boo: block local index space exceeds uint16')
    blk_nz_ptr = np.zeros(bkeys.size + 1, dtype=np.int64)
    np.cumsum(bcounts, out=blk_nz_ptr[1:])

    blk = np.searchsorted(bkeys, key)
    in_blk = np.zeros(nnz, dtype=bool)
    if bkeys.size:
        in_blk = bkeys[np.minimum(blk, bkeys.size - 1)] == key
    pos = np.arange(nnz)
    # entries in blocks: (block, order key, CSR position)
    e = pos[in_blk]
    eb = blk[in_blk]
    lrow = row_pos[r[e]]
    lcol = col_pos[c[e]]
    sh = shift[eb]
    idx = (lrow << sh) | lcol
    okey = idx if order == 0 else ((lcol << 16) | lrow)
    perm = np.lexsort((e, okey, eb))
    nz_idx = idx[perm].astype(np.uint16)
    nz_val = data[e[perm]].astype(vtype)

    # entries outside kept blocks
    o = pos[~in_blk]
    if policy == 3:
        tail_row, tail_col, tail_val = r[o], c[o], data[o]
        rem_indptr = np.zeros(rows + 1, dtype=np.int64)
        rem_col, rem_val = np.zeros(0, np.int64), np.zeros(0, vtype)
    else:
        tail_row = tail_col = np.zeros(0, np.int64)
        tail_val = np.zeros(0, vtype)
        rp = np.lexsort((data[o], c[o], r[o]))          # per row by (col, value)
        rem_col, rem_val = c[o][rp], data[o][rp]
        rem_indptr = np.zeros(rows + 1, dtype=np.int64)
        np.cumsum(np.bincount(r[o], minlength=rows), out=rem_indptr[1:])

    return dict(
        rows=rows, cols=cols, total_nnz=nnz,
        row_grp_ptr=row_grp_ptr, row_ids=row_ids, col_grp_ptr=col_grp_ptr, col_ids=col_ids,
        blk_row_grp=b_rg.astype(itype), blk_col_grp=b_cg.astype(itype),
        blk_nz_ptr=blk_nz_ptr.astype(itype), blk_shift=shift.astype(np.uint8),
        nz_idx=nz_idx, nz_val=nz_val,
        rem_indptr=rem_indptr.astype(itype), rem_col_ind=rem_col.astype(itype),
        rem_vals=rem_val.astype(vtype), tail_row=tail_row.astype(itype),
        tail_col=tail_col.astype(itype), tail_val=tail_val.astype(vtype),
        max_nr=int(n_r.max()) if n_r.size else 0, max_nc=int(n_c.max()) if n_c.size else 0,
        max_nnz_blk=int(bcounts.max()) if bcounts.size else 0, nz_order=order)


def _boo_entries(b: dict):
    """(global row, global col, value) of every block entry, in array order."""
    nzp = np.asarray(b['blk_nz_ptr'], dtype=np.int64)
    nb = nzp.size - 1
    blk = np.repeat(np.arange(nb), np.diff(nzp))
    sh = np.asarray(b['blk_shift'], dtype=np.int64)[blk]
    idx = np.asarray(b['nz_idx'], dtype=np.int64)
    rbase = np.asarray(b['row_grp_ptr'], dtype=np.int64)[np.asarray(b['blk_row_grp'], dtype=np.int64)[blk]]
    cbase = np.asarray(b['col_grp_ptr'], dtype=np.int64)[np.asarray(b['blk_col_grp'], dtype=np.int64)[blk]]
    gr = np.asarray(b['row_ids'], dtype=np.int64)[rbase + (idx >> sh)]
    gc = np.asarray(b['col_ids'], dtype=np.int64)[cbase + (idx & ((1 << sh) - 1))]
    return gr, gc, np.asarray(b['nz_val'])


def boo_decode(b: dict) -> sp.csr_matrix:
    """boo_to_csr (boo_matrix.cpp:277-333): all entries, each row sorted by
    (column, value)."""
    rows, cols = b['rows'], b['cols']
    gr, gc, gv = _boo_entries(b)
    ri = np.asarray(b['rem_indptr'], dtype=np.int64)
    rr = np.repeat(np.arange(rows), np.diff(ri))
    r = np.concatenate([gr, rr, np.asarray(b['tail_row'], dtype=np.int64)])
    c = np.concatenate([gc, np.asarray(b['rem_col_ind'], dtype=np.int64),
                        np.asarray(b['tail_col'], dtype=np.int64)])
    v = np.concatenate([gv, np.asarray(b['rem_vals']), np.asarray(b['tail_val'])])
    o = np.lexsort((v, c, r))
    indptr = np.zeros(rows + 1, dtype=np.int64)
    np.cumsum(np.bincount(r, minlength=rows), out=indptr[1:])
    return sp.csr_matrix((v[o], c[o], indptr), shape=(rows, cols))


def _ordered_axpy(y: np.ndarray, rows, cols, vals, x: np.ndarray):
    """y[rows[k]] += vals[k] * x[cols[k]] for k in order, each update rounded
    in y's dtype as a separate multiply then add (the reference's CPU loops
    are `yrow[f] += v * xrow[f]`, compiled without FMA contraction)."""
    for k in range(len(vals)):
        y[rows[k]] += vals[k] * x[cols[k]]


def boo_cpu_matmul(b: dict, x: np.ndarray) -> np.ndarray:
    """boo_batched_matmul_cpu (boo_matrix.cpp:336-396): blocks in array order,
    entries in order, then remainder rows, then the tail."""
    x3 = x[None] if x.ndim == 2 else x
    y = np.zeros((x3.shape[0], b['rows'], x3.shape[2]), dtype=x3.dtype)
    gr, gc, gv = _boo_entries(b)
    ri = np.asarray(b['rem_indptr'], dtype=np.int64)
    rr = np.repeat(np.arange(b['rows']), np.diff(ri))
    for bi in range(x3.shape[0]):
        _ordered_axpy(y[bi], gr, gc, gv, x3[bi])
        _ordered_axpy(y[bi], rr, np.asarray(b['rem_col_ind'], dtype=np.int64),
                      np.asarray(b['rem_vals']), x3[bi])
        _ordered_axpy(y[bi], np.asarray(b['tail_row'], dtype=np.int64),
                      np.asarray(b['tail_col'], dtype=np.int64), np.asarray(b['tail_val']), x3[bi])
    return y[0] if x.ndim == 2 else y


# ---------------------------------------------------------------------------
# PBR
# ---------------------------------------------------------------------------

def pbr_build(indptr, indices, data, rows: int, cols: int, block_rows: int = 8,
              block_cols: int = 8, min_nnz: int = 4) -> dict:
    """csr_to_pbr (pbr_matrix.cpp:333-448) with each stripe's blocks in
    ascending block-column order (the reference's order is its hash map's;
    see pbr_canonical).  Per block: bit (r%BR)*BC + c%BC of each entry; values
    in CSR order; kept iff popcount >= min_nnz (uint8).  A spilled block pairs
    its k-th set bit (row-major) with its k-th value into the remainder, whose
    rows are then sorted by (column, value)."""
    itype = np.asarray(indptr).dtype
    vtype = np.asarray(data).dtype
    indptr = np.asarray(indptr, dtype=np.int64)
    indices = np.asarray(indices, dtype=np.int64)
    data = np.asarray(data)
    nnz = int(indptr[-1]) if rows else 0
    r = np.repeat(np.arange(rows, dtype=np.int64), np.diff(indptr))
    c = indices[:nnz]
    ncb = (cols + block_cols - 1) // block_cols
    brow, bcol = r // block_rows, c // block_cols
    bit = (r % block_rows) * block_cols + (c % block_cols)
    key = brow * ncb + bcol
    order = np.lexsort((np.arange(nnz), key))          # by block, CSR order inside
    k_sorted = key[order]
    ukeys, start, counts = np.unique(k_sorted, return_index=True, return_counts=True)
    blk_of = np.repeat(np.arange(ukeys.size), counts)
    codes = np.zeros(ukeys.size, dtype=np.uint64)
    np.bitwise_or.at(codes, blk_of, np.left_shift(np.uint64(1), bit[order].astype(np.uint64)))
    pop = np.array([bin(int(v)).count('1') for v in codes], dtype=np.int64)
    kept = pop >= (min_nnz & 0xFF)
    # kept blocks: values in CSR order (all of them, duplicates included),
    # offsets advance by popcount
    kb = np.flatnonzero(kept)
    seg = [order[start[i]:start[i] + counts[i]] for i in kb]
    block_data = data[np.concatenate(seg)] if seg else np.zeros(0, vtype)
    offsets = np.zeros(kb.size + 1, dtype=np.int64)
    np.cumsum(pop[kb], out=offsets[1:])
    coords = np.stack([(ukeys[kb] // max(ncb, 1)) * block_rows,
                       (ukeys[kb] % max(ncb, 1)) * block_cols], axis=1).reshape(-1)
    # spilled blocks -> remainder
    rr, rc, rv = [], [], []
    for i in np.flatnonzero(~kept):
        vals = data[order[start[i]:start[i] + counts[i]]]
        code = int(codes[i])
        r0 = (int(ukeys[i]) // ncb) * block_rows
        c0 = (int(ukeys[i]) % ncb) * block_cols
        k = 0
        for p in range(block_rows * block_cols):
            if (code >> p) & 1:
                rr.append(r0 + p // block_cols)
                rc.append(c0 + p % block_cols)
                rv.append(vals[k])
                k += 1
    rr = np.asarray(rr, dtype=np.int64)
    rc = np.asarray(rc, dtype=np.int64)
    rv = np.asarray(rv, dtype=vtype)
    o = np.lexsort((rv, rc, rr))
    rem_indptr = np.zeros(rows + 1, dtype=np.int64)
    np.cumsum(np.bincount(rr, minlength=rows), out=rem_indptr[1:])
    return dict(rows=rows, cols=cols, block_rows=block_rows, block_cols=block_cols,
                total_nnz=nnz, block_codes=codes[kb], block_coords=coords.astype(itype),
                block_offsets=offsets.astype(itype), block_data=block_data.astype(vtype),
                remainder_indptr=rem_indptr.astype(itype), remainder_col_ind=rc[o].astype(itype),
                remainder_data=rv[o])


def pbr_canonical(p: dict) -> dict:
    """The same PBR with each stripe's blocks sorted by block column (data
    segments and offsets permuted with them).  Every other field unchanged."""
    coords = np.asarray(p['block_coords'], dtype=np.int64).reshape(-1, 2)
    offs = np.asarray(p['block_offsets'], dtype=np.int64)
    nb = coords.shape[0]
    perm = np.lexsort((coords[:, 1], coords[:, 0]))
    lens = np.diff(offs)
    data = np.asarray(p['block_data'])
    # data segments are contiguous per block only when values == popcount
    # (no duplicate entries); that is the case every caller uses.
    segs = [data[offs[i]:offs[i + 1]] for i in perm]
    out = dict(p)
    out['block_codes'] = np.asarray(p['block_codes'])[perm]
    out['block_coords'] = coords[perm].reshape(-1).astype(np.asarray(p['block_coords']).dtype)
    new_offs = np.zeros(nb + 1, dtype=np.int64)
    np.cumsum(lens[perm], out=new_offs[1:])
    out['block_offsets'] = new_offs.astype(np.asarray(p['block_offsets']).dtype)
    out['block_data'] = np.concatenate(segs) if segs else data[:0]
    return out


def _pbr_entries(p: dict):
    """Entries of the kept blocks in the reference's consumption order: blocks
    in array order, bits row-major, values taken sequentially
    (pbr_matrix.cpp:38-56, 292-313); positions past the matrix edge skipped."""
    br, bc = p['block_rows'], p['block_cols']
    coords = np.asarray(p['block_coords'], dtype=np.int64).reshape(-1, 2)
    codes = np.asarray(p['block_codes'], dtype=np.uint64)
    rows, cols = p['rows'], p['cols']
    gr, gc = [], []
    for code, (r0, c0) in zip(codes, coords):
        code = int(code)
        for rr in range(br):
            for cc in range(bc):
                if r0 + rr >= rows or c0 + cc >= cols:
                    continue
                if (code >> (rr * bc + cc)) & 1:
                    gr.append(r0 + rr)
                    gc.append(c0 + cc)
    n = len(gr)
    return (np.asarray(gr, dtype=np.int64), np.asarray(gc, dtype=np.int64),
            np.asarray(p['block_data'])[:n])


def pbr_decode(p: dict) -> sp.csr_matrix:
    """pbr_to_csr (pbr_matrix.cpp:279-331)."""
    rows, cols = p['rows'], p['cols']
    gr, gc, gv = _pbr_entries(p)
    ri = np.asarray(p['remainder_indptr'], dtype=np.int64)
    rr = np.repeat(np.arange(rows), np.diff(ri))
    r = np.concatenate([gr, rr])
    c = np.concatenate([gc, np.asarray(p['remainder_col_ind'], dtype=np.int64)])
    v = np.concatenate([gv, np.asarray(p['remainder_data'])])
    o = np.lexsort((v, c, r))
    indptr = np.zeros(rows + 1, dtype=np.int64)
    np.cumsum(np.bincount(r, minlength=rows), out=indptr[1:])
    return sp.csr_matrix((v[o], c[o], indptr), shape=(rows, cols))


def pbr_cpu_matmul(p: dict, x: np.ndarray) -> np.ndarray:
    """pbr_batched_matmul_cpu (pbr_matrix.cpp:17-68)."""
    x3 = x[None] if x.ndim == 2 else x
    y = np.zeros((x3.shape[0], p['rows'], x3.shape[2]), dtype=x3.dtype)
    gr, gc, gv = _pbr_entries(p)
    ri = np.asarray(p['remainder_indptr'], dtype=np.int64)
    rr = np.repeat(np.arange(p['rows']), np.diff(ri))
    for bi in range(x3.shape[0]):
        _ordered_axpy(y[bi], gr, gc, gv, x3[bi])
        _ordered_axpy(y[bi], rr, np.asarray(p['remainder_col_ind'], dtype=np.int64),
                      np.asarray(p['remainder_data']), x3[bi])
    return y


# ---------------------------------------------------------------------------
# SpMM numerics
# ---------------------------------------------------------------------------

def spmm_reference(A: sp.csr_matrix, x: np.ndarray):
    """(Y64, B): the fp64 product of the original CSR with X, and the
    elementwise bound |A|.|X| that tolerances are stated against.  x may be
    [cols, K] or [batch, cols, K]."""
    # A private copy: csr_matrix(A, dtype=...) shares A's index arrays, and
    # scipy canonicalises a matrix in place (abs() sorts its indices), which
    # would scramble a caller's matrix whose rows are not sorted.
    A64 = sp.csr_matrix((np.asarray(A.data, dtype=np.float64), np.array(A.indices, copy=True),
                         np.array(A.indptr, copy=True)), shape=A.shape)
    Aabs = abs(A64)
    x64 = np.asarray(x, dtype=np.float64)
    if x64.ndim == 2:
        return A64 @ x64, Aabs @ np.abs(x64)
    return (np.stack([A64 @ xb for xb in x64]), np.stack([Aabs @ np.abs(xb) for xb in x64]))


def within_bound(y, A: sp.csr_matrix, x, rel: float = 1e-5):
    """max_ij |y - A x|_ij / (|A||X|)_ij and whether every entry satisfies
    |y - Ax| <= rel * (|A||X|) (entries with a zero bound must be exact)."""
    ref, bound = spmm_reference(A, x)
    y64 = np.asarray(y, dtype=np.float64)
    err = np.abs(y64 - ref)
    ok = bool(np.all(err <= rel * bound))
    with np.errstate(divide='ignore', invalid='ignore'):
        ratio = np.where(bound > 0, err / np.where(bound > 0, bound, 1), np.where(err > 0, np.inf, 0))
    return (float(ratio.max()) if ratio.size else 0.0), ok


# ---------------------------------------------------------------------------
# HEM clustering (torch_fast_spdmm/clustering.py:128-351), plain loops over
# Python sets and dicts -- small inputs only.
# ---------------------------------------------------------------------------

def _row_sets(pat):
    pat = sp.csr_matrix(pat)
    return [set(pat.indices[pat.indptr[i]:pat.indptr[i + 1]].tolist()) for i in range(pat.shape[0])]


def hem_similarity(pat, hub_degree=1024, topk=32):
    """dict {(i, j): w}: w = |cols(i) & cols(j)| over columns with at most
    hub_degree entries, i != j, w > 0; row i keeps its topk entries by
    (w desc, j asc); then an edge is kept with the larger weight of its two
    directions if either direction kept it (clustering.py:128-183)."""
    rows = _row_sets(pat)
    degree = {}
    for cols in rows:
        for c in cols:
            degree[c] = degree.get(c, 0) + 1
    light = [{c for c in cols if degree[c] <= hub_degree} for cols in rows]
    n = len(rows)
    kept = {}
    if n <= 1:
        return kept
    for i in range(n):
        cand = []
        for j in range(n):
            if j != i:
                w = len(light[i] & light[j])
                if w > 0:
                    cand.append((-w, j))
        cand.sort()
        if topk is not None:
            cand = cand[:topk]
        for negw, j in cand:
            kept[(i, j)] = -negw
    out = {}
    for (i, j), w in kept.items():
        w2 = max(w, kept.get((j, i), 0))
        out[(i, j)] = w2
        out[(j, i)] = w2
    return out


_M64 = (1 << 64) - 1


def _mix64_int(z):
    z ^= z >> 30
    z = (z * 0xBF58476D1CE4E5B9) & _M64
    z ^= z >> 27
    z = (z * 0x94D049BB133111EB) & _M64
    return z ^ (z >> 31)


def hem_pair_hash(a, b):
    """Symmetric hash of the pair {a, b} (clustering.py:190-207), Python ints."""
    lo, hi = min(a, b), max(a, b)
    return _mix64_int(((lo * 0x9E3779B97F4A7C15) & _M64) ^ ((hi * 0xC2B2AE3D27D4EB4F) & _M64)) >> 1


def hem_mutual_max(edges, n, active, size, nnz, max_size=None, max_nnz=None, feasible_first=False):
    """One mutual-max round (clustering.py:210-267) over edges {(i, j): w}:
    returns the sorted list of pairs (i, j), i < j."""
    def fits(i, j):
        return ((max_size is None or size[i] + size[j] <= max_size) and
                (max_nnz is None or nnz[i] + nnz[j] <= max_nnz))
    best = {}
    for (i, j), w in edges.items():
        if not (active[i] and active[j]):
            continue
        if feasible_first and not fits(i, j):
            continue
        key = (w, hem_pair_hash(i, j))
        if i not in best or key > best[i][0]:
            best[i] = (key, j)
    pairs = []
    for i, (_, j) in best.items():
        if i < j and j in best and best[j][1] == i and fits(i, j):
            pairs.append((i, j))
    return sorted(pairs)


def hem_labels(pat, target, max_size=None, max_nnz=None, hub_degree=1024, topk=32,
               residual_rounds=3, feasible_first=False):
    """Multilevel HEM labels (clustering.py:270-351), original vertex -> group,
    before the cap pass and renumbering of cluster_axis."""
    pat = sp.csr_matrix(pat)
    n = pat.shape[0]
    labels = list(range(n))
    if n <= 1 or target <= 1:
        return np.array(labels, dtype=np.int64)
    sets = _row_sets(pat)
    size = [1] * n
    nnz = [len(s) for s in sets]
    levels = 8 * max(1, int(np.ceil(np.log2(target)))) + 16
    for _ in range(levels):
        m = len(sets)
        if m <= 1:
            break
        cols = sorted({c for s in sets for c in s})
        index = {c: k for k, c in enumerate(cols)}
        level = sp.csr_matrix((np.ones(sum(len(s) for s in sets)),
                               ([i for i, s in enumerate(sets) for _ in s],
                                [index[c] for s in sets for c in sorted(s)])), shape=(m, max(len(cols), 1)))
        edges = hem_similarity(level, hub_degree, topk)
        if not edges:
            break
        active = [True] * m
        pairs = []
        for _round in range(residual_rounds):
            got = hem_mutual_max(edges, m, active, size, nnz, max_size, max_nnz, feasible_first)
            if not got:
                break
            for i, j in got:
                active[i] = active[j] = False
            pairs += got
        if not pairs:
            break
        owner = list(range(m))
        for i, j in pairs:
            owner[j] = i
        survivors = [v for v in range(m) if owner[v] == v]
        rank = {v: k for k, v in enumerate(survivors)}
        new_id = [rank[owner[v]] for v in range(m)]
        new_sets = [set() for _ in survivors]
        new_size = [0] * len(survivors)
        new_nnz = [0] * len(survivors)
        for v in range(m):
            new_sets[new_id[v]] |= sets[v]
            new_size[new_id[v]] += size[v]
            new_nnz[new_id[v]] += nnz[v]
        sets, size, nnz = new_sets, new_size, new_nnz
        labels = [new_id[x] for x in labels]
    return np.array(labels, dtype=np.int64)
