"""Synthetic matrices of the benchmark configurations (seeded, deterministic).

All randomness is ``numpy.random.default_rng(seed)``.  Each generator returns
a canonical scipy CSR matrix (sorted indices, no duplicates) in float32 unless
asked otherwise; ``dense_x`` gives the matching dense operand.

1. ``laplacian_2d(256)``: 2-D 5-point Laplacian, diagonal 4, neighbours -1
   (the matrix of the reference's conftest.py:70-76, -LaplacianNd).
2. ``stencil_27pt(64)``: 3-D 27-point stencil, grid index x + n*(y + n*z);
   off-diagonals U(-1, 0); diagonal |sum of the row's off-diagonals| + 1.
3. ``block_sparse_pbr(524288)``: 8x8 tiles, 16 distinct uniform block columns
   per block row, each tile bit Bernoulli(1/2), values N(0, 1).
4. ``rmat(20, 16)``: R-MAT with (a, b, c, d) = (0.57, 0.19, 0.19, 0.05),
   16 * 2^scale sampled edges, symmetrised, deduplicated, self loops added,
   values 1/sqrt(d_i d_j) with d the row degrees of the final pattern.
5. ``permuted(stencil_27pt(128))``: the same stencil with rows and columns
   permuted by one seeded random permutation (P A P^T).
"""

from __future__ import annotations

import numpy as np
import scipy.sparse as sp

__all__ = ['laplacian_2d', 'stencil_27pt', 'block_sparse_pbr', 'rmat', 'permuted', 'dense_x',
           'CONFIGS', 'make_config']


def _csr_from_coo(rows, cols, vals, n_rows, n_cols, dtype):
    """Canonical CSR from COO triples whose (row, col) pairs are unique."""
    order = np.lexsort((cols, rows))
    indptr = np.zeros(n_rows + 1, dtype=np.int64)
    np.cumsum(np.bincount(rows, minlength=n_rows), out=indptr[1:])
    itype = np.int32 if max(n_rows, n_cols, len(vals)) < 2**31 else np.int64
    m = sp.csr_matrix((vals[order].astype(dtype), cols[order].astype(itype),
                       indptr.astype(itype)), shape=(n_rows, n_cols))
    m.has_sorted_indices = True
    return m


def laplacian_2d(n: int = 256, dtype=np.float32) -> sp.csr_matrix:
    N = n * n
    i = np.arange(N, dtype=np.int64)
    x, y = i % n, i // n
    rows, cols, vals = [i], [i], [np.full(N, 4.0)]
    for dx, dy in ((-1, 0), (1, 0), (0, -1), (0, 1)):
        ok = (x + dx >= 0) & (x + dx < n) & (y + dy >= 0) & (y + dy < n)
        rows.append(i[ok])
        cols.append(i[ok] + dx + n * dy)
        vals.append(np.full(int(ok.sum()), -1.0))
    return _csr_from_coo(np.concatenate(rows), np.concatenate(cols), np.concatenate(vals), N, N,
                         dtype)


def stencil_27pt(n: int = 64, seed: int = 0, dtype=np.float32) -> sp.csr_matrix:
    rng = np.random.default_rng(seed)
    N = n ** 3
    i = np.arange(N, dtype=np.int64)
    x, y, z = i % n, (i // n) % n, i // (n * n)
    rows, cols = [], []
    for dz in (-1, 0, 1):
        for dy in (-1, 0, 1):
            for dx in (-1, 0, 1):
                if dx == 0 and dy == 0 and dz == 0:
                    continue
                ok = ((x + dx >= 0) & (x + dx < n) & (y + dy >= 0) & (y + dy < n)
                      & (z + dz >= 0) & (z + dz < n))
                rows.append(i[ok])
                cols.append(i[ok] + dx + n * (dy + n * dz))
    r = np.concatenate(rows)
    c = np.concatenate(cols)
    order = np.lexsort((c, r))
    r, c = r[order], c[order]
    off = rng.uniform(-1.0, 0.0, size=r.size).astype(dtype)
    diag = (np.abs(np.bincount(r, weights=off.astype(np.float64), minlength=N)) + 1.0).astype(dtype)
    return _csr_from_coo(np.concatenate([r, i]), np.concatenate([c, i]),
                         np.concatenate([off, diag]), N, N, dtype)


def block_sparse_pbr(n: int = 524288, block: int = 8, blocks_per_row: int = 16, seed: int = 0,
                     dtype=np.float32) -> sp.csr_matrix:
    rng = np.random.default_rng(seed)
    nbr = n // block
    # 16 distinct block columns per block row: sorted sample without replacement.
    bcols = np.empty((nbr, blocks_per_row), dtype=np.int64)
    for s in range(0, nbr, 8192):
        e = min(nbr, s + 8192)
        keys = rng.random((e - s, nbr))
        bcols[s:e] = np.argpartition(keys, blocks_per_row, axis=1)[:, :blocks_per_row]
    bcols.sort(axis=1)
    bits = rng.random((nbr, blocks_per_row, block, block)) < 0.5
    br, bi, rr, cc = np.nonzero(bits)
    rows = br * block + rr
    cols = bcols[br, bi] * block + cc
    vals = rng.standard_normal(rows.size)
    return _csr_from_coo(rows, cols, vals, n, n, dtype)


def rmat(scale: int = 20, edge_factor: int = 16, abcd=(0.57, 0.19, 0.19, 0.05), seed: int = 0,
         dtype=np.float32) -> sp.csr_matrix:
    rng = np.random.default_rng(seed)
    N = 1 << scale
    m = edge_factor * N
    a, b, c, _ = abcd
    src = np.zeros(m, dtype=np.int64)
    dst = np.zeros(m, dtype=np.int64)
    for bit in range(scale):
        u = rng.random(m)
        right = ((u >= a) & (u < a + b)) | (u >= a + b + c)   # quadrants b and d
        down = u >= a + b                                      # quadrants c and d
        src |= down.astype(np.int64) << bit
        dst |= right.astype(np.int64) << bit
    r = np.concatenate([src, dst, np.arange(N)])
    c = np.concatenate([dst, src, np.arange(N)])
    key = np.unique(r * N + c)
    r, c = key // N, key % N
    deg = np.bincount(r, minlength=N).astype(np.float64)
    vals = 1.0 / np.sqrt(deg[r] * deg[c])
    return _csr_from_coo(r, c, vals, N, N, dtype)


def permuted(mat: sp.csr_matrix, seed: int = 0) -> sp.csr_matrix:
    """P A P^T with a seeded random permutation (row i of A becomes row p[i])."""
    N = mat.shape[0]
    perm = np.random.default_rng(seed).permutation(N)
    coo = mat.tocoo()
    return _csr_from_coo(perm[coo.row.astype(np.int64)], perm[coo.col.astype(np.int64)], coo.data,
                         N, N, mat.dtype)


def dense_x(n_rows: int, K: int, seed: int = 0, batch: int | None = None, dtype=np.float32):
    """X ~ N(0, 1), float32, shape [n_rows, K] (or [batch, n_rows, K])."""
    rng = np.random.default_rng(seed)
    shape = (n_rows, K) if batch is None else (batch, n_rows, K)
    return rng.standard_normal(shape, dtype=np.float32 if dtype == np.float32 else np.float64)


# name -> (matrix builder, K, formats run on it, build kwargs)
CONFIGS = {
    1: dict(name='laplacian2d_256', K=128, formats=('boo',),
            make=lambda: laplacian_2d(256)),
    2: dict(name='stencil27_64', K=64, formats=('boo', 'pbr'),
            make=lambda: stencil_27pt(64)),
    3: dict(name='blocksparse8_524288', K=256, formats=('pbr',), pbr_threshold=27,
            make=lambda: block_sparse_pbr(524288)),
    4: dict(name='rmat_s20_ef16', K=128, formats=('boo',),
            make=lambda: rmat(20, 16)),
    5: dict(name='stencil27_128_permuted', K=32, formats=('boo', 'pbr'),
            make=lambda: permuted(stencil_27pt(128))),
}


def make_config(cfg: int):
    spec = CONFIGS[cfg]
    return spec['make'](), spec
