"""Row/column labelling for BOO.

Every method returns an int32 label per row (cluster the rows of ``mat``; pass
``mat.T`` for columns) and the same post-processing applies to all of them:
groups over the size / nnz caps are split in member order, then labels are
renumbered 0..n_groups-1 in order of first label value.  This follows
``torch_fast_spdmm/clustering.py`` (reference): ``cluster_axis`` :454-509,
``cluster_axes`` :512-545, ``_enforce_caps`` :83-121, ``_relabel_consecutive``
:77-80, ``is_pattern_symmetric`` :58-67, ``_tile_by_permutation`` :70-74.

Implemented methods: identity, random, degree, rcm and hem (multilevel
heavy-edge matching on the shared-column graph, :128-351: similarity graph
:128-183, pair hash :190-207, mutual-max matching :210-267, coarsening
:270-351).  hem is deterministic and its labels are bit-exact with the
reference's, since the BOO built from them must be.  graclus and metis wrap
third-party packages (torch_cluster, pymetis); without them they raise the
reference's ImportError, as the reference does.
"""

from __future__ import annotations

from typing import Optional, Tuple

import numpy as np
import scipy.sparse as sp

__all__ = ['cluster_axes', 'cluster_axis', 'CLUSTER_METHODS', 'is_pattern_symmetric']

CLUSTER_METHODS = ('identity', 'random', 'degree', 'rcm', 'hem', 'graclus', 'metis')

# Similarity-graph knobs (clustering.py:33-42): columns with more entries than
# HUB_DEGREE are ignored when counting shared columns; each row keeps its TOPK
# heaviest neighbours; the product is formed CHUNK_ROWS rows at a time.
HUB_DEGREE = 1024
TOPK = 32
CHUNK_ROWS = 4096


def _pattern(mat) -> sp.csr_matrix:
    """0/1 CSR copy: duplicates summed away, values dropped."""
    out = sp.csr_matrix(mat, copy=True)
    out.data = np.ones_like(out.data, dtype=np.int32)
    out.sum_duplicates()
    out.data[:] = 1
    return out


def is_pattern_symmetric(mat) -> bool:
    """Square, and the sparsity pattern equals its transpose's."""
    if mat.shape[0] != mat.shape[1]:
        return False
    pat = _pattern(mat)
    return (pat != pat.T).nnz == 0


def _tile_by_permutation(perm: np.ndarray, n: int, target: int) -> np.ndarray:
    """Consecutive runs of ``target`` vertices in ``perm`` order share a label."""
    labels = np.empty(n, dtype=np.int64)
    labels[perm] = np.arange(n, dtype=np.int64) // max(target, 1)
    return labels


def _relabel_consecutive(labels: np.ndarray) -> np.ndarray:
    labels = np.asarray(labels)
    if labels.size and labels[0] == 0:
        d = np.diff(labels)
        if np.all((d == 0) | (d == 1)):          # already 0, 1, ... in order (identity)
            return labels.astype(np.int64, copy=False)
    _, inverse = np.unique(labels, return_inverse=True)
    return inverse.astype(np.int64, copy=False)


def _enforce_caps(labels: np.ndarray, row_nnz: np.ndarray, max_size: Optional[int],
                  max_nnz: Optional[int]) -> np.ndarray:
    """Split groups over ``max_size`` members or ``max_nnz`` nonzeros.

    Members are visited in ascending index order within each group (stable
    sort by label); a new label starts when the next member would overflow a
    cap, except that a group always takes at least one member.
    """
    if max_size is None and max_nnz is None:
        return labels
    labels = _relabel_consecutive(labels)
    if labels.size == 0:
        return labels
    order = np.argsort(labels, kind='stable')
    sorted_labels = labels[order]
    starts = np.flatnonzero(np.r_[True, sorted_labels[1:] != sorted_labels[:-1]])
    bounds = np.r_[starts, sorted_labels.size]
    if max_nnz is None:
        # size cap only: each group is cut into runs of max_size members in
        # member order, and the groups' runs are numbered one after another
        # -- the loop below, without the loop
        sizes = np.diff(bounds)
        pos = np.arange(labels.size, dtype=np.int64) - np.repeat(starts, sizes)
        runs = (sizes + max_size - 1) // max_size
        base = np.r_[0, np.cumsum(runs)[:-1]]
        out = np.empty_like(labels)
        out[order] = np.repeat(base, sizes) + pos // max_size
        return out
    out = np.empty_like(labels)
    nxt = 0
    for g in range(starts.size):
        size = 0
        nnz = 0
        for member in order[bounds[g]:bounds[g + 1]]:
            m_nnz = int(row_nnz[member])
            over_size = max_size is not None and size + 1 > max_size
            over_nnz = max_nnz is not None and size > 0 and nnz + m_nnz > max_nnz
            if size > 0 and (over_size or over_nnz):
                nxt += 1
                size = 0
                nnz = 0
            out[member] = nxt
            size += 1
            nnz += m_nnz
        nxt += 1
    return out


# ---------------------------------------------------------------------------
# heavy-edge matching
# ---------------------------------------------------------------------------

def _similarity_graph(pat: sp.csr_matrix, hub_degree: int, topk: Optional[int],
                      chunk_rows: int = CHUNK_ROWS) -> sp.csr_matrix:
    """Row-row weights W[i, j] = number of non-hub columns rows i and j share
    (i != j).  Each row keeps its ``topk`` heaviest neighbours (ties: lower
    column index first), then W = max(W, W^T), so an edge survives if either
    end kept it.  Rectangular input is fine: W is n x n.  clustering.py:128-183.
    """
    n, m = pat.shape
    if n <= 1:
        return sp.csr_matrix((n, n), dtype=np.int64)
    degree = np.bincount(pat.indices, minlength=m)
    light = np.flatnonzero(degree <= hub_degree)
    # dropping hub columns (and renumbering the rest) leaves every count of
    # shared columns unchanged
    P = pat if light.size == m else pat[:, light]
    P = sp.csr_matrix((np.ones(P.nnz, dtype=np.int64), P.indices, P.indptr), shape=P.shape)
    PT = P.T.tocsr()
    rows, cols, weights = [], [], []
    for r0 in range(0, n, chunk_rows):
        r1 = min(r0 + chunk_rows, n)
        prod = (P[r0:r1] @ PT).tocoo()
        r, c, w = prod.row.astype(np.int64), prod.col.astype(np.int64), prod.data
        keep = c != r + r0
        r, c, w = r[keep], c[keep], w[keep]
        if topk is not None and r.size:
            order = np.lexsort((c, -w, r))           # by row, heaviest first, then column
            r_sorted = r[order]
            first = np.searchsorted(r_sorted, r_sorted, side='left')
            order = order[np.arange(order.size) - first < topk]
            r, c, w = r[order], c[order], w[order]
        rows.append(r + r0)
        cols.append(c)
        weights.append(w)
    if not rows or sum(x.size for x in rows) == 0:
        return sp.csr_matrix((n, n), dtype=np.int64)
    W = sp.coo_matrix((np.concatenate(weights), (np.concatenate(rows), np.concatenate(cols))),
                      shape=(n, n)).tocsr()
    W.sum_duplicates()
    return W.maximum(W.T)


_U64 = np.uint64


def _mix64(z: np.ndarray) -> np.ndarray:
    """SplitMix64's output function (Steele, Lea and Flood 2014; constants of
    Vigna's splitmix64.c), on uint64 arrays, wrapping."""
    z = z ^ (z >> _U64(30))
    z = z * _U64(0xBF58476D1CE4E5B9)
    z = z ^ (z >> _U64(27))
    z = z * _U64(0x94D049BB133111EB)
    return z ^ (z >> _U64(31))


def _pair_hash(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Symmetric 63-bit hash of the unordered pair {a, b} (clustering.py:190-207):
    mix64(min * 0x9E3779B97F4A7C15 xor max * 0xC2B2AE3D27D4EB4F) >> 1."""
    lo = np.minimum(a, b).astype(_U64)
    hi = np.maximum(a, b).astype(_U64)
    with np.errstate(over='ignore'):
        h = _mix64((lo * _U64(0x9E3779B97F4A7C15)) ^ (hi * _U64(0xC2B2AE3D27D4EB4F)))
    return (h >> _U64(1)).astype(np.int64)


def _mutual_max_pairs(graph: sp.csr_matrix, active: np.ndarray, size: np.ndarray,
                      nnz: np.ndarray, max_size: Optional[int], max_nnz: Optional[int],
                      feasible_first: bool = False) -> Tuple[np.ndarray, np.ndarray]:
    """One round of mutual-max matching (clustering.py:210-267).

    Among its edges to active vertices (and, with ``feasible_first``, only
    those whose merged size / nnz fits the caps) every vertex picks the
    heaviest, ties broken by the larger pair hash.  Two vertices that picked
    each other form a pair (left < right); pairs over a cap are then dropped.
    """
    n = graph.shape[0]
    g = graph.tocoo()
    if g.nnz == 0:
        return np.empty(0, np.int64), np.empty(0, np.int64)
    r, c, w = g.row.astype(np.int64), g.col.astype(np.int64), g.data
    live = active[r] & active[c]
    if feasible_first:
        if max_size is not None:
            live &= size[r] + size[c] <= max_size
        if max_nnz is not None:
            live &= nnz[r] + nnz[c] <= max_nnz
    r, c, w = r[live], c[live], w[live]
    if r.size == 0:
        return np.empty(0, np.int64), np.empty(0, np.int64)
    order = np.lexsort((-_pair_hash(r, c), -w, r))
    r, c = r[order], c[order]
    head = np.ones(r.size, dtype=bool)
    head[1:] = r[1:] != r[:-1]
    choice = np.full(n, -1, dtype=np.int64)
    choice[r[head]] = c[head]
    v = np.arange(n, dtype=np.int64)
    other = np.where(choice >= 0, choice, v)
    mutual = (choice >= 0) & (choice[other] == v)
    left = v[mutual & (v < other)]
    right = other[left]
    if left.size:
        fits = np.ones(left.size, dtype=bool)
        if max_size is not None:
            fits &= size[left] + size[right] <= max_size
        if max_nnz is not None:
            fits &= nnz[left] + nnz[right] <= max_nnz
        left, right = left[fits], right[fits]
    return left, right


def _hem_labels(pat: sp.csr_matrix, target: int, max_size: Optional[int], max_nnz: Optional[int],
                hub_degree: int, topk: Optional[int], exact_recompute: bool = True,
                residual_rounds: int = 3, feasible_first: bool = False,
                hierarchy: Optional[list] = None) -> np.ndarray:
    """Multilevel heavy-edge matching (clustering.py:270-351).

    Each level rebuilds the similarity graph of the current supervertices (a
    supervertex's columns are the union of its members'), runs up to
    ``residual_rounds`` mutual-max rounds over the still-unmatched vertices,
    and contracts every pair: the right vertex joins the left one, and the
    surviving vertices are renumbered in index order.  Levels repeat until one
    matches nothing (at most 8 ceil(log2 target) + 16 levels); the size / nnz
    caps bound the growth.  ``hierarchy`` (a list) receives the labels of
    every level, identity first.
    """
    n = pat.shape[0]
    labels = np.arange(n, dtype=np.int64)
    if hierarchy is not None:
        hierarchy.append(labels.copy())
    if n <= 1 or target <= 1:
        return labels
    size = np.ones(n, dtype=np.int64)
    nnz = np.diff(pat.indptr).astype(np.int64)
    level = pat
    graph = None
    for _ in range(8 * max(1, int(np.ceil(np.log2(target)))) + 16):
        n_cur = level.shape[0]
        if n_cur <= 1:
            break
        if exact_recompute or graph is None:
            graph = _similarity_graph(level, hub_degree, topk)
        if graph.nnz == 0:
            break
        active = np.ones(n_cur, dtype=bool)
        lefts, rights = [], []
        for _round in range(residual_rounds):
            left, right = _mutual_max_pairs(graph, active, size, nnz, max_size, max_nnz,
                                            feasible_first)
            if left.size == 0:
                break
            lefts.append(left)
            rights.append(right)
            active[left] = False
            active[right] = False
        if not lefts:
            break
        left, right = np.concatenate(lefts), np.concatenate(rights)
        owner = np.arange(n_cur, dtype=np.int64)
        owner[right] = left                          # pairs are disjoint: one step
        survivor = owner == np.arange(n_cur)
        new_index = np.cumsum(survivor) - 1          # survivors keep their order
        new_id = new_index[owner]
        n_new = int(survivor.sum())
        size = np.bincount(new_id, weights=size, minlength=n_new).astype(np.int64)
        nnz = np.bincount(new_id, weights=nnz, minlength=n_new).astype(np.int64)
        labels = new_id[labels]
        if hierarchy is not None:
            hierarchy.append(labels.copy())
        merge = sp.csr_matrix((np.ones(n_cur, dtype=np.int64), (new_id, np.arange(n_cur))),
                              shape=(n_new, n_cur))
        level = merge @ level
        level.data[:] = 1                            # union of supports, not a count
        # without exact_recompute the graph is kept for the next level as is
    return labels


def cluster_axis(mat, method: str = 'hem', target: int = 32, max_size: Optional[int] = None,
                 max_nnz: Optional[int] = None, seed: int = 0, hub_degree: int = HUB_DEGREE,
                 topk: Optional[int] = TOPK, exact_recompute: bool = True,
                 feasible_first: bool = False, hem_hierarchy: Optional[list] = None) -> np.ndarray:
    """Cluster the ROWS of ``mat`` into groups of about ``target`` rows (int32 labels)."""
    if hem_hierarchy is not None and (method != 'hem' or len(hem_hierarchy)):
        raise ValueError('hem_hierarchy must be an empty list with method=hem')
    if method not in CLUSTER_METHODS:
        raise ValueError(f'unknown clustering method {method!r}; expected one of {CLUSTER_METHODS}')
    if method == 'graclus':
        # clustering.py:356-362: the backend is a third-party package
        try:
            from torch_cluster import graclus_cluster  # noqa: F401
        except (ImportError, OSError) as exc:
            raise ImportError("cluster='graclus' requires torch-cluster built for the installed "
                              "PyTorch version; no HEM fallback is performed") from exc
        raise NotImplementedError("cluster='graclus' is not implemented in spmm_amd")
    if method == 'metis':
        # clustering.py:407-412
        try:
            import pymetis  # noqa: F401
        except ImportError as exc:
            raise ImportError("cluster='metis' requires pymetis>=2025.2.2; "
                              "install the metis extra. No HEM fallback is performed") from exc
        raise NotImplementedError("cluster='metis' is not implemented in spmm_amd")

    pat = _pattern(mat)
    n = pat.shape[0]
    row_nnz = np.diff(pat.indptr).astype(np.int64)
    if n == 0:
        if hem_hierarchy is not None:
            hem_hierarchy.append(np.zeros(0, dtype=np.int64))
        return np.zeros(0, dtype=np.int32)

    if method == 'identity':
        labels = np.arange(n, dtype=np.int64) // max(target, 1)
    elif method == 'random':
        labels = _tile_by_permutation(np.random.default_rng(seed).permutation(n), n, target)
    elif method == 'degree':
        labels = _tile_by_permutation(np.argsort(row_nnz, kind='stable'), n, target)
    elif method == 'hem':
        labels = _hem_labels(pat, target, max_size, max_nnz, hub_degree, topk, exact_recompute,
                             feasible_first=feasible_first, hierarchy=hem_hierarchy)
    else:  # rcm
        if pat.shape[0] != pat.shape[1]:
            raise ValueError("cluster method 'rcm' requires a square matrix")
        from scipy.sparse.csgraph import reverse_cuthill_mckee
        sym = (pat + pat.T).tocsr()
        sym.data[:] = 1
        perm = reverse_cuthill_mckee(sym, symmetric_mode=True).astype(np.int64)
        labels = _tile_by_permutation(perm, n, target)

    labels = _enforce_caps(labels, row_nnz, max_size, max_nnz)
    return _relabel_consecutive(labels).astype(np.int32)


def cluster_axes(mat, method: str = 'hem', target_nr: int = 32, target_nc: int = 32,
                 max_nr: Optional[int] = None, max_nc: Optional[int] = None,
                 max_block_nnz: Optional[int] = None, seed: int = 0,
                 symmetric: Optional[bool] = None, hub_degree: int = HUB_DEGREE,
                 topk: Optional[int] = TOPK, exact_recompute: bool = True,
                 feasible_first: bool = False) -> Tuple[np.ndarray, np.ndarray]:
    """(row_labels, col_labels).  A pattern-symmetric matrix with equal targets
    reuses the row labels for the columns; otherwise columns come from A^T."""
    csr = sp.csr_matrix(mat)
    if symmetric is None:
        symmetric = (target_nr == target_nc) and is_pattern_symmetric(csr)
    row_labels = cluster_axis(csr, method=method, target=target_nr, max_size=max_nr,
                              max_nnz=max_block_nnz, seed=seed, hub_degree=hub_degree, topk=topk,
                              exact_recompute=exact_recompute, feasible_first=feasible_first)
    if symmetric:
        return row_labels, row_labels.copy()
    col_labels = cluster_axis(csr.T.tocsr(), method=method, target=target_nc, max_size=max_nc,
                              max_nnz=max_block_nnz, seed=seed, hub_degree=hub_degree, topk=topk,
                              exact_recompute=exact_recompute, feasible_first=feasible_first)
    return row_labels, col_labels
