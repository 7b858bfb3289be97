"""Row/column labelling for BOO.

Every method returns an int32 label per row (cluster the rows of ``mat``; pass
``mat.T`` for columns) and the same post-processing applies to all of them:
groups over the size / nnz caps are split in member order, then labels are
renumbered 0..n_groups-1 in order of first label value.  This follows
``torch_fast_spdmm/clustering.py`` (reference): ``cluster_axis`` :454-509,
``cluster_axes`` :512-545, ``_enforce_caps`` :83-121, ``_relabel_consecutive``
:77-80, ``is_pattern_symmetric`` :58-67, ``_tile_by_permutation`` :70-74.

Implemented methods: identity, random, degree, rcm.  The graph methods (hem,
graclus, metis) are not built yet and raise NotImplementedError.
"""

from __future__ import annotations

from typing import Optional, Tuple

import numpy as np
import scipy.sparse as sp

__all__ = ['cluster_axes', 'cluster_axis', 'CLUSTER_METHODS', 'is_pattern_symmetric']

CLUSTER_METHODS = ('identity', 'random', 'degree', 'rcm', 'hem', 'graclus', 'metis')
_IMPLEMENTED = ('identity', 'random', 'degree', 'rcm')


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


def cluster_axis(mat, method: str = 'hem', target: int = 32, max_size: Optional[int] = None,
                 max_nnz: Optional[int] = None, seed: int = 0, hub_degree: int = 1024,
                 topk: Optional[int] = 32, exact_recompute: bool = True,
                 feasible_first: bool = False, hem_hierarchy: Optional[list] = None) -> np.ndarray:
    """Cluster the ROWS of ``mat`` into groups of about ``target`` rows (int32 labels)."""
    if hem_hierarchy is not None and (method != 'hem' or len(hem_hierarchy)):
        raise ValueError('hem_hierarchy must be an empty list with method=hem')
    if method not in CLUSTER_METHODS:
        raise ValueError(f'unknown clustering method {method!r}; expected one of {CLUSTER_METHODS}')
    if method not in _IMPLEMENTED:
        raise NotImplementedError(
            f'clustering method {method!r} is not implemented in spmm_amd yet; '
            f'use one of {_IMPLEMENTED} or pass row_labels/col_labels')

    pat = _pattern(mat)
    n = pat.shape[0]
    row_nnz = np.diff(pat.indptr).astype(np.int64)
    if n == 0:
        return np.zeros(0, dtype=np.int32)

    if method == 'identity':
        labels = np.arange(n, dtype=np.int64) // max(target, 1)
    elif method == 'random':
        labels = _tile_by_permutation(np.random.default_rng(seed).permutation(n), n, target)
    elif method == 'degree':
        labels = _tile_by_permutation(np.argsort(row_nnz, kind='stable'), n, target)
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
                 symmetric: Optional[bool] = None, hub_degree: int = 1024,
                 topk: Optional[int] = 32, exact_recompute: bool = True,
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
