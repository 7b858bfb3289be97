"""Kernels that address X with 64-bit offsets: one batch's X slab of 4 GiB or
more, or more than 2^24 columns (the A32 = false instances of the BOO stream
kernel and the PBR stripe kernel).  X is generated on the GPU; only the X rows
the matrix references come back to the host for the oracle's fp64 product,
so the reference costs what the matrix costs, not what X costs."""

import numpy as np
import pytest
import scipy.sparse as sp
import torch

import spmm_amd as S
import spmm_amd.boo as SB
from oracle import oracle as O

pytestmark = pytest.mark.gpu

BIG_COLS = (1 << 24) + 4096


def _wide_matrix(rows, cols, per_row, seed, block=None):
    """rows x cols float32 CSR; columns spread over the whole range with most
    of them in the top 2^20 (above 2^24 when cols > 2^24), so that 64-bit
    X offsets are exercised.  block: 8 -> entries come in 8x8 blocks (PBR)."""
    rng = np.random.default_rng(seed)
    if block:
        nb = rows // block * per_row
        br = np.repeat(np.arange(rows // block), per_row)
        bc = np.where(rng.random(nb) < 0.8, cols // block - 1 - rng.integers(0, (1 << 20) // block, nb),
                      rng.integers(0, cols // block, nb))
        bits = rng.random((nb, block, block)) < 0.5
        bb, rr, cc = np.nonzero(bits)
        r = br[bb] * block + rr
        c = bc[bb] * block + cc
    else:
        r = np.repeat(np.arange(rows), per_row)
        c = np.where(rng.random(r.size) < 0.8, cols - 1 - rng.integers(0, 1 << 20, r.size),
                     rng.integers(0, cols, r.size))
    v = rng.standard_normal(r.size).astype(np.float32)
    A = sp.csr_matrix((v, (r, c)), shape=(rows, cols))
    A.sum_duplicates()
    return A


def _check(y, A, X):
    """y against the fp64 product, through the referenced X rows only."""
    used = np.unique(A.indices)
    Xs = X[0][torch.from_numpy(used).to(X.device).long()].cpu().numpy()
    remap = np.full(A.shape[1], -1, np.int64)
    remap[used] = np.arange(used.size)
    As = sp.csr_matrix((A.data, remap[A.indices], A.indptr), shape=(A.shape[0], used.size))
    ratio, ok = O.within_bound(y[0].cpu().numpy(), As, Xs, 1e-5)
    assert ok, f'max |err| / (|A||X|) = {ratio:.3e}'


@pytest.fixture(autouse=True)
def _free():
    yield
    torch.cuda.empty_cache()


@pytest.mark.parametrize('K', [8, 64])
@pytest.mark.parametrize('path', ['tile', 'gather'])
def test_boo_more_than_2_24_columns(K, path, monkeypatch):
    """cols > 2^24: the stream kernel forms X offsets in 64 bits (K = 64 also
    makes X a 4.3 GB slab); the gather pass always does."""
    monkeypatch.setattr(SB, 'MIN_COL_REUSE', 0.0 if path == 'tile' else 1e9)
    A = _wide_matrix(2048, BIG_COLS, 12, seed=K)
    assert A.indices.max() >= 1 << 24
    boo = S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32).to('cuda')
    d = boo._gpu_meta.desc
    assert (d['n_tiles'] > 0) == (path == 'tile')
    X = torch.randn((1, BIG_COLS, K), device='cuda')
    y = S.boo_matmul(boo, X)
    torch.cuda.synchronize()
    _check(y, A, X)


def test_pbr_x_slab_of_4_gib():
    """cols * K * 4 bytes = 4 GiB: the stripe kernel forms X offsets in 64 bits."""
    cols, K = 1 << 24, 64
    A = _wide_matrix(1024, cols, 6, seed=9, block=8)
    assert A.indices.max() >= (1 << 24) - (1 << 20)
    p = S.csr_to_pbr(A, 8, 8, 4).to('cuda')
    X = torch.randn((1, cols, K), device='cuda')
    assert X.numel() * 4 >= 1 << 32
    y = S.pbr_matmul(p, X)
    torch.cuda.synchronize()
    _check(y, A, X)
