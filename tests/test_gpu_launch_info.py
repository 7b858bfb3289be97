"""Launch introspection (boo_launch_info / pbr_launch_info, the C ABI's
spmm_*_launch_info) against what the multiply really launches, as the
reference checks boo_nnzflat_launch_info against the profiler's kernel names
(tests/torch_fast_spdmm/test_boo_nnzflat_fpt.py:276-303).  Every kernel
reports the runtime's attributes; none of them spills (no scratch)."""

import re

import numpy as np
import pytest
import scipy.sparse as sp
import torch

import spmm_amd as S
import spmm_amd.boo as SB
from spmm_amd import matrices as M
from test_gpu_large import _check as check_through_used_rows

pytestmark = pytest.mark.gpu

FAMILIES = {'boo_stream_kernel', 'boo_stream_dma_kernel', 'boo_blob_kernel', 'boo_rows_kernel',
            'gather_chunk_kernel', 'gather_fix_kernel', 'boo_fixup_kernel', 'rows_long_kernel',
            'fill_zero_kernel', 'pbr_stripe_kernel'}


def _launched(fn):
    """Kernel family names of this library's kernels that fn launches, in order."""
    from torch.profiler import ProfilerActivity, profile
    fn()
    torch.cuda.synchronize()
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        fn()
        torch.cuda.synchronize()
    evs = sorted((e for e in prof.events() if e.device_type == torch.autograd.DeviceType.CUDA),
                 key=lambda e: e.time_range.start)
    out = []
    for e in evs:
        m = re.search(r'(\w+)(?:<[^(]*>)?\(', e.name)
        fam = m.group(1) if m else None
        if fam in FAMILIES:
            out.append(fam)
    return out


def _check_attributes(info):
    assert info, 'no launches reported'
    for k in info:
        assert k['kernel'] in FAMILIES, k
        assert k['local_bytes_per_thread'] == 0, f"{k['kernel']} spills: {k}"
        assert k['registers_per_thread'] > 0 and k['static_shared_bytes'] >= 0, k
        assert k['max_active_blocks_per_cu'] >= 1, k
        assert k['threads'] <= k['max_threads_per_block'], k
        assert all(g >= 1 for g in k['grid']), k


def _boo(A, monkeypatch, path):
    monkeypatch.setattr(SB, 'MIN_COL_REUSE', {'tile': 0.0, 'gather': 1e9, 'default': 1.5}[path])
    return S.csr_to_boo(A, cluster='identity', target_nr=32, target_nc=32).to('cuda')


@pytest.mark.parametrize('case', [
    ('stencil16', 'tile', 64, torch.float32, False),
    ('stencil16', 'tile', 64, torch.float32, True),
    ('stencil16', 'tile', 5, torch.float32, False),
    ('stencil16', 'tile', 64, torch.float64, False),
    ('stencil16', 'tile', 20, torch.float64, False),
    ('permuted16', 'gather', 32, torch.float32, False),
    ('rmat12', 'default', 128, torch.float32, False),
    ('rmat12', 'default', 24, torch.float64, False),
])
def test_boo_launch_info_is_what_runs(case, monkeypatch):
    which, path, K, dtype, records = case
    monkeypatch.setattr(SB, 'RECORD_STREAM', records)
    np_dtype = np.float32 if dtype == torch.float32 else np.float64
    if which == 'stencil16':
        A = M.stencil_27pt(16, dtype=np_dtype)
    elif which == 'permuted16':
        A = M.permuted(M.stencil_27pt(16, dtype=np_dtype), seed=1)
    else:
        A = M.rmat(12, 16).astype(np_dtype)
    boo = _boo(A, monkeypatch, path)
    x = torch.randn((2, A.shape[1], K), dtype=dtype, generator=torch.Generator().manual_seed(1)).cuda()
    info = S.boo_launch_info(boo, K, batch=2, x=x)
    _check_attributes(info)
    if records and dtype == torch.float32 and K % 64 == 0:
        assert info[0]['kernel'] == 'boo_blob_kernel'
    assert [k['kernel'] for k in info] == _launched(lambda: S.boo_matmul(boo, x))
    # boo_info of a staged matrix carries the runtime's figures of the first kernel
    bi = S.boo_info(boo, p=K)
    assert bi.arena_bytes == info[0]['static_shared_bytes']
    assert bi.ctas_per_sm == info[0]['max_active_blocks_per_cu']


def test_boo_launch_info_needs_a_staged_matrix():
    boo = S.csr_to_boo(M.stencil_27pt(4), cluster='identity', target_nr=32, target_nc=32)
    with pytest.raises(RuntimeError, match='not on a GPU'):
        S.boo_launch_info(boo, 64)


def _block_matrix(rows, cols, blocks_per_stripe, seed, block=8):
    """rows x cols float32 CSR made of random 8x8 blocks, half their bits set."""
    rng = np.random.default_rng(seed)
    n_str = rows // block
    nb = n_str * blocks_per_stripe
    br = np.repeat(np.arange(n_str), blocks_per_stripe)
    bc = rng.integers(0, cols // block, nb)
    bits = rng.random((nb, block, block)) < 0.5
    bb, rr, cc = np.nonzero(bits)
    A = sp.csr_matrix((rng.standard_normal(bb.size).astype(np.float32),
                       (br[bb] * block + rr, bc[bb] * block + cc)), shape=(rows, cols))
    A.sum_duplicates()
    return A


@pytest.fixture
def slab_knob():
    yield S.set_pbr_slab_bytes
    S.set_pbr_slab_bytes(0)


@pytest.mark.parametrize('cols,K,slab,n_launch,grid_y', [
    (4096, 64, 0, 1, 1),              # one 64-feature tile
    (4096, 256, 0, 1, 1),             # one 256-feature tile
    (4096, 320, 0, 1, 2),             # 256-feature tiles over a grid of 2
    (262144, 256, 0, 1, 1),           # X of 268 MB, one launch (the default)
    (262144, 256, 192 << 20, 4, 1),   # X above the knob: 64-feature tiles, one launch each
    (4096, 256, 192 << 20, 1, 1),     # X below the knob: unchanged
])
def test_pbr_launch_info_and_serial_feature_tiles(cols, K, slab, n_launch, grid_y, slab_knob):
    slab_knob(slab)
    A = _block_matrix(2048, cols, 8, seed=K)
    p = S.csr_to_pbr(A, 8, 8, 4).to('cuda')
    X = torch.randn((1, cols, K), device='cuda')
    info = S.pbr_launch_info(p, K, x=X)
    _check_attributes(info)
    stripes = [k for k in info if k['kernel'] == 'pbr_stripe_kernel']
    assert len(stripes) == n_launch and all(k['grid'][1] == grid_y for k in stripes)
    assert [k['kernel'] for k in info] == _launched(lambda: S.pbr_matmul(p, X))
    y = S.pbr_matmul(p, X)
    torch.cuda.synchronize()
    check_through_used_rows(y, A, X)
    assert torch.equal(S.pbr_matmul(p, X), y)
