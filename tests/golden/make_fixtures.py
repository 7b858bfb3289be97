"""Write the golden fixtures under tests/golden/ from the compiled reference.

Run in a container where /root/reference exists and `make -C oracle ref` has
built oracle/_ref/torch_fast_spdmm_core*.so (the reference's own
boo_matrix.cpp / pbr_matrix.cpp / bindings.cpp, CPU only).  The fixtures are
data: inputs and the reference's outputs, so the tests can check exact
encodings -- including csr_to_pbr's in-stripe block order, which only the
reference's libstdc++ hash map fixes -- where the reference is not available.

    python tests/golden/make_fixtures.py          # every fixture
    python tests/golden/make_fixtures.py wide     # only the wide-K (kernel-path) fixtures
"""

import sys
from pathlib import Path

import numpy as np
import scipy.sparse as sp

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT / 'oracle' / '_ref'))
import torch  # noqa: E402,F401  (the reference module links libtorch)
import torch_fast_spdmm_core as ref  # noqa: E402

PBR_FIELDS = ('block_codes', 'block_coords', 'block_offsets', 'block_data', 'remainder_indptr',
              'remainder_col_ind', 'remainder_data')
BOO_FIELDS = ('row_grp_ptr', 'row_ids', 'col_grp_ptr', 'col_ids', 'blk_row_grp', 'blk_col_grp',
              'blk_nz_ptr', 'blk_shift', 'nz_idx', 'nz_val', 'rem_indptr', 'rem_col_ind',
              'rem_vals', 'tail_row', 'tail_col', 'tail_val')


def pbr_cases():
    rng = np.random.default_rng(7)
    out = []
    # random square, several densities, both index types and value types
    for i, (n, dens) in enumerate([(64, 0.1), (100, 0.3), (257, 0.05), (13, 0.4), (9, 0.5)]):
        itype = np.int32 if i % 2 == 0 else np.int64
        vtype = np.float32 if i % 2 == 0 else np.float64
        m = sp.random(n, n, density=dens, format='csr', random_state=rng, dtype=vtype)
        m.sort_indices()
        m.indptr, m.indices = m.indptr.astype(itype), m.indices.astype(itype)
        for bs in (2, 4, 8):
            for thr in (1, 4, 20):
                out.append((f'pbr_rand{i}_b{bs}_t{thr}', m, bs, thr))
    # a wide rectangle: many block columns per stripe (several hash buckets)
    m = sp.random(40, 3000, density=0.02, format='csr', random_state=rng, dtype=np.float32)
    m.sort_indices()
    out.append(('pbr_wide_b8_t1', m, 8, 1))
    out.append(('pbr_wide_b4_t2', m, 4, 2))
    return out


def boo_cases():
    out = []
    entries = [(0, 0, 2), (0, 2, -1), (2, 6, 3), (2, 0, 1), (0, 1, 4), (1, 1, 2), (1, 4, -3),
               (4, 7, 1), (4, 9, 2), (4, 3, -2), (3, 5, 1)]
    r, c, v = zip(*entries)
    m = sp.csr_matrix((np.array(v, dtype=np.float32), (r, c)), shape=(7, 11))
    rl = np.array([0, 1, 0, 2, 1, 0, 2], np.int32)
    cl = np.array([0, 1, 0, 2, 1, 2, 0, 1, 2, 1, 2], np.int32)
    for pol in (0, 2, 3):
        for order in (0, 1):
            out.append((f'boo_7x11_p{pol}_o{order}', m, rl, cl, pol, 4, order))
    rng = np.random.default_rng(11)
    m = sp.random(300, 200, density=0.05, format='csr', random_state=rng, dtype=np.float64)
    m.sort_indices()
    rl = rng.integers(0, 17, size=300).astype(np.int32)
    cl = rng.integers(0, 9, size=200).astype(np.int32)
    for pol in (0, 2, 3):
        out.append((f'boo_rand_p{pol}', m, rl, cl, pol, 4, 0))
    return out


def stencil_27pt(n, seed):
    """The 27-point stencil of the benchmark configs (off-diagonal U(-1, 0),
    diagonal |row off-diagonal sum| + 1) on an n^3 grid, float32."""
    rng = np.random.default_rng(seed)
    idx = np.arange(n ** 3).reshape(n, n, n)
    rows, cols = [], []
    for dz in (-1, 0, 1):
        for dy in (-1, 0, 1):
            for dx in (-1, 0, 1):
                src = idx[max(0, -dz):n - max(0, dz), max(0, -dy):n - max(0, dy), max(0, -dx):n - max(0, dx)]
                dst = idx[max(0, dz):n - max(0, -dz), max(0, dy):n - max(0, -dy), max(0, dx):n - max(0, -dx)]
                rows.append(src.ravel())
                cols.append(dst.ravel())
    r, c = np.concatenate(rows), np.concatenate(cols)
    v = -rng.random(r.size)
    v[r == c] = 0.0
    off = np.bincount(r, weights=np.abs(v), minlength=n ** 3)
    v[r == c] = off[r[r == c]] + 1.0
    m = sp.csr_matrix((v.astype(np.float32), (r, c)), shape=(n ** 3, n ** 3))
    m.sort_indices()
    return m


def wide_cases():
    """Cases whose K reaches the 64-feature kernels: (name, fmt, matrix,
    K, build args).  Identity labels (i // 32) for BOO, as the configs use."""
    out = []
    st = stencil_27pt(8, seed=3)                       # 512 rows: every slice in the tile stream
    perm = np.random.default_rng(5).permutation(st.shape[0])
    pst = sp.csr_matrix(st[perm][:, perm])
    pst.sort_indices()                                 # 512 rows: every slice in the gather pass
    lap = sp.csr_matrix(sp.kron(sp.eye(16), sp.diags([-np.ones(15), 4 * np.ones(16), -np.ones(15)],
                                                       [-1, 0, 1])) - sp.diags([np.ones(240), np.ones(240)],
                                                                               [-16, 16]), dtype=np.float32)
    lap.sort_indices()
    for name, m, K in (('boo_stencil8_k64', st, 64), ('boo_stencil8_k128', st, 128), ('boo_perm8_k64', pst, 64),
                       ('boo_lap16_k128', lap, 128)):
        out.append((name, 'boo', m, K, None))
    for name, m, K, thr in (('pbr_stencil8_b8_t4_k64', st, 64, 4), ('pbr_perm8_b8_t4_k64', pst, 64, 4),
                            ('pbr_stencil8_b8_t27_k256', st, 256, 27)):
        out.append((name, 'pbr', m, K, thr))
    return out


def main():
    blobs = {}
    only_wide = sys.argv[1:] == ['wide']
    for name, fmt, m, K, thr in wide_cases():
        x = np.random.default_rng(4).standard_normal((m.shape[1], K)).astype(m.dtype)
        if fmt == 'boo':
            lab = (np.arange(m.shape[0]) // 32).astype(np.int32)
            b = ref.csr_to_boo(m.indptr, m.indices, m.data, m.shape[0], m.shape[1], lab, lab, 2, 4, 0)
            blobs[name] = dict(indptr=m.indptr, indices=m.indices, data=m.data, shape=np.array(m.shape),
                               params=np.array([2, 4, 0]), row_labels=lab, col_labels=lab,
                               maxima=np.array([b.max_nr, b.max_nc, b.max_nnz_blk]),
                               **{f: np.asarray(getattr(b, f)) for f in BOO_FIELDS})
            blobs[name]['y_cpu'] = ref.boo_batched_matmul_cpu(b, torch.from_numpy(x)).numpy()
        else:
            p = ref.csr_to_pbr(m.indptr, m.indices, m.data, m.shape[0], m.shape[1], 8, 8, thr)
            blobs[name] = dict(indptr=m.indptr, indices=m.indices, data=m.data, shape=np.array(m.shape),
                               params=np.array([8, 8, thr]), **{f: np.asarray(getattr(p, f)) for f in PBR_FIELDS})
            blobs[name]['y_cpu'] = ref.pbr_batched_matmul_cpu(p, torch.from_numpy(x)).numpy()
        blobs[name]['x'] = x
    if only_wide:
        for name, d in blobs.items():
            np.savez_compressed(HERE / f'{name}.npz', **d)
        print(f'wrote {len(blobs)} fixtures to {HERE}')
        return
    for name, m, bs, thr in pbr_cases():
        p = ref.csr_to_pbr(m.indptr, m.indices, m.data, m.shape[0], m.shape[1], bs, bs, thr)
        blobs[name] = dict(indptr=m.indptr, indices=m.indices, data=m.data,
                           shape=np.array(m.shape), params=np.array([bs, bs, thr]),
                           **{f: np.asarray(getattr(p, f)) for f in PBR_FIELDS})
        x = np.random.default_rng(1).standard_normal((m.shape[1], 5)).astype(m.dtype)
        blobs[name]['x'] = x
        blobs[name]['y_cpu'] = ref.pbr_batched_matmul_cpu(p, torch.from_numpy(x)).numpy()
    for name, m, rl, cl, pol, thr, order in boo_cases():
        b = ref.csr_to_boo(m.indptr, m.indices, m.data, m.shape[0], m.shape[1], rl, cl, pol, thr, order)
        blobs[name] = dict(indptr=m.indptr, indices=m.indices, data=m.data,
                           shape=np.array(m.shape), params=np.array([pol, thr, order]),
                           row_labels=rl, col_labels=cl,
                           maxima=np.array([b.max_nr, b.max_nc, b.max_nnz_blk]),
                           **{f: np.asarray(getattr(b, f)) for f in BOO_FIELDS})
        x = np.random.default_rng(2).standard_normal((m.shape[1], 6)).astype(m.dtype)
        blobs[name]['x'] = x
        blobs[name]['y_cpu'] = ref.boo_batched_matmul_cpu(b, torch.from_numpy(x)).numpy()
    for name, d in blobs.items():
        np.savez_compressed(HERE / f'{name}.npz', **d)
    print(f'wrote {len(blobs)} fixtures to {HERE}')


if __name__ == '__main__':
    main()
