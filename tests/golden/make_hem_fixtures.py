"""Write tests/golden/hem_labels.npz: HEM clustering labels computed by the
reference's own clustering module (torch_fast_spdmm/torch_fast_spdmm/
clustering.py, pure numpy/scipy, loaded by file path -- the compiled core is
not needed) on small seeded matrices.

The composed multilevel labels of cluster_axis(method='hem') are not fixed by
any known answer in the reference's tests, so these vectors pin them.  The
fixture is data: each case's CSR pattern (indptr, indices, shape), its
arguments, and the reference's labels.  Run where /root/reference exists:

    python tests/golden/make_hem_fixtures.py
"""

import importlib.util
from pathlib import Path

import numpy as np
import scipy.sparse as sp

HERE = Path(__file__).resolve().parent
SRC = Path('/root/reference/torch_fast_spdmm/torch_fast_spdmm/clustering.py')


def load_reference():
    spec = importlib.util.spec_from_file_location('ref_clustering', SRC)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def cases():
    """(name, matrix, kwargs for cluster_axis)."""
    out = []
    for seed, (n, m, dens) in enumerate([(97, 97, 0.12), (73, 89, 0.12), (256, 256, 0.05),
                                         (200, 150, 0.03), (128, 128, 0.2), (300, 300, 0.01)]):
        a = sp.random(n, m, density=dens, format='csr', random_state=seed)
        for target, max_size, max_nnz, ff in [(8, 8, None, True), (16, 16, None, False),
                                              (16, 16, 60, True), (32, 32, None, True),
                                              (8, None, None, False)]:
            out.append((f's{seed}_t{target}_m{max_size}_z{max_nnz}_f{int(ff)}', a,
                        dict(method='hem', target=target, max_size=max_size, max_nnz=max_nnz,
                             feasible_first=ff)))
    # a banded matrix (neighbours share columns), hub pruning and top-k in play
    band = sp.diags([np.ones(511), np.ones(512), np.ones(511)], [-1, 0, 1], shape=(512, 512),
                    format='csr')
    out.append(('band512_t16', band, dict(method='hem', target=16, max_size=16, feasible_first=True)))
    hub = sp.random(150, 120, density=0.05, format='lil', random_state=9)
    hub[:, 3] = 1.0                                   # a column in every row
    out.append(('hub_t8_h20', hub.tocsr(), dict(method='hem', target=8, max_size=8, hub_degree=20,
                                                 topk=4, feasible_first=True)))
    return out


def main():
    ref = load_reference()
    blobs = {}
    for name, a, kw in cases():
        a = sp.csr_matrix(a)
        a.sum_duplicates()
        a.sort_indices()
        labels = ref.cluster_axis(a, **kw)
        blobs[f'{name}__indptr'] = a.indptr.astype(np.int64)
        blobs[f'{name}__indices'] = a.indices.astype(np.int64)
        blobs[f'{name}__shape'] = np.array(a.shape, dtype=np.int64)
        blobs[f'{name}__labels'] = np.asarray(labels, dtype=np.int32)
        blobs[f'{name}__kw'] = np.array(repr(kw))
        # the symmetric two-axis entry point on square inputs
        if a.shape[0] == a.shape[1]:
            r, c = ref.cluster_axes(a, method='hem', target_nr=kw['target'], target_nc=kw['target'],
                                    max_nr=kw['max_size'], max_nc=kw['max_size'],
                                    feasible_first=kw['feasible_first'])
            blobs[f'{name}__axes_rows'] = np.asarray(r, dtype=np.int32)
            blobs[f'{name}__axes_cols'] = np.asarray(c, dtype=np.int32)
    np.savez_compressed(HERE / 'hem_labels.npz', **blobs)
    print('wrote', len(blobs), 'arrays')


if __name__ == '__main__':
    main()
