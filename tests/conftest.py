"""Shared test setup.

Markers: ``gpu`` -- needs an MI355X (run with ``-m gpu``); everything else runs
on the CPU.  The oracle (oracle/oracle.py) is the checker; the compiled
reference (oracle/_ref, built from /root/reference by ``make -C oracle ref``)
is used when present and its tests skip otherwise.
"""

import importlib
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = Path(__file__).resolve().parent / 'golden'
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs a GPU (MI355X); run with -m gpu')


@pytest.fixture(scope='session')
def ref_core():
    """The reference's CPU module compiled from its own sources, or skip."""
    ref_dir = ROOT / 'oracle' / '_ref'
    if not any(ref_dir.glob('torch_fast_spdmm_core*.so')):
        pytest.skip('oracle/_ref not built (needs /root/reference: make -C oracle ref)')
    import torch  # noqa: F401  (links libtorch first)
    if str(ref_dir) not in sys.path:
        sys.path.insert(0, str(ref_dir))
    return importlib.import_module('torch_fast_spdmm_core')


def load_fixture(name):
    with np.load(GOLDEN / f'{name}.npz', allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def fixture_names(prefix):
    return sorted(p.stem for p in GOLDEN.glob(f'{prefix}*.npz'))


def csr_of(fx):
    import scipy.sparse as sp
    m = sp.csr_matrix((fx['data'], fx['indices'], fx['indptr']), shape=tuple(fx['shape']))
    # scipy narrows int64 indices when they fit; keep the fixture's index type
    m.indptr, m.indices = fx['indptr'], fx['indices']
    return m


@pytest.fixture
def rng():
    return np.random.default_rng(0)
