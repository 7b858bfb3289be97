"""Loader for the native extension.

``import torch`` comes first so that torch's HIP runtime is the one the
extension binds to (both are ``libamdhip64.so.7``; one process gets one copy).
There is no fallback: if the extension is not built, importing spmm_amd fails
with a message saying how to build it.

``SPMM_AMD_CORE`` names another build of the same module to load instead (the
AddressSanitizer/UBSan build, ``python spmm_amd/build.py core-san``); it is a
host-code debugging aid and changes nothing on the GPU side.
"""

import importlib.util
import os
import sys

import torch  # noqa: F401  -- must precede the extension (shared HIP runtime)


def _load_from(path):
    spec = importlib.util.spec_from_file_location(__package__ + '._core', path)
    if spec is None or spec.loader is None:
        raise ImportError(f'SPMM_AMD_CORE={path}: not a loadable extension module')
    mod = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = mod
    spec.loader.exec_module(mod)
    return mod


try:
    if os.environ.get('SPMM_AMD_CORE'):
        core = _load_from(os.environ['SPMM_AMD_CORE'])
    else:
        from . import _core as core  # type: ignore[attr-defined]
except ImportError as exc:  # pragma: no cover - exercised only on a broken install
    raise ImportError(
        'spmm_amd native extension is not built (spmm_amd/_core*.so, spmm_amd/libspmm_amd.so); '
        'run `python spmm_amd/build.py` or `python -c "import __graft_entry__ as g; g.build()"`'
    ) from exc

__all__ = ['core']
