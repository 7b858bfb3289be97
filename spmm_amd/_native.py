"""Loader for the native extension.

``import torch`` comes first so that torch's HIP runtime is the one the
extension binds to (both are ``libamdhip64.so.7``; one process gets one copy).
There is no fallback: if the extension is not built, importing spmm_amd fails
with a message saying how to build it.
"""

import torch  # noqa: F401  -- must precede the extension (shared HIP runtime)

try:
    from . import _core as core  # type: ignore[attr-defined]
except ImportError as exc:  # pragma: no cover - exercised only on a broken install
    raise ImportError(
        'spmm_amd native extension is not built (spmm_amd/_core*.so, spmm_amd/libspmm_amd.so); '
        'run `python spmm_amd/build.py` or `python -c "import __graft_entry__ as g; g.build()"`'
    ) from exc

__all__ = ['core']
