"""spmm_amd -- sparse x dense matrix multiply (SpMM) for MI355X (gfx950).

Public names follow the reference package ``torch_fast_spdmm``
(torch_fast_spdmm/__init__.py:400-438): BOO (``csr_to_boo``, ``boo_matmul``,
``boo_to_csr``, ``boo_info``), PBR (``csr_to_pbr``, ``pbr_matmul``,
``pbr_to_csr``, ``pbr_info``), the naive CSR baseline ``spdmm_csr_naive``,
and ``.to('cuda')`` on the format objects.  GPU work runs in hand-written HIP
kernels in ``libspmm_amd.so``; host work (format builders, CPU ops) in the
native ``_core`` module.  Importing fails if either is not built.
"""

from ._native import core as _core  # noqa: F401  (loads the native extension)
from .boo import (  # noqa: E402
    BOOInfo, BOOMatrix, BOOMatrixInt32Double, BOOMatrixInt32Float, BOOMatrixInt64Double,
    BOOMatrixInt64Float, BooNzOrder, BooSmallBlockPolicy, NZ_ORDERS, SMALL_BLOCK_POLICIES,
    boo_arena_bytes, boo_info, boo_launch_info, boo_matmul, boo_to_csr, csr_to_boo,
)
from .clustering import CLUSTER_METHODS, cluster_axes, cluster_axis  # noqa: E402
from .csr import spdmm_csr_naive  # noqa: E402
from .pbr import (  # noqa: E402
    BlockFillStats, BlockStripeStats, DataOrder, PBRInfo, PBRMatrix, PBRMatrixInt32Double,
    PBRMatrixInt32Float, PBRMatrixInt64Double, PBRMatrixInt64Float, csr_to_pbr,
    pbr_batched_matmul_chunkcols_cuda, pbr_batched_matmul_cpu, pbr_batched_matmul_cuda,
    get_pbr_slab_bytes, pbr_batched_matmul_nnzflat_cuda, pbr_batched_matmul_variant_cuda, pbr_info,
    pbr_launch_info, pbr_matmul, pbr_to_csr, set_pbr_slab_bytes,
)
from .plan import BOOExecutionPlan, prepare_boo_cuda  # noqa: E402
from .timed import BOOTimedSpMM, DirectSpMM, PBRTimedSpMM  # noqa: E402

__version__ = '0.1.0'

__all__ = [
    'spdmm_csr_naive',
    'csr_to_boo', 'boo_to_csr', 'boo_info', 'boo_matmul', 'boo_arena_bytes', 'BOOInfo',
    'SMALL_BLOCK_POLICIES', 'NZ_ORDERS', 'cluster_axes', 'cluster_axis', 'CLUSTER_METHODS',
    'csr_to_pbr', 'pbr_to_csr', 'pbr_info', 'PBRInfo', 'BlockFillStats', 'BlockStripeStats',
    'pbr_matmul', 'pbr_batched_matmul_cpu', 'pbr_batched_matmul_cuda',
    'pbr_batched_matmul_chunkcols_cuda', 'pbr_batched_matmul_nnzflat_cuda',
    'pbr_batched_matmul_variant_cuda', 'BOOExecutionPlan', 'prepare_boo_cuda',
    'BOOTimedSpMM', 'PBRTimedSpMM', 'DirectSpMM',
]
