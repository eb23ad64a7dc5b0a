"""MI355X (gfx950) kernel_library: hand-written HIP kernels behind a C ABI.

Public kernels (torch device tensors in, torch device tensor out):

* :func:`matmul_lhsT_rhs` -- ``lhs_T[K,M].T @ rhs[K,N]``, bf16 or fp32
* :func:`matmul_lhs_rhs` -- ``lhs[M,K] @ rhs[K,N]``, bf16
* :func:`rmsnorm_matmul` -- ``rmsnorm(lhs) * gamma @ rhs``, bf16

plus the reference names ``matmul_lhsT_rhs_nkigym``, ``matmul_lhs_rhs_nkigym`` and
``rmsnorm_matmul_online``, the tile search space (:class:`TileConfig`), and
:func:`release_workspace` (returns the cached split-K workspace memory).
"""

from kernel_library.config import (
    TileConfig,
    baseline_grid,
    check,
    compiled_configs,
    default_config,
    legal_configs,
)
from kernel_library.ops import (
    EPS,
    matmul_lhs_rhs,
    matmul_lhs_rhs_nkigym,
    matmul_lhsT_rhs,
    matmul_lhsT_rhs_nkigym,
    release_workspace,
    rmsnorm_matmul,
    rmsnorm_matmul_online,
)

__all__ = [
    "EPS",
    "TileConfig",
    "baseline_grid",
    "check",
    "compiled_configs",
    "default_config",
    "legal_configs",
    "matmul_lhs_rhs",
    "matmul_lhs_rhs_nkigym",
    "matmul_lhsT_rhs",
    "matmul_lhsT_rhs_nkigym",
    "release_workspace",
    "rmsnorm_matmul",
    "rmsnorm_matmul_online",
]
