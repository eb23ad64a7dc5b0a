"""Vendor-library baseline row (reference autotune/src/autotune/runner/baseline.py:75-144).

The reference profiles the compiler's own lowering of ``lhs_T.T @ rhs``
(numpy -> nkipy -> neuronx-cc, seed 42, :117) beside the hand kernels.  The
MI355X analogue is the vendor GEMM: ``torch.matmul(lhs_T.t(), rhs)``, which
dispatches to hipBLASLt.  It is timed with the same hipEvent schedule and
reported as a ``ProfileResult`` with the same summary fields, so it can sit
in the same results table.  It is a comparison row only: nothing in the
kernel_library path calls it.
"""

from __future__ import annotations

import statistics

from autotune.runner.benchmark import generate_tensors, time_launches, upload, utilisation, work_of
from autotune.runner.types import ProfileResult, capture_error

BASELINE_SEED = 42


def profile_torch_baseline(M: int, N: int, K: int, dtype: str = "bfloat16", seed: int = BASELINE_SEED,
                           warmup: int = 10, reps: int = 50, dists: dict | None = None,
                           kernel_name: str = "hipblaslt_baseline", flush_bytes: int = 0,
                           lhs_layout: str = "KM") -> ProfileResult:
    """Time ``torch.matmul`` (hipBLASLt) of the left operand and rhs at (M, N, K).

    ``lhs_layout`` "KM" stores the left operand as lhs_T[K,M] (the
    matmul_lhsT_rhs layout), "MK" as lhs[M,K] (matmul_lhs_rhs: the product
    is ``torch.matmul(lhs, rhs)``).  ``flush_bytes`` > 0 overwrites a buffer
    of that size before every timed launch, as the kernel sweep does, so that
    neither side is timed from a warm L2/MALL.
    """
    import torch

    if lhs_layout not in ("KM", "MK"):
        raise ValueError(f"lhs_layout must be 'KM' or 'MK', got {lhs_layout!r}")
    specs = {"lhs_T": ((K, M), dtype)} if lhs_layout == "KM" else {"lhs": ((M, K), dtype)}
    specs["rhs"] = ((K, N), dtype)
    try:
        dev = upload(generate_tensors(specs, seed, dists), specs, torch.device("cuda:0"))
        a, b = (dev["lhs_T"].t(), dev["rhs"]) if lhs_layout == "KM" else (dev["lhs"], dev["rhs"])
        out = torch.empty((M, N), dtype=a.dtype, device=a.device)
        flush = torch.empty(flush_bytes // 4, dtype=torch.float32, device=a.device).zero_ if flush_bytes else None
        times = time_launches(lambda: torch.matmul(a, b, out=out), warmup, reps, flush)
        med = statistics.median(times)
        flops, nbytes = work_of("matmul_lhsT_rhs", M, N, K, dtype)
        summary = {"total_time": med, "min_time": min(times), "warmup": warmup, "reps": reps, "flops": flops,
                   "bytes": nbytes, "library": "torch.matmul (hipBLASLt)", "flush_bytes": flush_bytes,
                   **utilisation(flops, nbytes, med, dtype)}
        return ProfileResult(kernel_name, f"[{M}, {N}] {dtype}", summary)
    except Exception as exc:
        return ProfileResult(kernel_name, capture_error(exc))
