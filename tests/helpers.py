"""Shared helpers for the parity tests (host side only)."""

from __future__ import annotations

import numpy as np

from oracle import inputs as oinputs
from oracle import metrics

# Pass criteria.  The reference passes a kernel with np.allclose(atol, rtol)
# against the float golden (kernel_transforms.py:592-596; atol = rtol = 5e-3
# for fp32, test/codegen/test_render.py:49) and reports
# max_rel = max(|a-e| / (|e| + atol)) beside it.
#
# bf16 matmul: allclose with the reference's atol = 5e-3 and the benchmark's
#   rtol = 1e-2.  The kernel multiplies bf16 values exactly and accumulates in
#   fp32, so the error is the final bf16 rounding (<= 2^-8 |e|, 8 significant
#   bits) plus an fp32 accumulation error (~1e-4 absolute at K = 8192, far
#   under atol).
BF16_ATOL = 5e-3
BF16_RTOL = 1e-2
# fp32 matmul: the reference's fp32 contract, allclose(atol=rtol=5e-3)
#   (test/codegen/test_render.py:35-49); atol=rtol=1e-4 at 128^3
#   (test/ops/test_direct_numpy_call.py:38).
F32_ATOL = F32_RTOL = 5e-3
# rmsnorm_matmul: the normalised rows are rounded to bf16 before the product
#   (the reference kernel does the same, kernel_hand_online.py:139-149).  Each
#   rounded element carries a relative error of at most 2^-8 (rms ~1.5e-3), so
#   an output gets an absolute error of ~1.5e-3 * RMS(out) (std) whatever its
#   own size; the largest over the 16 M outputs of the 4096^3 case measures
#   ~6e-3 * RMS(out).  The absolute floor is therefore 1e-2 * RMS(out); rtol
#   stays 1e-2.
RMS_ATOL_FRAC = 1e-2
RMS_RTOL = 1e-2


def mm_check(actual: np.ndarray, expected: np.ndarray) -> dict:
    """Report for a bf16 matmul output; ``ok`` is the allclose gate."""
    rep = metrics.report(actual, expected, atol=BF16_ATOL, rtol=BF16_RTOL)
    rep["ok"] = rep["allclose"] and rep["nonfinite"] == 0
    return rep


def rms_check(actual: np.ndarray, expected: np.ndarray) -> dict:
    """Report for an rmsnorm_matmul output; ``ok`` is the allclose gate with the RMS-scaled floor."""
    e = np.asarray(expected, dtype=np.float64)
    floor = RMS_ATOL_FRAC * (float(np.sqrt(np.mean(e * e))) if e.size else 1.0)
    rep = metrics.report(actual, expected, atol=floor, rtol=RMS_RTOL)
    rep["atol_floor"] = floor
    rep["ok"] = rep["allclose"] and rep["nonfinite"] == 0
    return rep


def mm_inputs(K: int, M: int, N: int, seed: int = 0, dist="uniform", dtype="bfloat16") -> dict:
    return oinputs.generate({"lhs_T": ((K, M), dtype), "rhs": ((K, N), dtype)}, seed,
                            {"lhs_T": dist, "rhs": dist})


def rms_inputs(M: int, K: int, N: int, seed: int = 0, with_gamma: bool = True) -> dict:
    specs = {"lhs": ((M, K), "bfloat16")}
    dists = {"lhs": "normal", "rhs": ("normal", 1.0 / np.sqrt(K)), "gamma": "gamma"}
    if with_gamma:
        specs["gamma"] = ((K,), "bfloat16")
    specs["rhs"] = ((K, N), "bfloat16")
    return oinputs.generate(specs, seed, dists)
