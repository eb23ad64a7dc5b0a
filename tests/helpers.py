"""Shared helpers for the parity tests (host side only)."""

from __future__ import annotations

import numpy as np

from oracle import inputs as oinputs
from oracle import metrics

# Parity contract: bf16 inputs against an fp32/fp64
# reference on the same bf16-rounded inputs, max-relative-error <= 1e-2.
# matmul: the reference's elementwise metric max(|a-e|/(|e|+5e-3))
#   (kernel_transforms.py:594-597).  The kernel multiplies the bf16 inputs
#   exactly and accumulates in fp32, so only the final bf16 rounding (2^-9
#   relative) separates it from the golden.
BF16_MATMUL_MAX_REL = 1e-2
# fp32 kernel: the reference's fp32 contract is allclose(atol=rtol=5e-3)
# end to end (test/codegen/test_render.py:35-49, examples/
# tune_matmul_lhsT_rhs.py:156-172) and atol=rtol=1e-4 at 128^3
# (test/ops/test_direct_numpy_call.py:38).
F32_ATOL = F32_RTOL = 5e-3
# rmsnorm_matmul: the normalised rows are rounded to bf16 before the MFMA
# (the reference kernel does the same, kernel_hand_online.py:139-149), so an
# output near zero carries an absolute error of ~2^-9 * sqrt(K) * |y||w| that
# no relative bound can absorb.  The gate is max-rel 1e-2 with the atol floor
# set to the RMS of the expected output, plus the normwise max-rel 1e-2.
RMS_MAX_REL = 1e-2
RMS_NORMWISE = 1e-2


def rms_report(actual: np.ndarray, expected: np.ndarray) -> dict:
    e = np.asarray(expected, dtype=np.float64)
    floor = float(np.sqrt(np.mean(e * e))) if e.size else 1.0
    rep = metrics.report(actual, expected, atol=floor)
    rep["atol_floor"] = floor
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
