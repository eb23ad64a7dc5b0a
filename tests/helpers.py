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


def rms_check_full(actual, expected) -> dict:
    """``rms_check`` over a whole output on the GPU: ``actual`` a device
    tensor, ``expected`` the float64 device tensor of the closed form on the
    same bf16 inputs.  The figures are computed on the device in float64
    with the definitions of ``oracle.metrics.report`` (max_abs, max_rel with
    the atol floor, normwise, non-finite count, allclose), so every one of
    the M*N outputs is compared without a host copy."""
    import torch

    a = actual.to(torch.float64)
    e = expected.to(torch.float64)
    if a.shape != e.shape:
        raise ValueError(f"shape mismatch {tuple(a.shape)} vs {tuple(e.shape)}")
    floor = RMS_ATOL_FRAC * (float(torch.sqrt(torch.mean(e * e))) if e.numel() else 1.0)
    diff = (a - e).abs()
    emax = float(e.abs().max()) if e.numel() else 0.0
    finite = torch.isfinite(a)
    rep = {
        "elements": int(a.numel()),
        "max_abs": float(diff.max()) if diff.numel() else 0.0,
        "max_rel": float((diff / (e.abs() + floor)).max()) if diff.numel() else 0.0,
        "normwise": float(diff.max() / emax) if diff.numel() and emax > 0 else 0.0,
        "nonfinite": int((~finite).sum()),
        "allclose": bool(finite.all() and (diff <= floor + RMS_RTOL * e.abs()).all()),
        "atol_floor": floor,
    }
    rep["ok"] = rep["allclose"] and rep["nonfinite"] == 0
    return rep


def rms_closed_form_gpu(x, w, gamma=None, eps: float = 1e-6):
    """float64 closed form (x * rsqrt(mean x^2 + eps) * gamma) @ W of bf16 device tensors, on the device
    (reference kernel_library/rmsnorm_matmul/kernel_hand_online.py:5-8; eps :195, 1/K :213)."""
    xd, wd = x.double(), w.double()
    y = xd * (xd * xd).mean(dim=1, keepdim=True).add(eps).rsqrt()
    if gamma is not None:
        y = y * gamma.double()[None, :]
    return y @ wd


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
