"""Error report and pass criterion of the reference (kernel_transforms.py:592-596).

The reference passes a kernel when ``np.allclose(actual, expected, atol,
rtol)`` holds, i.e. ``|a - e| <= atol + rtol * |e|`` elementwise (atol =
rtol = 5e-3 for fp32; test/codegen/test_render.py:49,
examples/tune_matmul_lhsT_rhs.py:172), and prints
``max_rel = max(|a - e| / (|e| + atol))`` and ``max_abs`` beside it.
``report`` returns those figures plus the normwise ``||a - e||_inf /
||e||_inf``; ``within`` is the allclose criterion.
"""

from __future__ import annotations

import numpy as np

ATOL = 5e-3


def report(actual: np.ndarray, expected: np.ndarray, atol: float = ATOL, rtol: float | None = None) -> dict:
    """max_abs, max_rel (atol floor), normwise error, non-finite count; ``allclose`` when rtol is given."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    if a.shape != e.shape:
        raise ValueError(f"shape mismatch {a.shape} vs {e.shape}")
    diff = np.abs(a - e)
    emax = float(np.abs(e).max()) if e.size else 0.0
    rep = {
        "max_abs": float(diff.max()) if diff.size else 0.0,
        "max_rel": float((diff / (np.abs(e) + atol)).max()) if diff.size else 0.0,
        "normwise": float(diff.max() / emax) if diff.size and emax > 0 else 0.0,
        "nonfinite": int((~np.isfinite(a)).sum()),
    }
    if rtol is not None:
        rep["allclose"] = bool(within(a, e, atol, rtol))
    return rep


def within(actual: np.ndarray, expected: np.ndarray, atol: float, rtol: float) -> bool:
    """``np.allclose`` semantics: every ``|a - e| <= atol + rtol * |e|`` and every value finite."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    return bool(np.all(np.isfinite(a)) and np.all(np.abs(a - e) <= atol + rtol * np.abs(e)))
