"""Error report of the reference (kernel_transforms.py:594-597).

``max_rel = max(|a - e| / (|e| + atol))`` with the atol floor (5e-3 in the
reference) so that outputs near zero do not dominate, plus ``max_abs`` and
a normwise ``||a - e||_inf / ||e||_inf``.
"""

from __future__ import annotations

import numpy as np

ATOL = 5e-3


def report(actual: np.ndarray, expected: np.ndarray, atol: float = ATOL) -> dict[str, float]:
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    if a.shape != e.shape:
        raise ValueError(f"shape mismatch {a.shape} vs {e.shape}")
    diff = np.abs(a - e)
    emax = float(np.abs(e).max()) if e.size else 0.0
    return {
        "max_abs": float(diff.max()) if diff.size else 0.0,
        "max_rel": float((diff / (np.abs(e) + atol)).max()) if diff.size else 0.0,
        "normwise": float(diff.max() / emax) if diff.size and emax > 0 else 0.0,
        "nonfinite": int((~np.isfinite(a)).sum()),
    }
