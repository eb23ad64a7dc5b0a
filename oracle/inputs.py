"""Seeded synthetic inputs, drawn in signature order.

Follows the reference's generator: ``np.random.default_rng(seed)`` and one
draw per tensor in ``input_specs`` order
(reference autotune/src/autotune/runner/benchmark.py:156-169, which draws
``standard_normal`` for every tensor) and the numerics check's draw
(examples/tune_matmul_lhsT_rhs.py:163-165).  The benchmark configs add
U(-1,1), N(0, sigma) and ``gamma = 1 + 0.1 N(0,1)``; ``dist`` selects them.
bf16 tensors are drawn in fp32 and rounded RNE (see ``oracle.bf16``).
"""

from __future__ import annotations

import numpy as np

from oracle.bf16 import round_bf16


def draw(rng: np.random.Generator, shape: tuple[int, ...], dist) -> np.ndarray:
    """One tensor from ``rng``: dist is "normal", "uniform", "gamma" or ("normal", sigma)."""
    if dist == "normal":
        return rng.standard_normal(shape).astype(np.float32)
    if dist == "uniform":
        return rng.uniform(-1.0, 1.0, shape).astype(np.float32)
    if dist == "gamma":
        return (1.0 + 0.1 * rng.standard_normal(shape)).astype(np.float32)
    if isinstance(dist, (tuple, list)) and dist[0] == "normal":
        return (float(dist[1]) * rng.standard_normal(shape)).astype(np.float32)
    raise ValueError(f"unknown distribution {dist!r}")


def generate(specs: dict, seed: int, dists: dict | None = None) -> dict[str, np.ndarray]:
    """``{name: array}`` for ``specs = {name: (shape, dtype)}`` in order; bf16 rounded, fp32 storage."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, (shape, dtype) in specs.items():
        a = draw(rng, tuple(shape), (dists or {}).get(name, "normal"))
        out[name] = round_bf16(a) if dtype == "bfloat16" else a.astype(np.float32)
    return out
