"""rmsnorm_matmul: two-pass closed form and the online "Algorithm 4" emulation.

Reference kernel: kernel_library/rmsnorm_matmul/kernel_hand_online.py.

* :func:`closed_form` is the "vanilla two-pass" of the kernel docstring
  (:5-8): ``m = sum_k lhs^2``; ``rms = 1/sqrt(m/K + eps)`` (``scale = 1/K``,
  :213; ``EPS = 1e-6``, :195; rsqrt = ``1/np.sqrt``, nkigym/src/nkigym/ops/
  activation.py:20-28,58-64); ``O = (lhs * rms) @ rhs``.  The benchmark
  config adds a ``gamma[K]`` weight on the normalised row; ``gamma=None`` is
  the reference kernel exactly (it has no gamma).  float64 throughout.
* :func:`online` restates the kernel's single-pass recurrence (:10-17) over
  its blocking (M blocks of 1024 rows, K blocks of 512, N blocks of 512;
  :212-221, :307-346): per K block ``m += sum x^2`` (:93-108, fp32),
  ``rms_new = rsqrt(m/K + eps)`` (:111-124), ``s = rms_new * (1/rms_old)``
  (:127-136) with ``rms_old = +inf`` at the first block (:236-249, so
  ``s_0 = 0``), ``lhs *= rms_new`` in the tile dtype (:139-149), then
  ``O = s * O + lhs^T-scaled @ rhs`` (:165-192) with O in the output dtype.
  ``tile_dtype="float32"`` gives the fp32 CPU-simulation semantics; with
  "bfloat16" the scaled tile and O are rounded to bf16 as on hardware.
"""

from __future__ import annotations

import numpy as np

from oracle.bf16 import round_bf16

EPS = 1e-6
BLOCK_M = 1024
BLOCK_K = 512
BLOCK_N = 512


def inv_rms(lhs: np.ndarray, eps: float = EPS) -> np.ndarray:
    """Per-row ``1/sqrt(mean_k lhs^2 + eps)`` in float64."""
    x = np.asarray(lhs, dtype=np.float64)
    K = x.shape[1]
    return 1.0 / np.sqrt((x * x).sum(axis=1) * (1.0 / K) + eps)


def closed_form(lhs: np.ndarray, rhs: np.ndarray, gamma: np.ndarray | None = None, eps: float = EPS) -> np.ndarray:
    """float64 ``(lhs * inv_rms[:, None] * gamma[None, :]) @ rhs``."""
    x = np.asarray(lhs, dtype=np.float64)
    w = np.asarray(rhs, dtype=np.float64)
    if x.ndim != 2 or w.ndim != 2 or x.shape[1] != w.shape[0]:
        raise ValueError(f"shape mismatch: lhs {x.shape}, rhs {w.shape}")
    y = x * inv_rms(x, eps)[:, None]
    if gamma is not None:
        g = np.asarray(gamma, dtype=np.float64)
        if g.shape != (x.shape[1],):
            raise ValueError("gamma must have shape [K]")
        y = y * g[None, :]
    return y @ w


def _cast(x: np.ndarray, dtype: str) -> np.ndarray:
    return round_bf16(x) if dtype == "bfloat16" else x.astype(np.float32)


def online(lhs: np.ndarray, rhs: np.ndarray, gamma: np.ndarray | None = None, eps: float = EPS,
           tile_dtype: str = "float32") -> np.ndarray:
    """Single-pass online recurrence of ``rmsnorm_matmul_online`` for any shape."""
    x = np.asarray(lhs, dtype=np.float32)
    w = np.asarray(rhs, dtype=np.float32)
    M, K = x.shape
    K2, N = w.shape
    if K != K2:
        raise ValueError("K mismatch")
    g = None if gamma is None else np.asarray(gamma, dtype=np.float32)
    scale = np.float32(1.0 / K)
    out = np.zeros((M, N), dtype=np.float32)
    for m0 in range(0, M, BLOCK_M):
        m1 = min(m0 + BLOCK_M, M)
        m_state = np.zeros(m1 - m0, dtype=np.float32)              # memset 0 (:256)
        rms_old = np.full(m1 - m0, np.inf, dtype=np.float32)        # +inf init (:249)
        o = np.zeros((m1 - m0, N), dtype=np.float32)                # sbuf_output 0 (:283)
        for k0 in range(0, K, BLOCK_K):
            k1 = min(k0 + BLOCK_K, K)
            tile = x[m0:m1, k0:k1]
            m_state = m_state + (tile * tile).sum(axis=1, dtype=np.float32)   # f_X
            rms_new = (1.0 / np.sqrt(m_state * scale + np.float32(eps))).astype(np.float32)  # g_B
            s = (rms_new * (np.float32(1.0) / rms_old)).astype(np.float32)    # s_k
            scaled = _cast(tile * rms_new[:, None], tile_dtype)                # lhs *= rms_new
            if g is not None:
                scaled = _cast(scaled * g[None, k0:k1], tile_dtype)
            for n0 in range(0, N, BLOCK_N):
                n1 = min(n0 + BLOCK_N, N)
                psum = scaled.T.T @ w[k0:k1, n0:n1]                            # lhs_T^T @ rhs
                o[:, n0:n1] = _cast(o[:, n0:n1] * s[:, None] + psum, tile_dtype)
            rms_old = rms_new
        out[m0:m1] = o
    return out
