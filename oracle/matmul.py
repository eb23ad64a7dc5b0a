"""``out[M,N] = lhs_T[K,M].T @ rhs[K,N]`` -- closed form, brute force, tile emulation.

* :func:`closed_form` is the reference's golden ``lhs_T.T @ rhs``
  (examples/tune_matmul_lhsT_rhs.py:165; test/codegen/test_render.py:46),
  evaluated in float64 on the (already bf16-rounded) inputs.
* :func:`brute_force` is a plain triple loop in float64, an implementation
  independent of BLAS, for tiny shapes.
* :func:`tiled` restates the hand kernel's loop nest
  (kernel_library/matmul/lhsT_rhs/kernel_hand_90.92mfu.py:101-131): N blocks
  of 512 columns (:109), K blocks of 1024 rows (:114), M blocks of 512
  (:121); inside ``matmul_block`` (:72-98) each (128-row M tile, <=512-col
  N tile) gets a fresh fp32 PSUM tile (:84-85), K tiles of 128 accumulate
  ``stationary.T @ moving`` in fp32 (:86-91; NKIMatmul._run,
  nkigym/src/nkigym/ops/matmul.py:43-45), the PSUM drains to the output
  dtype (:92) and is added into the output accumulator in that dtype
  (:93-98).  With ``out_dtype="bfloat16"`` every drain and add is rounded
  to bf16 -- the reference's 2-stage K reduction; with "float32" it is the
  fp32 CPU simulation (simulate_fp32 rewrites bf16 to fp32,
  nkigym/src/nkigym/synthesis/simulate_nki.py:36-37).
"""

from __future__ import annotations

import numpy as np

from oracle.bf16 import round_bf16

TILE_K = 128       # nc_matmul K = partition size (ops/matmul.py:31-32)
TILE_M = 128
TILE_N_MAX = 512   # _TILE_N_MAX (kernel_hand_90.92mfu.py:73)
BLOCK_K = 1024     # i_block_d0 K block (kernel_hand_90.92mfu.py:114-120)
BLOCK_M = 512      # i_block_d1 M block (:121-127)
BLOCK_N = 512      # i_block_d2 N block (:109)


def closed_form(lhs_T: np.ndarray, rhs: np.ndarray) -> np.ndarray:
    """float64 ``lhs_T.T @ rhs``."""
    a = np.asarray(lhs_T, dtype=np.float64)
    b = np.asarray(rhs, dtype=np.float64)
    if a.ndim != 2 or b.ndim != 2 or a.shape[0] != b.shape[0]:
        raise ValueError(f"shape mismatch: lhs_T {a.shape}, rhs {b.shape}")
    return a.T @ b


def closed_form_lhs(lhs: np.ndarray, rhs: np.ndarray) -> np.ndarray:
    """float64 ``lhs @ rhs`` with lhs[M,K] K-contiguous: the product of
    ``matmul_lhs_rhs_nkigym`` (kernel_library/matmul/lhs_rhs/kernel_handtuned_89.26mfu.py:226-287)."""
    a = np.asarray(lhs, dtype=np.float64)
    b = np.asarray(rhs, dtype=np.float64)
    if a.ndim != 2 or b.ndim != 2 or a.shape[1] != b.shape[0]:
        raise ValueError(f"shape mismatch: lhs {a.shape}, rhs {b.shape}")
    return a @ b


def brute_force(lhs_T: np.ndarray, rhs: np.ndarray) -> np.ndarray:
    """float64 triple loop (tiny shapes only): out[m][n] = sum_k lhs_T[k][m] * rhs[k][n]."""
    K, M = lhs_T.shape
    K2, N = rhs.shape
    if K != K2:
        raise ValueError("K mismatch")
    a = [[float(v) for v in row] for row in np.asarray(lhs_T, dtype=np.float64)]
    b = [[float(v) for v in row] for row in np.asarray(rhs, dtype=np.float64)]
    out = np.zeros((M, N), dtype=np.float64)
    for m in range(M):
        for n in range(N):
            s = 0.0
            for k in range(K):
                s += a[k][m] * b[k][n]
            out[m, n] = s
    return out


def _cast(x: np.ndarray, out_dtype: str) -> np.ndarray:
    return round_bf16(x) if out_dtype == "bfloat16" else x.astype(np.float32)


def tiled(lhs_T: np.ndarray, rhs: np.ndarray, out_dtype: str = "bfloat16") -> np.ndarray:
    """Loop-nest emulation of ``matmul_lhsT_rhs_nkigym`` for any shape (edge tiles clipped)."""
    a = np.asarray(lhs_T, dtype=np.float32)
    b = np.asarray(rhs, dtype=np.float32)
    K, M = a.shape
    K2, N = b.shape
    if K != K2:
        raise ValueError("K mismatch")
    out = np.zeros((M, N), dtype=np.float32)  # sbuf_output, memset 0 (:113)
    for n0 in range(0, N, BLOCK_N):
        n1 = min(n0 + BLOCK_N, N)
        for kb0 in range(0, K, BLOCK_K):
            kb1 = min(kb0 + BLOCK_K, K)
            for mb0 in range(0, M, BLOCK_M):
                mb1 = min(mb0 + BLOCK_M, M)
                for m0 in range(mb0, mb1, TILE_M):          # matmul_block m_idx
                    m1 = min(m0 + TILE_M, mb1)
                    for t0 in range(n0, n1, TILE_N_MAX):     # n_idx
                        t1 = min(t0 + TILE_N_MAX, n1)
                        psum = np.zeros((m1 - m0, t1 - t0), dtype=np.float32)
                        for k0 in range(kb0, kb1, TILE_K):   # k_idx: nc_matmul
                            k1 = min(k0 + TILE_K, kb1)
                            psum += a[k0:k1, m0:m1].T @ b[k0:k1, t0:t1]
                        acc = _cast(psum, out_dtype)          # tensor_copy PSUM -> acc_tile
                        out[m0:m1, t0:t1] = _cast(out[m0:m1, t0:t1] + acc, out_dtype)  # tensor_tensor add
    return out


def tiled_lhs(lhs: np.ndarray, rhs: np.ndarray, out_dtype: str = "bfloat16") -> np.ndarray:
    """The reference lhs.rhs kernel's reduction order
    (kernel_library/matmul/lhs_rhs/kernel_handtuned_89.26mfu.py:226-287).

    It transposes 1024x1024 blocks of lhs by DMA into the lhs_T layout
    (dma_transpose_block, :54-92; :269-272) and runs the same
    ``matmul_block`` (:120-166): per (128-row M tile, <=512-col N tile) an
    fp32 PSUM over the 128-row K tiles of one 1024-row K block, drained to
    the output dtype and added into the output accumulator in that dtype,
    the accumulator zeroed once per M block (:255).  Its M/N blocking
    (1024 / 512, :243-283) differs from the lhs_T kernel's, but blocking
    along M or N changes no output element's reduction order, so the result
    is :func:`tiled` of the transposed operand.
    """
    a = np.asarray(lhs)
    if a.ndim != 2:
        raise ValueError(f"lhs must be 2-D, got {a.shape}")
    return tiled(np.ascontiguousarray(a.T), rhs, out_dtype)
