"""The hot-path kernels, callable on torch device tensors.

Drop-in for the reference kernel_library call signatures:

* ``matmul_lhsT_rhs(lhs_T, rhs) -> out`` replaces ``matmul_lhsT_rhs_nkigym``
  (reference kernel_library/matmul/lhsT_rhs/kernel_hand_90.92mfu.py:101-131):
  ``out[M,N] = lhs_T[K,M].T @ rhs[K,N]``, output allocated by the kernel
  wrapper and returned, dtype of the first input.
* ``matmul_lhs_rhs(lhs, rhs) -> out`` replaces ``matmul_lhs_rhs_nkigym``
  (reference kernel_library/matmul/lhs_rhs/kernel_handtuned_89.26mfu.py:226-287):
  ``out[M,N] = lhs[M,K] @ rhs[K,N]`` with lhs K-contiguous, bf16.
* ``rmsnorm_matmul(lhs, rhs, gamma=None, eps=1e-6) -> out`` replaces
  ``rmsnorm_matmul_online`` (reference
  kernel_library/rmsnorm_matmul/kernel_hand_online.py:198-353):
  ``out = (lhs / sqrt(mean_k lhs^2 + eps) * gamma) @ rhs``; with
  ``gamma=None`` it is exactly the reference kernel (EPS = 1e-6, :195).

Shape mismatches raise ``ValueError`` (the reference asserts its fixed
shapes, :103-104).  Every call runs a HIP kernel from libmi_kernels.so on the
current torch stream; there is no fallback path.
"""

from __future__ import annotations

import ctypes

import torch

from kernel_library import _lib
from kernel_library.config import TileConfig, default_config

EPS = 1e-6


def _stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _same_device(first: str, ref: torch.Tensor, **others: torch.Tensor | None) -> None:
    """Every operand lives on ``ref``'s device (the kernel runs there and reads raw pointers)."""
    for name, t in others.items():
        if t is not None and t.device != ref.device:
            raise ValueError(f"{name} is on {t.device}, {first} on {ref.device}: all operands must share a device")


def _no_overlap(out: torch.Tensor, **inputs: torch.Tensor | None) -> None:
    """``out`` shares no bytes with an input: the kernels read the inputs while they write ``out``."""
    o0 = out.data_ptr()
    o1 = o0 + out.numel() * out.element_size()
    for name, t in inputs.items():
        if t is None or t.numel() == 0 or out.numel() == 0:
            continue
        t0 = t.data_ptr()
        if t0 < o1 and o0 < t0 + t.numel() * t.element_size():
            raise ValueError(f"out overlaps {name}: the output must not alias an input")


def _check_operand(name: str, t: torch.Tensor, dtypes: tuple[torch.dtype, ...]) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor on a HIP device, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must live on a HIP device (got {t.device})")
    if t.dim() != 2 and name != "gamma":
        raise ValueError(f"{name} must be 2-D, got shape {tuple(t.shape)}")
    if t.dtype not in dtypes:
        raise ValueError(f"{name} dtype {t.dtype} not in {dtypes}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous (row-major)")


def matmul_lhsT_rhs(
    lhs_T: torch.Tensor,
    rhs: torch.Tensor,
    cfg: TileConfig | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """``out[M,N] = lhs_T[K,M].T @ rhs[K,N]`` on the GPU (bf16 or fp32)."""
    _check_operand("lhs_T", lhs_T, (torch.bfloat16, torch.float32))
    _check_operand("rhs", rhs, (torch.bfloat16, torch.float32))
    if lhs_T.dtype != rhs.dtype:
        raise ValueError(f"dtype mismatch: lhs_T {lhs_T.dtype} vs rhs {rhs.dtype}")
    _same_device("lhs_T", lhs_T, rhs=rhs, out=out)
    K, M = lhs_T.shape
    K2, N = rhs.shape
    if K != K2:
        raise ValueError(f"contraction mismatch: lhs_T has K={K}, rhs has K={K2}")
    if out is None:
        out = torch.empty((M, N), dtype=lhs_T.dtype, device=lhs_T.device)
    elif out.shape != (M, N) or out.dtype != lhs_T.dtype or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous {lhs_T.dtype} [{M},{N}] tensor")
    else:
        _no_overlap(out, lhs_T=lhs_T, rhs=rhs)
    fp32 = lhs_T.dtype == torch.float32
    name = "matmul_lhsT_rhs_f32" if fp32 else "matmul_lhsT_rhs"
    cfg = cfg if cfg is not None else default_config(name, M, N, K)
    c = cfg.to_c()
    L = _lib.lib()
    fn = L.mi_matmul_lhsT_rhs_f32 if fp32 else L.mi_matmul_lhsT_rhs_bf16
    with torch.cuda.device(lhs_T.device):
        rc = fn(lhs_T.data_ptr(), rhs.data_ptr(), out.data_ptr(), M, N, K, ctypes.byref(c),
                _stream_handle(lhs_T.device))
    _lib.check_rc(rc, name)
    return out


def matmul_lhs_rhs(
    lhs: torch.Tensor,
    rhs: torch.Tensor,
    cfg: TileConfig | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """``out[M,N] = lhs[M,K] @ rhs[K,N]`` on the GPU (bf16, lhs K-contiguous)."""
    _check_operand("lhs", lhs, (torch.bfloat16,))
    _check_operand("rhs", rhs, (torch.bfloat16,))
    _same_device("lhs", lhs, rhs=rhs, out=out)
    M, K = lhs.shape
    K2, N = rhs.shape
    if K != K2:
        raise ValueError(f"contraction mismatch: lhs has K={K}, rhs has K={K2}")
    if out is None:
        out = torch.empty((M, N), dtype=lhs.dtype, device=lhs.device)
    elif out.shape != (M, N) or out.dtype != lhs.dtype or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous bf16 [{M},{N}] tensor")
    else:
        _no_overlap(out, lhs=lhs, rhs=rhs)
    cfg = cfg if cfg is not None else default_config("matmul_lhs_rhs", M, N, K)
    c = cfg.to_c()
    with torch.cuda.device(lhs.device):
        rc = _lib.lib().mi_matmul_lhs_rhs_bf16(lhs.data_ptr(), rhs.data_ptr(), out.data_ptr(), M, N, K,
                                               ctypes.byref(c), _stream_handle(lhs.device))
    _lib.check_rc(rc, "matmul_lhs_rhs")
    return out


def rmsnorm_matmul(
    lhs: torch.Tensor,
    rhs: torch.Tensor,
    gamma: torch.Tensor | None = None,
    eps: float = EPS,
    cfg: TileConfig | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """``out[M,N] = (lhs[M,K] / sqrt(mean_k lhs^2 + eps) * gamma[K]) @ rhs[K,N]`` (bf16)."""
    _check_operand("lhs", lhs, (torch.bfloat16,))
    _check_operand("rhs", rhs, (torch.bfloat16,))
    _same_device("lhs", lhs, rhs=rhs, gamma=gamma, out=out)
    M, K = lhs.shape
    K2, N = rhs.shape
    if K != K2:
        raise ValueError(f"contraction mismatch: lhs has K={K}, rhs has K={K2}")
    if gamma is not None:
        _check_operand("gamma", gamma, (torch.bfloat16,))
        if gamma.shape != (K,):
            raise ValueError(f"gamma must have shape [{K}], got {tuple(gamma.shape)}")
    if out is None:
        out = torch.empty((M, N), dtype=lhs.dtype, device=lhs.device)
    elif out.shape != (M, N) or out.dtype != lhs.dtype or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous bf16 [{M},{N}] tensor")
    else:
        _no_overlap(out, lhs=lhs, rhs=rhs, gamma=gamma)
    if cfg is None:
        # Without gamma (the reference's contract) the no-gamma default: its
        # own tuned winner for the shape first.
        cfg = default_config("rmsnorm_matmul_online" if gamma is None else "rmsnorm_matmul", M, N, K)
    c = cfg.to_c()
    gptr = gamma.data_ptr() if gamma is not None else None
    with torch.cuda.device(lhs.device):
        rc = _lib.lib().mi_rmsnorm_matmul_bf16(lhs.data_ptr(), gptr, rhs.data_ptr(), out.data_ptr(), M, N, K,
                                               float(eps), ctypes.byref(c), _stream_handle(lhs.device))
    _lib.check_rc(rc, "rmsnorm_matmul")
    return out


def release_workspace() -> None:
    """Return the device memory cached for split-K and two-pass workspace (``mi_release_workspace``).

    Memory behind a call still running is kept; after ``torch.cuda.synchronize()`` everything goes."""
    _lib.check_rc(_lib.lib().mi_release_workspace(), "release_workspace")


# Reference names (drop-in aliases).
matmul_lhsT_rhs_nkigym = matmul_lhsT_rhs
matmul_lhs_rhs_nkigym = matmul_lhs_rhs


def rmsnorm_matmul_online(lhs: torch.Tensor, rhs: torch.Tensor) -> torch.Tensor:
    """The reference kernel's exact contract: no gamma, EPS = 1e-6."""
    return rmsnorm_matmul(lhs, rhs, None, EPS)
