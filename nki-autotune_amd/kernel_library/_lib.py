"""ctypes binding of libmi_kernels.so, the C ABI of include/mi_kernels.h.

The library is built in-tree by ``nki-autotune_amd/build_lib.py``.  Loading
fails loudly when it is missing: there is no CPU or PyTorch fallback for any
kernel of this package.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmi_kernels.so"

# Kernel ids (include/mi_kernels.h).
MI_KERNEL_MATMUL_LHST_RHS_BF16 = 0
MI_KERNEL_MATMUL_LHST_RHS_F32 = 1
MI_KERNEL_RMSNORM_MATMUL_BF16 = 2
MI_KERNEL_MATMUL_LHS_RHS_BF16 = 3
MI_NUM_KERNELS = 4

# Legality codes (positive return values).
MI_OK = 0
MI_E_NO_INSTANCE = 1
MI_E_LDS = 2
MI_E_WAVE_TILE = 3
MI_E_ALIGN = 4
MI_E_RANGE = 5
MI_E_ARGS = 6
MI_E_KERNEL = 7
MI_E_SPLIT = 8
MI_E_TILE = 9

CODE_NAMES = {
    MI_E_NO_INSTANCE: "no compiled instance",
    MI_E_LDS: "LDS over budget",
    MI_E_WAVE_TILE: "wave tile smaller than one MFMA tile",
    MI_E_ALIGN: "alignment",
    MI_E_RANGE: "operand too large for 32-bit buffer offsets",
    MI_E_ARGS: "bad arguments",
    MI_E_KERNEL: "unknown kernel",
    MI_E_SPLIT: "split_k unsupported",
    MI_E_TILE: "block size outside the template range",
}

# Every symbol the header declares; the library must export all of them.
EXPORTED_SYMBOLS = (
    "mi_cfg_check",
    "mi_num_configs",
    "mi_get_config",
    "mi_default_config",
    "mi_default_config_no_gamma",
    "mi_matmul_lhsT_rhs_bf16",
    "mi_matmul_lhsT_rhs_bf16_noalloc",
    "mi_matmul_lhs_rhs_bf16",
    "mi_matmul_lhsT_rhs_f32",
    "mi_rmsnorm_matmul_bf16",
    "mi_device_info",
    "mi_release_workspace",
    "mi_last_error",
    "mi_version",
)


# Exported by libmi_kernels.so only (not by the single-config libraries the
# autotuner builds just in time).
PREBUILT_ONLY_SYMBOLS = frozenset({"mi_matmul_lhsT_rhs_bf16_noalloc"})
# Bytes of the static device scratch of mi_matmul_lhsT_rhs_bf16_noalloc
# (MI_NOALLOC_SCRATCH_BYTES).
NOALLOC_SCRATCH_BYTES = 64 << 20


class MiTileCfg(ctypes.Structure):
    """``mi_tile_cfg`` of include/mi_kernels.h."""

    _fields_ = [
        ("block_m", ctypes.c_int),
        ("block_n", ctypes.c_int),
        ("block_k", ctypes.c_int),
        ("waves", ctypes.c_int),
        ("lds_stages", ctypes.c_int),
        ("split_k", ctypes.c_int),
        ("group_m", ctypes.c_int),
        ("variant", ctypes.c_int),
    ]


class KernelLibraryError(RuntimeError):
    """A launch or legality failure reported by libmi_kernels.so."""

    def __init__(self, code: int, message: str) -> None:
        super().__init__(f"[mi rc={code}] {message}")
        self.code = code
        self.message = message


_LIBS: dict[str, ctypes.CDLL] = {}


def _declare(lib: ctypes.CDLL) -> None:
    c_int, c_void_p, c_float, c_char_p = ctypes.c_int, ctypes.c_void_p, ctypes.c_float, ctypes.c_char_p
    cfgp = ctypes.POINTER(MiTileCfg)
    sigs = {
        "mi_cfg_check": (c_int, [c_int, cfgp, c_int, c_int, c_int]),
        "mi_num_configs": (c_int, [c_int]),
        "mi_get_config": (c_int, [c_int, c_int, cfgp]),
        "mi_default_config": (c_int, [c_int, c_int, c_int, c_int, cfgp]),
        "mi_default_config_no_gamma": (c_int, [c_int, c_int, c_int, cfgp]),
        "mi_matmul_lhsT_rhs_bf16": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, cfgp, c_void_p]),
        "mi_matmul_lhsT_rhs_bf16_noalloc": (
            c_int,
            [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, cfgp, c_void_p],
        ),
        "mi_matmul_lhs_rhs_bf16": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, cfgp, c_void_p]),
        "mi_matmul_lhsT_rhs_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, cfgp, c_void_p]),
        "mi_rmsnorm_matmul_bf16": (
            c_int,
            [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_float, cfgp, c_void_p],
        ),
        "mi_device_info": (c_int, [ctypes.POINTER(c_int), c_char_p, c_int, ctypes.POINTER(c_int)]),
        "mi_release_workspace": (c_int, []),
        "mi_last_error": (c_char_p, []),
        "mi_version": (c_char_p, []),
    }
    for name, (res, args) in sigs.items():
        if name in PREBUILT_ONLY_SYMBOLS and not hasattr(lib, name):
            continue
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


def load(path: str | os.PathLike) -> ctypes.CDLL:
    """Load (once per path) a library exporting the C ABI of include/mi_kernels.h.

    ``libmi_kernels.so`` holds every prebuilt instance; the autotune
    pipeline also loads per-config libraries built just in time from a
    generated instance source.  Both export the same symbols.
    """
    given = str(path)
    handle = _LIBS.get(given)
    if handle is not None:
        # Every kernel call comes through here: resolving the path (a few
        # filesystem lookups) only on the first load keeps the call cheap.
        return handle
    key = str(Path(path).resolve())
    handle = _LIBS.get(key)
    if handle is None:
        if not Path(key).exists():
            raise ImportError(
                f"{key} not found: build it with `python nki-autotune_amd/build_lib.py` (there is no fallback path)"
            )
        handle = ctypes.CDLL(key)
        _declare(handle)
        _LIBS[key] = handle
    _LIBS[given] = handle
    return handle


def lib() -> ctypes.CDLL:
    """Load (once) and return libmi_kernels.so; raise if it was never built."""
    return load(os.environ.get("MI_KERNELS_LIB", LIB_PATH))


def last_error() -> str:
    msg = lib().mi_last_error()
    return msg.decode() if msg else ""


def check_rc(rc: int, what: str) -> None:
    """Raise KernelLibraryError for a non-zero return code (ValueError-like for legality)."""
    if rc != 0:
        raise KernelLibraryError(rc, f"{what}: {last_error() or CODE_NAMES.get(rc, 'HIP error')}")
