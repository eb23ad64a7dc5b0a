"""Tile meta-parameters of the MI355X kernels and their search space.

``TileConfig`` replaces the NKI block knobs of the reference library
(``tbm/tbn/tbk``, ``dim_order`` and the multi-buffer counts,
reference kernel_library/README.md:12-13;
kernel_library/matmul/lhsT_rhs/kernel_hand_90.92mfu.py:107-112) with the
CDNA4 knobs: workgroup tile (block_m, block_n, block_k), wavefronts per
workgroup, LDS stages, L2 raster group and a kernel-specific variant.
"""

from __future__ import annotations

import ctypes
import itertools
import json
from dataclasses import asdict, dataclass, replace
from pathlib import Path

from kernel_library import _lib

KERNEL_IDS = {
    "matmul_lhsT_rhs": _lib.MI_KERNEL_MATMUL_LHST_RHS_BF16,
    "matmul_lhsT_rhs_f32": _lib.MI_KERNEL_MATMUL_LHST_RHS_F32,
    "rmsnorm_matmul": _lib.MI_KERNEL_RMSNORM_MATMUL_BF16,
    "matmul_lhs_rhs": _lib.MI_KERNEL_MATMUL_LHS_RHS_BF16,
}

# The 72-point search grid (72 points before legality pruning).
GRID_BLOCK_MN = (64, 128, 256)
GRID_BLOCK_K = (32, 64)
GRID_WAVES = (4, 8)
GRID_STAGES = (1, 2)

LDS_BYTES_MAX = 160 * 1024
TUNED_TABLE = Path(__file__).resolve().parent / "tuned_configs.json"


@dataclass(frozen=True)
class TileConfig:
    """One point of the CDNA4 tile search space (``mi_tile_cfg``)."""

    block_m: int = 256
    block_n: int = 256
    block_k: int = 64
    waves: int = 8
    lds_stages: int = 2
    split_k: int = 1
    group_m: int = 8
    variant: int = 0

    def to_c(self) -> _lib.MiTileCfg:
        return _lib.MiTileCfg(
            self.block_m,
            self.block_n,
            self.block_k,
            self.waves,
            self.lds_stages,
            self.split_k,
            self.group_m,
            self.variant,
        )

    @staticmethod
    def from_c(c: _lib.MiTileCfg) -> "TileConfig":
        return TileConfig(c.block_m, c.block_n, c.block_k, c.waves, c.lds_stages, c.split_k, c.group_m, c.variant)

    @property
    def name(self) -> str:
        """Stable file-name stem of this config."""
        s = f"bm{self.block_m}_bn{self.block_n}_bk{self.block_k}_w{self.waves}_s{self.lds_stages}"
        if self.group_m != 8:
            s += f"_g{self.group_m}"
        if self.variant:
            s += f"_v{self.variant}"
        if self.split_k != 1:
            s += f"_k{self.split_k}"
        return s

    @classmethod
    def from_name(cls, name: str) -> "TileConfig":
        """Inverse of ``name`` (``bm256_bn256_bk32_w8_s3[_g4][_v1][_k2]``)."""
        fields = {"bm": "block_m", "bn": "block_n", "bk": "block_k", "w": "waves", "s": "lds_stages",
                  "g": "group_m", "v": "variant", "k": "split_k"}
        kw = {}
        for part in name.split("_"):
            key = part.rstrip("0123456789")
            if key not in fields or key == part:
                raise ValueError(f"bad tile config name {name!r}")
            kw[fields[key]] = int(part[len(key):])
        if not {"block_m", "block_n", "block_k", "waves", "lds_stages"} <= kw.keys():
            raise ValueError(f"bad tile config name {name!r}")
        return cls(**kw)

    def lds_bytes(self, elem_bytes: int = 2) -> int:
        """LDS bytes of the K-panel ring (the static-legality budget)."""
        return self.lds_stages * (self.block_m + self.block_n) * self.block_k * elem_bytes

    def asdict(self) -> dict:
        return asdict(self)


# The reference's kernel names, and the family each one is.
REFERENCE_NAMES = {
    "matmul_lhsT_rhs_nkigym": "matmul_lhsT_rhs",
    "matmul_lhs_rhs_nkigym": "matmul_lhs_rhs",
    "rmsnorm_matmul_online": "rmsnorm_matmul",
}


def canonical_name(func_name: str) -> str:
    """The kernel family of a family or reference kernel name."""
    return REFERENCE_NAMES.get(func_name, func_name)


def kernel_id(func_name: str) -> int:
    """C ABI kernel id of a family or reference kernel name."""
    try:
        return KERNEL_IDS[canonical_name(func_name)]
    except KeyError as exc:
        raise ValueError(f"unknown kernel {func_name!r}; known: {sorted(KERNEL_IDS) + sorted(REFERENCE_NAMES)}") from exc


def check(func_name: str, cfg: TileConfig, M: int, N: int, K: int) -> tuple[int, str]:
    """Static legality of ``cfg`` at (M, N, K): ``(code, message)``, code 0 = legal."""
    c = cfg.to_c()
    rc = _lib.lib().mi_cfg_check(kernel_id(func_name), ctypes.byref(c), M, N, K)
    return rc, (_lib.last_error() if rc else "")


def compiled_configs(func_name: str) -> list[TileConfig]:
    """Every tile config compiled into libmi_kernels.so for ``func_name``."""
    kid = kernel_id(func_name)
    L = _lib.lib()
    out = []
    for i in range(L.mi_num_configs(kid)):
        c = _lib.MiTileCfg()
        _lib.check_rc(L.mi_get_config(kid, i, ctypes.byref(c)), "mi_get_config")
        out.append(TileConfig.from_c(c))
    return out


def baseline_grid(variants: tuple[int, ...] = (0,)) -> list[TileConfig]:
    """The 72-point search grid (x variants), before legality pruning."""
    return [
        TileConfig(bm, bn, bk, w, s, 1, 8, v)
        for bm, bn, bk, w, s, v in itertools.product(
            GRID_BLOCK_MN, GRID_BLOCK_MN, GRID_BLOCK_K, GRID_WAVES, GRID_STAGES, variants
        )
    ]


def legal_configs(func_name: str, M: int, N: int, K: int, grid: list[TileConfig] | None = None,
                  with_gamma: bool = True) -> list[TileConfig]:
    """Configs of ``grid`` (default: all compiled ones) that pass static legality at (M, N, K).

    This plays the role of ``KernelMDP.legal_actions`` (reference
    nkigym/src/nkigym/environment/mdp.py:44-54): the action space of the
    search is the set of legal tile configs.  ``with_gamma`` (the fused
    kernel called with a gamma) drops the variants that compute the
    product without gamma only.
    """
    if grid is None:
        grid = compiled_configs(func_name)
        # Stream-K configs only where split-K copies are offered too: shapes
        # whose output tiles fill fewer than two waves of workgroups.
        grid = [c for c in grid if not (is_streamk(func_name, c) and -(-M // c.block_m) * -(-N // c.block_n) >= 512)]
        grid = grid + split_k_variants(func_name, grid, M, N)
    if with_gamma:
        grid = [c for c in grid if c.variant not in GAMMA_FREE_VARIANTS.get(func_name, ())]
    return [c for c in grid if check(func_name, c, M, N, K)[0] == 0]


# Fused variants that compute the product without gamma only (the C ABI
# rejects them with a gamma): rmsnorm_matmul 14 and 16.
GAMMA_FREE_VARIANTS = {"rmsnorm_matmul": (14, 16), "rmsnorm_matmul_online": (14, 16)}


# Stream-K variants (mi_streamk.hpp): lhsT.rhs 5 (rhs cached) and 6 (rhs non-temporal).
STREAMK_VARIANTS = {"matmul_lhsT_rhs": (5, 6), "matmul_lhsT_rhs_nkigym": (5, 6)}


def is_streamk(func_name: str, cfg: TileConfig) -> bool:
    """Whether ``cfg`` is a stream-K config of ``func_name`` (one workgroup per CU over all tiles' K loops)."""
    return cfg.variant in STREAMK_VARIANTS.get(func_name, ())


SPLIT_K_PARTS = (2, 4, 8, 16)


def split_k_variants(func_name: str, grid: list[TileConfig], M: int, N: int) -> list[TileConfig]:
    """Split-K copies of the pipelined matmul and register-staged fused configs whose output tiles fill
    fewer than two waves of workgroups on the GPU (< 512 tiles): K is then
    the only axis left to spread the work over more compute units.  Part
    counts keep the grid within 1024 workgroups (four per compute unit)."""
    splittable = {"matmul_lhsT_rhs": (1, 3, 4), "matmul_lhsT_rhs_nkigym": (1, 3, 4), "matmul_lhs_rhs": (0, 2),
                  "matmul_lhs_rhs_nkigym": (0, 2), "rmsnorm_matmul": (4, 5, 11, 12, 13),
                  "rmsnorm_matmul_online": (4, 5, 11, 12, 13)}.get(func_name, ())
    out = []
    for c in grid:
        tiles = -(-M // c.block_m) * -(-N // c.block_n)
        if c.variant in splittable and c.split_k == 1 and tiles < 512:
            out += [replace(c, split_k=p) for p in SPLIT_K_PARTS if tiles * p <= 1024]
    return out


def default_config(func_name: str, M: int, N: int, K: int) -> TileConfig:
    """Tuned config from ``tuned_configs.json`` if present for this shape, else the library default.

    ``rmsnorm_matmul_online`` (the fused product without gamma) takes its own
    tuned entry, else the gamma one, else ``mi_default_config_no_gamma``.

    Memoised per (name, shape) until the tuned table is reloaded: a call
    without a config pays a dict lookup, not a table scan and a library call."""
    key = (func_name, M, N, K)
    cfg = _DEFAULT_CACHE.get(key)
    if cfg is not None:
        return cfg
    no_gamma = func_name == "rmsnorm_matmul_online"
    tuned = tuned_table().get(table_key(func_name, M, N, K))
    if tuned is None and no_gamma:
        # Every gamma variant also computes the product without gamma.
        tuned = tuned_table().get(table_key("rmsnorm_matmul", M, N, K))
    if tuned is not None:
        cfg = TileConfig(**tuned)
    else:
        c = _lib.MiTileCfg()
        if no_gamma:
            rc = _lib.lib().mi_default_config_no_gamma(M, N, K, ctypes.byref(c))
        else:
            rc = _lib.lib().mi_default_config(kernel_id(func_name), M, N, K, ctypes.byref(c))
        _lib.check_rc(rc, "mi_default_config")
        cfg = TileConfig.from_c(c)
    _DEFAULT_CACHE[key] = cfg
    return cfg


def table_key(func_name: str, M: int, N: int, K: int) -> str:
    return f"{func_name}:{M}x{N}x{K}"


_TABLE_CACHE: dict | None = None
_DEFAULT_CACHE: dict[tuple, TileConfig] = {}


def tuned_table(reload: bool = False) -> dict:
    """The persisted autotune winners: ``{"<kernel>:<M>x<N>x<K>": {tile fields}}``."""
    global _TABLE_CACHE
    if _TABLE_CACHE is None or reload:
        _DEFAULT_CACHE.clear()
        data = {}
        if TUNED_TABLE.exists():
            data = json.loads(TUNED_TABLE.read_text()).get("configs", {})
        _TABLE_CACHE = data
    return _TABLE_CACHE


def record_tuned(func_name: str, M: int, N: int, K: int, cfg: TileConfig, path: Path = TUNED_TABLE,
                 extra: dict | None = None) -> None:
    """Persist an autotune winner into the tuned-config table."""
    doc = {"configs": {}, "measurements": {}}
    if path.exists():
        doc = json.loads(path.read_text())
        doc.setdefault("configs", {})
        doc.setdefault("measurements", {})
    key = table_key(func_name, M, N, K)
    doc["configs"][key] = cfg.asdict()
    if extra:
        doc["measurements"][key] = extra
    path.write_text(json.dumps(doc, indent=2, sort_keys=True) + "\n")
    tuned_table(reload=True)


__all__ = [
    "TileConfig",
    "KERNEL_IDS",
    "baseline_grid",
    "check",
    "compiled_configs",
    "default_config",
    "is_streamk",
    "legal_configs",
    "record_tuned",
    "tuned_table",
]
