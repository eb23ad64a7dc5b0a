"""CPU tests of the C ABI (libmi_kernels.so): it loads, exports every symbol of
include/mi_kernels.h, and its host-side legality checks return the documented
codes.  No call here launches a kernel or touches a GPU buffer.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

from kernel_library import _lib
from kernel_library.config import TileConfig, check, compiled_configs, default_config

ROOT = Path(__file__).resolve().parents[1]
MM, F32, RMS = _lib.MI_KERNEL_MATMUL_LHST_RHS_BF16, _lib.MI_KERNEL_MATMUL_LHST_RHS_F32, _lib.MI_KERNEL_RMSNORM_MATMUL_BF16
LHS = _lib.MI_KERNEL_MATMUL_LHS_RHS_BF16


def header_symbols() -> set[str]:
    syms = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        syms |= set(re.findall(r"^\s*(?:int|const\s+char\s*\*)\s+(mi_\w+)\s*\(", text, flags=re.M))
    return syms


def test_library_exports_every_header_symbol():
    syms = header_symbols()
    assert syms, "no declarations parsed from include/*.h"
    assert syms == set(_lib.EXPORTED_SYMBOLS)
    raw = ctypes.CDLL(str(_lib.LIB_PATH))
    for s in sorted(syms):
        assert getattr(raw, s) is not None, s
    assert _lib.lib().mi_version().decode().startswith("mi_kernels")


def test_probe_library_loads_and_exports_its_probes():
    from kernel_library import _probe

    h = _probe.lib()
    for s in ("mi_probe_clocked_lhsT_rhs", "mi_probe_mfma", "mi_probe_panel_stream"):
        assert getattr(h, s) is not None, s


def test_panel_stream_probe_rejects_bad_arguments_before_any_gpu_call():
    """The stream probe checks its region / row / pitch arguments on the host (fake pointers, no launch)."""
    from kernel_library import _probe

    h, fake, clk = _probe.lib(), 0x100000, 0x200000
    args = lambda region, rb, pitch, w=4, inf=8: h.mi_probe_panel_stream(fake, region, rb, pitch, w, inf, 256, 1,
                                                                          clk, None)
    assert args(1 << 20, 96, 1024) == _lib.MI_E_ARGS            # row_bytes not a power of two
    assert args(1 << 20, 2048, 2048) == _lib.MI_E_ARGS          # row_bytes above 1 KiB
    assert args(1 << 20, 128, 1000) == _lib.MI_E_ARGS           # pitch not a multiple of row_bytes
    assert args((1 << 20) + 4096, 128, 4096) == _lib.MI_E_ARGS  # region not a whole number of 8-row groups
    assert args(1 << 32, 1024, 1024) == _lib.MI_E_ARGS          # region past the 32-bit buffer offsets
    assert args(1 << 20, 1024, 1024, w=4, inf=3) == _lib.MI_E_NO_INSTANCE
    assert h.mi_probe_panel_stream(fake + 8, 1 << 20, 1024, 1024, 4, 8, 256, 1, clk, None) == _lib.MI_E_ARGS


def test_every_compiled_config_is_enumerable_and_legal():
    for fam, shape in (("matmul_lhsT_rhs", (2048, 2048, 2048)), ("rmsnorm_matmul", (2048, 2048, 2048)),
                       ("matmul_lhs_rhs", (2048, 2048, 2048)), ("matmul_lhsT_rhs_f32", (256, 512, 512))):
        cfgs = compiled_configs(fam)
        assert len(cfgs) == len(set(cfgs)) > 0
        for c in cfgs:
            assert check(fam, c, *shape) == (0, ""), (fam, c)
            assert TileConfig.from_name(c.name) == c


@pytest.mark.parametrize(
    "kid,cfg,shape,code",
    [
        (MM, TileConfig(256, 256, 64, 8, 2), (8192, 8192, 8192), _lib.MI_OK),
        (MM, TileConfig(256, 256, 128, 8, 2), (8192, 8192, 8192), _lib.MI_E_LDS),        # 256 KiB of panels
        (MM, TileConfig(32, 32, 64, 8, 1), (1024, 1024, 1024), _lib.MI_E_WAVE_TILE),     # 8 waves, 1 MFMA tile
        (MM, TileConfig(128, 192, 32, 4, 2), (1024, 1024, 1024), _lib.MI_E_TILE),        # 192 not a power of 2
        (RMS, TileConfig(128, 128, 16, 4, 1), (1024, 1024, 1024), _lib.MI_E_TILE),       # fused kernel needs bk >= 32
        (MM, TileConfig(128, 128, 64, 4, 2, split_k=2), (1024, 1024, 1024), _lib.MI_E_SPLIT),
        (MM, TileConfig(128, 128, 64, 4, 2), (1020, 1024, 1024), _lib.MI_E_ALIGN),       # M % 8
        (RMS, TileConfig(128, 128, 64, 8, 2), (1024, 1024, 1020), _lib.MI_E_ALIGN),      # K % 8 (fused)
        (MM, TileConfig(128, 128, 64, 4, 2), (65536, 65536, 65536), _lib.MI_E_RANGE),    # 8 GiB operand
        (RMS, TileConfig(256, 256, 32, 8, 3, variant=6), (1024, 1024, 1024), _lib.MI_E_TILE),     # no variant 6
        (RMS, TileConfig(256, 256, 32, 8, 3, variant=10), (1024, 1024, 1024), _lib.MI_E_TILE),    # no variant 10
        # the two-pass kernel (variant 13) has no gamma limit: its main pass is the lhsT core
        (RMS, TileConfig(256, 256, 32, 4, 3, variant=13), (4096, 4096, 4096), _lib.MI_OK),
        (RMS, TileConfig(256, 256, 32, 4, 3, variant=13), (1024, 1024, 32768), _lib.MI_OK),
        (RMS, TileConfig(128, 128, 64, 4, 3, split_k=4, variant=13), (512, 512, 16384), _lib.MI_OK),
        (RMS, TileConfig(256, 256, 32, 4, 3, variant=13), (1024, 1024, 1020), _lib.MI_E_ALIGN),   # K % 8
        (RMS, TileConfig(256, 256, 32, 4, 1, variant=13), (1024, 1024, 1024), _lib.MI_E_TILE),    # pipelined core
        (RMS, TileConfig(256, 256, 64, 4, 3, variant=13), (1024, 1024, 1024), _lib.MI_E_LDS),     # 3 x 64 KiB
        (MM, TileConfig(256, 512, 32, 4, 3, variant=1), (1024, 1024, 1024), _lib.MI_E_WAVE_TILE),  # 512 acc regs
        (MM, TileConfig(256, 512, 32, 8, 2, variant=1), (1024, 1024, 1024), _lib.MI_E_WAVE_TILE),  # 2 waves/SIMD
        (RMS, TileConfig(256, 256, 32, 8, 3, variant=5), (1024, 1024, 8200), _lib.MI_E_RANGE),
        (RMS, TileConfig(256, 256, 32, 8, 3, variant=5), (1024, 1024, 8192), _lib.MI_OK),
        # four 32 KiB stages leave room for 7936 fp32 gamma entries
        (RMS, TileConfig(256, 256, 32, 8, 4, variant=4), (1024, 1024, 7968), _lib.MI_E_RANGE),
        (RMS, TileConfig(256, 256, 32, 8, 4, variant=4), (1024, 1024, 7936), _lib.MI_OK),
        # variants 11 / 12 walk K one tile at a time, like 4 / 5
        (RMS, TileConfig(128, 128, 32, 4, 3, variant=12), (1024, 1024, 8200), _lib.MI_E_RANGE),
        (RMS, TileConfig(128, 128, 32, 4, 3, variant=12), (1024, 1024, 8192), _lib.MI_OK),
        (RMS, TileConfig(64, 128, 64, 4, 2, variant=11), (16, 28672, 8192), _lib.MI_OK),
        # split-K: the pipelined matmul body only, every part non-empty, workspace <= 2 GiB
        (MM, TileConfig(128, 128, 64, 4, 3, split_k=2, variant=1), (2048, 1024, 8192), _lib.MI_OK),
        (MM, TileConfig(32, 128, 128, 4, 3, split_k=16, variant=3), (128, 28672, 8192), _lib.MI_OK),
        (MM, TileConfig(128, 128, 64, 4, 3, split_k=17, variant=1), (2048, 1024, 8192), _lib.MI_E_SPLIT),
        (MM, TileConfig(128, 128, 64, 4, 3, split_k=0, variant=1), (2048, 1024, 8192), _lib.MI_E_SPLIT),
        (MM, TileConfig(128, 128, 64, 4, 3, split_k=2, variant=1), (2048, 1024, 64), _lib.MI_E_SPLIT),   # 1 K tile
        (MM, TileConfig(128, 128, 64, 4, 3, split_k=3, variant=1), (2048, 1024, 256), _lib.MI_E_SPLIT),  # 2+2+0
        (MM, TileConfig(128, 128, 64, 4, 3, split_k=2, variant=2), (2048, 1024, 8192), _lib.MI_E_SPLIT),
        # variant 4: K sub-steps split over the waves, each wave holding the whole block
        (MM, TileConfig(128, 128, 64, 4, 4, variant=4), (1024, 4096, 14336), _lib.MI_OK),
        (MM, TileConfig(128, 128, 64, 4, 4, split_k=2, variant=4), (2048, 1024, 8192), _lib.MI_OK),
        (MM, TileConfig(128, 128, 64, 4, 3, variant=4), (1024, 1024, 1024), _lib.MI_E_TILE),        # odd stages x 1 sub-step
        (MM, TileConfig(256, 128, 64, 4, 2, variant=4), (1024, 1024, 1024), _lib.MI_E_WAVE_TILE),   # 512 acc regs
        (MM, TileConfig(128, 128, 32, 4, 2, variant=4), (1024, 1024, 1024), _lib.MI_E_WAVE_TILE),   # 2 sub-steps, 4 waves
        (MM, TileConfig(128, 128, 128, 4, 3, variant=4), (1024, 1024, 1024), _lib.MI_E_LDS),        # 3 x 64 KiB
        (LHS, TileConfig(128, 128, 64, 4, 3, split_k=2), (2048, 1024, 8192), _lib.MI_OK),
        (LHS, TileConfig(128, 128, 64, 4, 3, split_k=4, variant=2), (128, 28672, 8192), _lib.MI_OK),
        (LHS, TileConfig(256, 256, 32, 8, 3, split_k=2, variant=1), (2048, 1024, 8192), _lib.MI_E_SPLIT),
        (RMS, TileConfig(128, 128, 64, 4, 2, split_k=2, variant=0), (2048, 1024, 4096), _lib.MI_E_SPLIT),
        (RMS, TileConfig(128, 128, 64, 4, 2, split_k=2, variant=4), (2048, 1024, 4096), _lib.MI_OK),
        # split parts stage the gamma of their own K range: 2 x 8192 fits, 2 x 8256 does not
        (RMS, TileConfig(128, 128, 64, 4, 2, split_k=2, variant=4), (256, 1024, 16384), _lib.MI_OK),
        (RMS, TileConfig(128, 128, 64, 4, 2, split_k=2, variant=4), (256, 1024, 16448), _lib.MI_E_RANGE),
        (RMS, TileConfig(128, 128, 64, 4, 2, variant=4), (256, 1024, 16384), _lib.MI_E_RANGE),
        (MM, TileConfig(32, 128, 64, 4, 4, split_k=16, variant=1), (16384, 16384, 8192), _lib.MI_E_RANGE),
        (MM, TileConfig(128, 128, 48, 4, 2), (1024, 1024, 1024), _lib.MI_E_TILE),
        (MM, TileConfig(64, 512, 32, 8, 2), (1024, 1024, 1024), _lib.MI_E_NO_INSTANCE),   # legal, not prebuilt
        (MM, TileConfig(512, 512, 32, 8, 1), (1024, 1024, 1024), _lib.MI_E_WAVE_TILE),    # 256x128 per wave
        (MM, TileConfig(0, 128, 64, 4, 2), (1024, 1024, 1024), _lib.MI_E_ARGS),
        (LHS, TileConfig(256, 256, 32, 4, 3), (8192, 8192, 8192), _lib.MI_OK),
        (LHS, TileConfig(256, 256, 32, 4, 3), (1024, 1024, 1020), _lib.MI_E_ALIGN),      # K % 8 (K-contiguous lhs)
        (LHS, TileConfig(128, 128, 16, 4, 2), (1024, 1024, 1024), _lib.MI_E_TILE),       # pipelined core: bk >= 32
        (LHS, TileConfig(256, 256, 32, 4, 3, variant=3), (1024, 1024, 1024), _lib.MI_E_TILE),     # no variant 3
        (LHS, TileConfig(256, 256, 64, 4, 2), (65536, 65536, 65536), _lib.MI_E_RANGE),
        (LHS, TileConfig(64, 128, 128, 4, 3, variant=1), (1024, 1024, 1024), _lib.MI_E_TILE),    # pairs: bk <= 64
        (MM, TileConfig(256, 256, 32, 8, 1, variant=1), (1024, 1024, 1024), _lib.MI_E_TILE),     # pipelined: >= 2 stages
        (MM, TileConfig(256, 256, 16, 8, 2, variant=3), (1024, 1024, 1024), _lib.MI_E_TILE),     # pipelined: bk >= 32
        (F32, TileConfig(64, 64, 16, 4, 1, variant=1), (256, 512, 512), _lib.MI_OK),
        (F32, TileConfig(128, 128, 16, 4, 1, variant=1), (37, 53, 129), _lib.MI_OK),     # any M, N, K
        (F32, TileConfig(128, 64, 16, 4, 1, variant=1), (256, 512, 512), _lib.MI_E_TILE),  # square blocks only
        (F32, TileConfig(64, 64, 32, 4, 1, variant=1), (256, 512, 512), _lib.MI_E_TILE),   # block_k 16
        (F32, TileConfig(64, 64, 16, 4, 1, variant=2), (256, 512, 512), _lib.MI_E_TILE),   # no variant 2
        (RMS, TileConfig(128, 128, 64, 4, 3, variant=14), (2048, 2048, 2048), _lib.MI_OK),
        (RMS, TileConfig(128, 128, 64, 4, 3, variant=14), (2048, 2048, 2044), _lib.MI_E_ALIGN),   # K % 8
        (RMS, TileConfig(128, 128, 64, 4, 1, variant=14), (2048, 2048, 2048), _lib.MI_E_TILE),    # pipelined core
        (RMS, TileConfig(128, 128, 64, 4, 3, split_k=2, variant=14), (512, 512, 8192), _lib.MI_E_SPLIT),
        # variant 15: the two-pass kernel on the paired-load core (its LDS: the core's plus BM row scales)
        (RMS, TileConfig(256, 256, 32, 4, 3, variant=15), (4096, 4096, 4096), _lib.MI_OK),
        (RMS, TileConfig(256, 256, 32, 4, 4, variant=15), (4096, 4096, 4096), _lib.MI_E_LDS),    # 160 KiB + 1 KiB
        (RMS, TileConfig(256, 256, 32, 4, 3, variant=15), (4096, 4096, 4092), _lib.MI_E_ALIGN),  # K % 8
        (RMS, TileConfig(128, 128, 32, 4, 4, split_k=2, variant=15), (512, 512, 8192), _lib.MI_E_SPLIT),
        # variant 16: the paired-load core's legality (block_k 32 or 64, whole pair loads per wave)
        (RMS, TileConfig(256, 256, 32, 8, 3, variant=16), (4096, 4096, 4096), _lib.MI_OK),
        (RMS, TileConfig(256, 256, 32, 8, 3, variant=16), (4096, 4096, 4092), _lib.MI_E_ALIGN),   # K % 8
        (RMS, TileConfig(128, 128, 128, 4, 3, variant=16), (2048, 2048, 2048), _lib.MI_E_TILE),   # block_k 128
        (RMS, TileConfig(128, 128, 32, 4, 4, split_k=2, variant=16), (512, 512, 8192), _lib.MI_E_SPLIT),
    ],
)
def test_cfg_check_codes(kid, cfg, shape, code):
    c = cfg.to_c()
    rc = _lib.lib().mi_cfg_check(kid, ctypes.byref(c), *shape)
    assert rc == code, (rc, _lib.last_error())
    assert (_lib.last_error() == "") == (code == 0)


def test_split_k_variants_are_named_and_legal():
    """The sweep's split-K copies (few output tiles only) round-trip through their names and pass the check."""
    from kernel_library.config import legal_configs, split_k_variants

    c = TileConfig(128, 128, 64, 4, 3, split_k=4, variant=1)
    assert c.name == "bm128_bn128_bk64_w4_s3_v1_k4" and TileConfig.from_name(c.name) == c
    few = legal_configs("matmul_lhsT_rhs", 2048, 1024, 8192)
    split = [x for x in few if x.split_k > 1]
    assert split and all(x.variant in (1, 3, 4) for x in split)
    assert not [x for x in legal_configs("matmul_lhsT_rhs", 8192, 8192, 8192) if x.split_k > 1 and x.block_m >= 128
                and x.block_n >= 128]
    assert split_k_variants("matmul_lhsT_rhs_f32", compiled_configs("matmul_lhsT_rhs_f32"), 16, 16) == []
    rms = [x for x in legal_configs("rmsnorm_matmul", 512, 512, 8192) if x.split_k > 1]
    assert rms and all(x.variant in (4, 5, 11, 12, 13) for x in rms)
    lhs = [x for x in legal_configs("matmul_lhs_rhs", 512, 512, 32768) if x.split_k > 1]
    assert lhs and all(x.variant in (0, 2) for x in lhs)


def test_cfg_check_rejects_unknown_kernel_and_null():
    L = _lib.lib()
    c = TileConfig().to_c()
    assert L.mi_cfg_check(99, ctypes.byref(c), 8, 8, 8) == _lib.MI_E_KERNEL
    assert L.mi_cfg_check(MM, None, 8, 8, 8) == _lib.MI_E_ARGS
    assert L.mi_get_config(MM, 10_000, ctypes.byref(c)) == _lib.MI_E_ARGS


@pytest.mark.parametrize("M,N,K", [(8192, 8192, 8192), (4096, 4096, 4096), (2048, 1024, 8192), (4096, 14336, 1024),
                                   (1024, 4096, 14336), (16, 28672, 8192), (64, 28672, 8192), (128, 28672, 8192),
                                   (256, 512, 512)])
def test_default_configs_are_legal_at_baseline_shapes(M, N, K):
    for fam in ("matmul_lhsT_rhs", "rmsnorm_matmul", "matmul_lhs_rhs"):
        cfg = default_config(fam, M, N, K)
        assert check(fam, cfg, M, N, K)[0] == 0, (fam, cfg)
    assert check("matmul_lhsT_rhs_f32", default_config("matmul_lhsT_rhs_f32", 256, 512, 512), 256, 512, 512)[0] == 0


def test_library_default_is_legal_everywhere():
    """The C default (used when no config is passed and no tuned entry exists)
    is a prebuilt, legal config over skinny, ragged, mid and large shapes,
    including K past the gamma capacity of the register-staged fused kernels."""
    L = _lib.lib()
    for kid in (MM, LHS, RMS, F32):
        for M in (8, 16, 24, 40, 64, 72, 128, 136, 200, 2048, 8192, 16384):
            for N in (8, 136, 4096, 28672):
                for K in (8, 264, 8192, 8200, 16384, 65536):
                    if kid == F32 and M * N * K > 2 ** 30:
                        continue
                    c = _lib.MiTileCfg()
                    assert L.mi_default_config(kid, M, N, K, ctypes.byref(c)) == _lib.MI_OK
                    rc = L.mi_cfg_check(kid, ctypes.byref(c), M, N, K)
                    assert rc == _lib.MI_OK, (kid, M, N, K, TileConfig.from_c(c), _lib.last_error())


@pytest.mark.parametrize("fam,shape,name", [
    ("matmul_lhsT_rhs", (1024, 1024, 1024), "bm64_bn64_bk64_w4_s4_v1"),       # 64x64 fills the CUs; 128x128 gives 64 tiles
    ("matmul_lhsT_rhs", (3072, 3072, 3072), "bm256_bn256_bk32_w4_s3_v1"),     # one round of 144 big tiles beats two of 128x256
    ("matmul_lhsT_rhs", (8192, 8192, 8192), "bm256_bn256_bk32_w4_s3_v1"),
    ("matmul_lhsT_rhs", (8192, 1024, 8192), "bm128_bn256_bk32_w4_s3_v1"),     # 256x256 would give 128 tiles
    ("matmul_lhsT_rhs", (1024, 8192, 16384), "bm256_bn128_bk32_w4_s3_v1"),    # long side along the shorter output side
    ("matmul_lhsT_rhs", (4096, 14336, 1024), "bm128_bn256_bk32_w4_s3_v1"),    # K <= 2048: long side along N
    ("matmul_lhsT_rhs", (640, 10240, 2048), "bm128_bn256_bk32_w4_s3_v1"),
    ("matmul_lhsT_rhs", (2048, 1024, 8192), "bm128_bn128_bk32_w4_s4_v1_k2"),  # small block, long K: 128x128 split fills the chip
    ("matmul_lhsT_rhs", (136, 4096, 4096), "bm128_bn128_bk32_w4_s4_v1_k4"),   # 64x64 from K = 3072 likewise
    ("matmul_lhsT_rhs", (512, 1024, 16384), "bm128_bn128_bk32_w4_s4_v1_k8"),  # not a 256-long block split 16 ways
    ("matmul_lhsT_rhs", (2048, 1024, 4096), "bm64_bn128_bk64_w4_s4_v1"),      # K < 8192: the split's partials cost more
    ("matmul_lhsT_rhs", (1088, 3840, 4096), "bm64_bn256_bk64_w4_s3_v1"),      # 255 tiles of 64x256: one round where 128x128 needs two
    ("matmul_lhsT_rhs", (7616, 2112, 1280), "bm256_bn128_bk32_w4_s3_v1"),     # the other orientation: 510 tiles (2 rounds) against 540
    ("matmul_lhsT_rhs", (896, 1472, 7872), "bm128_bn128_bk32_w4_s4_v1_k2"),  # each part of the split keeps >= 3072 of K
    ("matmul_lhsT_rhs", (512, 960, 4096), "bm64_bn64_bk64_w4_s4_v1_k2"),     # a thin 256 split: short parts, 64x64
    ("matmul_lhsT_rhs", (512, 960, 8192), "bm64_bn128_bk64_w4_s4_v1_k4"),     # ... the 64-wide block from 1792 of K per part
    ("matmul_lhsT_rhs", (384, 1024, 16384), "bm128_bn128_bk32_w4_s4_v1_k8"),  # ... 128x128 from 1536 of K per part
    ("matmul_lhsT_rhs", (512, 4096, 4096), "bm128_bn64_bk64_w4_s4_v1"),       # N >= 4M: 128 along M
    ("matmul_lhsT_rhs", (512, 512, 32768), "bm128_bn128_bk32_w4_s4_v1_k16"),  # few tiles, long K: the largest block a split fills the chip with
    ("matmul_lhsT_rhs", (16, 28672, 8192), "bm32_bn256_bk64_w4_s4_v3_k2"),    # skinny, weight streamed non-temporally, 256 wide in 2 parts
    ("matmul_lhsT_rhs", (32, 14336, 4096), "bm32_bn128_bk64_w4_s4_v3_k2"),    # skinny: least panel bytes per workgroup
    ("matmul_lhsT_rhs", (64, 4096, 4096), "bm64_bn64_bk64_w4_s4_v3_k4"),
    ("matmul_lhsT_rhs", (16, 4096, 8192), "bm32_bn128_bk64_w4_s4_v3_k8"),    # split to fill the CUs
    ("matmul_lhsT_rhs", (32, 2048, 16384), "bm64_bn64_bk64_w4_s4_v3_k8"),
    ("matmul_lhsT_rhs", (64, 12288, 16384), "bm64_bn256_bk64_w4_s3_v3_k4"),
    ("matmul_lhsT_rhs", (96, 8192, 8192), "bm128_bn128_bk32_w4_s4_v3_k4"),
    ("matmul_lhsT_rhs", (96, 4544, 16256), "bm128_bn256_bk32_w4_s3_v3_k8"),  # long K: 256-wide blocks split over K
    ("matmul_lhsT_rhs", (16, 5440, 1216), "bm64_bn64_bk64_w4_s4_v3_k2"),      # short K: every part keeps >= 512 of K
    ("rmsnorm_matmul", (4096, 4096, 4096), "bm128_bn512_bk32_w8_s3_v4"),
    ("rmsnorm_matmul", (4096, 2048, 4096), "bm128_bn256_bk32_w4_s3_v5"),
    ("rmsnorm_matmul", (512, 4096, 8192), "bm128_bn256_bk32_w4_s3_v5_k4"),
    ("rmsnorm_matmul", (1024, 4096, 4096), "bm128_bn128_bk32_w4_s4_v15"),     # one full round of two-pass tiles beats a split
    ("rmsnorm_matmul", (48, 5504, 704), "bm32_bn128_bk64_w4_s3_v11"),         # cached weight, short K: 32-row, unsplit
    ("rmsnorm_matmul", (8, 4096, 3072), "bm32_bn128_bk64_w4_s3_v11_k8"),      # from K = 1024: split to fill the CUs
    ("rmsnorm_matmul", (128, 1024, 5248), "bm32_bn128_bk64_w4_s3_v11_k8"),
    ("rmsnorm_matmul", (768, 8064, 12992), "bm256_bn128_bk64_w4_s3_v13"),     # K > 8192: the estimate, 256 x 128 two-pass
    ("rmsnorm_matmul", (384, 4096, 16384), "bm128_bn512_bk32_w8_s3_v4_k8"),   # K > 8192: one-pass split until gamma fits
    ("rmsnorm_matmul", (64, 4416, 14080), "bm64_bn128_bk64_w4_s3_v11_k4"),    # skinny past K = 8192: split to fill the CUs
    ("rmsnorm_matmul", (16, 9088, 9536), "bm32_bn128_bk128_w4_s3_v11_k2"),    # 32-row split leaving CUs idle: block_k 128
    ("rmsnorm_matmul", (128, 5760, 10944), "bm128_bn128_bk64_w4_s3_v11_k4"),  # 128 rows kept: each part keeps >= 1024 of K
    ("rmsnorm_matmul", (128, 1792, 11008), "bm64_bn128_bk64_w4_s3_v11_k8"),   # and 64-row blocks before a split
    ("matmul_lhs_rhs", (48, 2880, 14912), "bm64_bn128_bk64_w4_s4_v2_k8"),     # skinny lhs: non-temporal 64 x 128, split
    ("matmul_lhs_rhs", (128, 9920, 1600), "bm64_bn128_bk128_w4_s3_v2"),      # skinny lhs, short K: no 800-long parts
    ("matmul_lhs_rhs", (128, 1856, 14272), "bm64_bn128_bk128_w4_s3_v2_k8"),  # ... the 64-row block still split to fill the CUs
    ("rmsnorm_matmul", (2048, 2048, 2048), "bm128_bn128_bk32_w4_s4_v15"),     # x packed in its own layout, the paired-load core
    ("rmsnorm_matmul", (256, 8192, 4096), "bm64_bn128_bk64_w4_s4_v13"),       # x scaled once, then the lhsT core (128x128 grid half idle)
    ("rmsnorm_matmul", (128, 4096, 4096), "bm64_bn128_bk64_w4_s3_v11_k4"),    # skinny, few tiles: 64-row blocks, split
    ("matmul_lhs_rhs", (4096, 14336, 1024), "bm128_bn256_bk32_w4_s3_v1"),     # paired loads of the K-contiguous lhs
    ("matmul_lhs_rhs", (512, 4096, 4096), "bm64_bn128_bk64_w4_s4"),
    ("matmul_lhs_rhs", (512, 2048, 12288), "bm128_bn128_bk64_w4_s3_k4"),     # small block, K >= 8192: 128x128 split
    ("matmul_lhs_rhs", (2048, 2048, 2048), "bm128_bn128_bk32_w4_s4_v1"),     # unsplit 128x128: paired loads, block_k 32
    ("matmul_lhs_rhs", (256, 9216, 16384), "bm256_bn128_bk64_w8_s3_k2"),     # idle 128x128 grid, long K, whole 256-row blocks
    ("matmul_lhs_rhs", (384, 8192, 12288), "bm128_bn128_bk32_w4_s4_v1"),     # ... not with a 256-row tail
    ("matmul_lhsT_rhs", (8, 3072, 12288), "bm32_bn128_bk64_w4_s4_v3_k8"),     # skinny: at most 8 parts
])
def test_library_default_picks_the_measured_winners(fam, shape, name):
    """mi_default_config's rounds-of-tiles estimate reproduces the sweep winners it was fitted to."""
    c = _lib.MiTileCfg()
    from kernel_library.config import kernel_id

    assert _lib.lib().mi_default_config(kernel_id(fam), *shape, ctypes.byref(c)) == _lib.MI_OK
    assert TileConfig.from_c(c).name == name


def test_release_workspace_without_pools_is_a_no_op():
    """Before any call has needed workspace there is no pool: release returns 0 and touches no device."""
    assert _lib.lib().mi_release_workspace() == _lib.MI_OK


def test_library_default_rejects_negative_sizes_and_survives_huge_ones():
    """A negative size is MI_E_ARGS; sizes near INT_MAX still give a config (no overflow in the tile counts)."""
    L = _lib.lib()
    c = _lib.MiTileCfg()
    for kid in (MM, LHS, RMS):
        assert L.mi_default_config(kid, -8, 8, 8, ctypes.byref(c)) == _lib.MI_E_ARGS
        assert L.mi_default_config(kid, 8, 8, -1, ctypes.byref(c)) == _lib.MI_E_ARGS
        for M, N in ((2 ** 31 - 8, 8), (8, 2 ** 31 - 8), (2 ** 31 - 8, 2 ** 31 - 8)):
            assert L.mi_default_config(kid, M, N, 4096, ctypes.byref(c)) == _lib.MI_OK
            assert c.block_m > 0 and c.block_n > 0 and 1 <= c.split_k <= 16


def test_library_default_is_legal_at_large_shapes():
    """Very tall operands (x or lhsT of 1-2 GiB): the default never takes a config whose workspace or
    operand spans the call would reject."""
    L = _lib.lib()
    for kid in (MM, LHS, RMS):
        for M, N, K in ((131072, 4096, 8192), (262144, 1024, 4096), (131072, 256, 8192), (65536, 8192, 16384),
                        (512, 131072, 8192)):
            c = _lib.MiTileCfg()
            assert L.mi_default_config(kid, M, N, K, ctypes.byref(c)) == _lib.MI_OK
            rc = L.mi_cfg_check(kid, ctypes.byref(c), M, N, K)
            assert rc == _lib.MI_OK, (kid, M, N, K, TileConfig.from_c(c), _lib.last_error())


@settings(max_examples=400, deadline=None)
@given(kid=st.sampled_from([MM, LHS, RMS]), m=st.integers(1, 16384), n=st.integers(1, 16384),
       k=st.integers(1, 16384), big=st.sampled_from([1, 1, 1, 8]))
def test_library_default_is_legal_for_random_shapes(kid, m, n, k, big):
    """Property: for any shape the C ABI accepts (M, N multiples of 8, K too for the K-contiguous families,
    operand spans under 4 GiB), the library default is a prebuilt config that mi_cfg_check accepts there."""
    M, N, K = 8 * m * big, 8 * n, 8 * k if kid != MM else k * big
    if 2 * (K + 1024) * max(M, N) >= 2 ** 32 or 2 * (M + 512) * K >= 2 ** 32:
        return  # an operand span past the 32-bit buffer offsets: no config takes it
    c = _lib.MiTileCfg()
    L = _lib.lib()
    assert L.mi_default_config(kid, M, N, K, ctypes.byref(c)) == _lib.MI_OK
    assert L.mi_cfg_check(kid, ctypes.byref(c), M, N, K) == _lib.MI_OK, (kid, M, N, K, TileConfig.from_c(c),
                                                                          _lib.last_error())


@settings(max_examples=300, deadline=None)
@given(m=st.integers(1, 4096), n=st.integers(1, 4096), k=st.integers(1, 65536))
def test_library_default_split_fits_the_noalloc_scratch(m, n, k):
    """With no config, the no-allocation entry point never meets MI_E_RANGE: the default splits only
    grids of at most one workgroup per CU, so its fp32 partials stay within 256 blocks of 256 x 256."""
    M, N, K = 8 * m, 8 * n, k
    c = _lib.MiTileCfg()
    assert _lib.lib().mi_default_config(MM, M, N, K, ctypes.byref(c)) == _lib.MI_OK
    ws = c.split_k * M * N * 4 if c.split_k > 1 else 0
    assert ws <= 64 << 20, (M, N, K, TileConfig.from_c(c).name, ws)


def test_entry_points_reject_bad_arguments_before_any_gpu_call():
    """Negative sizes, null pointers and a non-finite eps are refused on the host; empty outputs are no-ops."""
    L = _lib.lib()
    c = TileConfig(128, 128, 64, 4, 2).to_c()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: every call below returns before a launch
    assert L.mi_matmul_lhsT_rhs_bf16(fake, fake, fake, -1, 8, 8, ctypes.byref(c), None) == _lib.MI_E_ARGS
    assert L.mi_matmul_lhsT_rhs_bf16(fake, fake, None, 8, 8, 8, ctypes.byref(c), None) == _lib.MI_E_ARGS
    assert L.mi_matmul_lhsT_rhs_bf16(None, fake, fake, 8, 8, 8, ctypes.byref(c), None) == _lib.MI_E_ARGS
    assert L.mi_matmul_lhsT_rhs_bf16(fake, fake, fake, 0, 8, 8, ctypes.byref(c), None) == _lib.MI_OK
    assert L.mi_matmul_lhsT_rhs_f32(fake, fake, fake, 8, -8, 8, ctypes.byref(c), None) == _lib.MI_E_ARGS
    assert L.mi_matmul_lhs_rhs_bf16(fake, fake, fake, 8, 8, -8, ctypes.byref(c), None) == _lib.MI_E_ARGS
    assert L.mi_matmul_lhs_rhs_bf16(fake, None, fake, 8, 8, 8, ctypes.byref(c), None) == _lib.MI_E_ARGS
    assert L.mi_matmul_lhs_rhs_bf16(fake, fake, fake, 8, 0, 8, ctypes.byref(c), None) == _lib.MI_OK
    assert L.mi_rmsnorm_matmul_bf16(fake, None, fake, fake, 8, 8, 0, 1e-6, ctypes.byref(c), None) == _lib.MI_E_ARGS
    assert L.mi_rmsnorm_matmul_bf16(fake, None, fake, fake, 8, 8, 8, float("nan"), ctypes.byref(c),
                                    None) == _lib.MI_E_ARGS
    assert L.mi_rmsnorm_matmul_bf16(fake, None, fake, fake, 8, 8, 8, -1.0, ctypes.byref(c), None) == _lib.MI_E_ARGS
    assert L.mi_rmsnorm_matmul_bf16(fake, None, None, fake, 8, 8, 8, 1e-6, ctypes.byref(c), None) == _lib.MI_E_ARGS
    assert "null" in _lib.last_error()
    # an illegal config is refused before the launch as well (operands 128 MiB apart: no overlap)
    bad = TileConfig(256, 256, 128, 8, 2).to_c()
    a, b, o = (ctypes.c_void_p(0x10000000 + i * (1 << 28)) for i in range(3))
    assert L.mi_matmul_lhsT_rhs_bf16(a, b, o, 8192, 8192, 8192, ctypes.byref(bad), None) == _lib.MI_E_LDS


def test_no_gamma_default():
    """mi_default_config_no_gamma: the gamma default, except 128x128, 64x128
    and 64x64 blocks (split or not) at M > 128 go gamma-free, unsplit: 64x128
    and 64x64 to variant 14, 128x128 to the largest block whose grid keeps
    more than half the CUs busy (variant 16 at 128x128, else variant 14 at
    64x128, else at 64x64); always legal where the gamma default is."""
    import random

    from kernel_library.config import default_config

    L = _lib.lib()

    def pick(M, N, K, fn):
        c = _lib.MiTileCfg()
        assert (fn(M, N, K, ctypes.byref(c)) if fn is L.mi_default_config_no_gamma
                else fn(RMS, M, N, K, ctypes.byref(c))) == _lib.MI_OK
        return TileConfig.from_c(c)

    assert pick(2048, 2048, 2048, L.mi_default_config_no_gamma).name == "bm128_bn128_bk32_w4_s4_v16"
    assert pick(1024, 1024, 1024, L.mi_default_config_no_gamma).name == "bm64_bn64_bk64_w4_s4_v14"   # 64 tiles of 128x128
    assert pick(512, 4096, 4096, L.mi_default_config_no_gamma).name == "bm64_bn128_bk64_w4_s4_v14"
    for shape in ((4096, 4096, 4096), (16, 28672, 8192), (128, 28672, 8192), (8192, 8192, 8192)):
        assert pick(*shape, L.mi_default_config_no_gamma) == pick(*shape, L.mi_default_config), shape
    rng = random.Random(5)
    for _ in range(300):
        M, N, K = rng.randint(1, 80) * 64, rng.randint(1, 80) * 64, rng.randint(1, 160) * 64
        ng, g = pick(M, N, K, L.mi_default_config_no_gamma), pick(M, N, K, L.mi_default_config)
        assert check("rmsnorm_matmul", ng, M, N, K)[0] == 0, (M, N, K, ng)
        small = {(128, 128), (64, 128), (64, 64)}
        assert ng == g or (ng.split_k == 1 and ng.variant == (16 if ng.block_m == 128 else 14)
                           and (g.block_m, g.block_n) in small
                           and ((ng.block_m, ng.block_n) == (g.block_m, g.block_n)
                                or (g.block_m, g.block_n) == (128, 128))), (M, N, K, g, ng)
    c = _lib.MiTileCfg()
    assert L.mi_default_config_no_gamma(-1, 8, 8, ctypes.byref(c)) == _lib.MI_E_ARGS
    assert L.mi_default_config_no_gamma(8, 8, 8, None) == _lib.MI_E_ARGS
    # The Python host: the no-gamma tuned entry, else the gamma one, else this default.
    assert default_config("rmsnorm_matmul_online", 2048, 2048, 2048).variant == 16
    assert default_config("rmsnorm_matmul_online", 16, 28672, 8192) == default_config("rmsnorm_matmul", 16, 28672, 8192)
    assert default_config("rmsnorm_matmul_online", 1024, 1024, 1024).name == "bm64_bn64_bk64_w4_s4_v14"


@pytest.mark.parametrize("cfg", [TileConfig(128, 128, 64, 4, 3, variant=14), TileConfig(128, 128, 32, 4, 4, variant=16)],
                         ids=["v14", "v16"])
def test_gamma_free_variant_rejects_gamma_before_any_gpu_call(cfg):
    """rmsnorm_matmul variants 14 and 16 compute the product without gamma: a
    call with gamma is refused with MI_E_TILE on the host, and the sweep of a
    call with gamma never offers them."""
    L = _lib.lib()
    c = cfg.to_c()
    x, g, w, o = (ctypes.c_void_p(0x10000000 + i * (1 << 28)) for i in range(4))
    assert L.mi_rmsnorm_matmul_bf16(x, g, w, o, 2048, 2048, 2048, 1e-6, ctypes.byref(c), None) == _lib.MI_E_TILE
    assert "without gamma" in _lib.last_error()
    from kernel_library.config import legal_configs

    with_g = legal_configs("rmsnorm_matmul", 2048, 2048, 2048)
    without = legal_configs("rmsnorm_matmul", 2048, 2048, 2048, with_gamma=False)
    assert not [x for x in with_g if x.variant == cfg.variant]
    assert [x for x in without if x.variant == cfg.variant]
    assert {x.name for x in with_g} < {x.name for x in without}


def test_entry_points_reject_misaligned_pointers():
    """Kernels move 16-byte vectors (the fp32 one, 4-byte elements): an
    operand not aligned to that is refused with MI_E_ALIGN before any launch
    (for instance a contiguous view at an odd element offset)."""
    L = _lib.lib()
    c = TileConfig(128, 128, 64, 4, 2).to_c()
    ok, odd = ctypes.c_void_p(0x1000), ctypes.c_void_p(0x1002)
    assert L.mi_matmul_lhsT_rhs_bf16(odd, ok, ok, 8, 8, 8, ctypes.byref(c), None) == _lib.MI_E_ALIGN
    assert "16-byte" in _lib.last_error()
    assert L.mi_matmul_lhsT_rhs_bf16(ok, ok, odd, 8, 8, 8, ctypes.byref(c), None) == _lib.MI_E_ALIGN
    assert L.mi_matmul_lhs_rhs_bf16(ok, odd, ok, 8, 8, 8, ctypes.byref(c), None) == _lib.MI_E_ALIGN
    assert L.mi_rmsnorm_matmul_bf16(ok, odd, ok, ok, 8, 8, 8, 1e-6, ctypes.byref(c), None) == _lib.MI_E_ALIGN
    assert L.mi_rmsnorm_matmul_bf16(ok, None, ok, odd, 8, 8, 8, 1e-6, ctypes.byref(c), None) == _lib.MI_E_ALIGN
    assert L.mi_matmul_lhsT_rhs_f32(ctypes.c_void_p(0x1002), ok, ok, 8, 8, 8, ctypes.byref(c), None) == \
        _lib.MI_E_ALIGN


def test_reference_kernel_names_resolve():
    """The reference's kernel names resolve to their families everywhere a family name does."""
    import kernel_library as kl
    from kernel_library.config import canonical_name, kernel_id

    for ref, fam in (("matmul_lhsT_rhs_nkigym", "matmul_lhsT_rhs"), ("matmul_lhs_rhs_nkigym", "matmul_lhs_rhs"),
                     ("rmsnorm_matmul_online", "rmsnorm_matmul")):
        assert canonical_name(ref) == fam and kernel_id(ref) == kernel_id(fam)
        assert kl.legal_configs(ref, 2048, 2048, 2048) == kl.legal_configs(fam, 2048, 2048, 2048)
        assert kl.check(ref, kl.default_config(ref, 3000, 2048, 1000), 3000, 2048, 1000)[0] == 0
    with pytest.raises(ValueError, match="unknown kernel"):
        kernel_id("matmul_nothing")


def test_python_wrappers_validate_on_the_host():
    torch = pytest.importorskip("torch")
    import kernel_library as kl

    a = torch.zeros((64, 32), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="HIP device"):
        kl.matmul_lhsT_rhs(a, a)
    with pytest.raises(TypeError):
        kl.matmul_lhsT_rhs([[1.0]], a)
    with pytest.raises(ValueError):
        kl.rmsnorm_matmul(a, a, eps=1e-6)
    with pytest.raises(ValueError, match="HIP device"):
        kl.matmul_lhs_rhs(a, a.t().contiguous())


def test_c_abi_rejects_an_output_that_overlaps_an_input():
    """The entry points compare pointer ranges on the host (fake pointers, nothing launched)."""
    L = _lib.lib()
    c = TileConfig(128, 128, 64, 4, 2).to_c()
    base = 0x10000000
    p = lambda off: ctypes.c_void_p(base + off)  # noqa: E731
    M = N = K = 64  # 8 KiB per bf16 operand
    assert L.mi_matmul_lhsT_rhs_bf16(p(0), p(1 << 20), p(4096), M, N, K, ctypes.byref(c), None) == _lib.MI_E_ARGS
    assert L.mi_matmul_lhs_rhs_bf16(p(0), p(1 << 20), p((1 << 20) + 8192 - 16), M, N, K, ctypes.byref(c),
                                    None) == _lib.MI_E_ARGS
    assert L.mi_rmsnorm_matmul_bf16(p(0), p(1 << 19), p(1 << 20), p((1 << 19) + 64), M, N, K, 1e-6,
                                    ctypes.byref(c), None) == _lib.MI_E_ARGS   # out over gamma
    assert "overlaps" in _lib.last_error()


def test_output_aliasing_an_input_is_rejected():
    """The wrappers refuse an ``out`` that shares bytes with an input (host-side pointer ranges)."""
    import torch

    from kernel_library.ops import _no_overlap

    buf = torch.zeros(4096, dtype=torch.bfloat16)
    a, b = buf[:1024].view(32, 32), buf[1024:2048].view(32, 32)
    _no_overlap(buf[2048:3072].view(32, 32), lhs=a, rhs=b)            # disjoint: accepted
    _no_overlap(buf[2048:3072].view(32, 32), lhs=a, rhs=b, gamma=None)
    with pytest.raises(ValueError, match="overlaps rhs"):
        _no_overlap(buf[1500:2524].view(32, 32), lhs=a, rhs=b)
    with pytest.raises(ValueError, match="overlaps lhs"):
        _no_overlap(a, lhs=a, rhs=b)


def test_library_needs_no_hip_symbol_newer_than_torchs_runtime():
    """torch loads its own libamdhip64 (ROCm 7.0) first, and the library's
    HIP calls bind to it, so every HIP symbol the library imports must carry
    a version that runtime has: hip_7.0 or older."""
    import re
    import shutil
    import subprocess

    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    out = subprocess.run([nm, "-D", "--undefined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    versions = {tuple(int(x) for x in m.group(1).split(".")) for m in re.finditer(r"@hip_(\d+\.\d+)", out)}
    assert versions, "no versioned HIP imports found"
    assert max(versions) <= (7, 0), sorted(versions)
