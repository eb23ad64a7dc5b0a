"""GPU parity of the fused rmsnorm_matmul kernel against the CPU oracle.

Calls go through mi_rmsnorm_matmul_bf16 (C ABI).  The oracle is the
two-pass closed form in float64 on the same bf16 inputs (reference
kernel_library/rmsnorm_matmul/kernel_hand_online.py:5-8 plus the benchmark's
gamma).  Tolerances are explained in tests/helpers.py.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import rms_check, rms_check_full, rms_closed_form_gpu, rms_inputs
from oracle import rmsnorm as orms

pytestmark = pytest.mark.gpu

# Every variant of the fused kernel (include/mi_kernels.h).
VARIANTS = (0, 1, 4, 5, 11, 12, 13, 15)


def _dev(a, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).to(device)


def _host(t) -> np.ndarray:
    import torch

    return t.to(torch.float32).cpu().numpy()


def _ok(rep) -> bool:
    return rep["ok"]


def test_every_config_small(gpu):
    """M=256, K=512, N=256 with gamma: every compiled config and both variants."""
    import kernel_library as kl

    d = rms_inputs(256, 512, 256, seed=0)
    x, g, w = _dev(d["lhs"], gpu), _dev(d["gamma"], gpu), _dev(d["rhs"], gpu)
    expected = orms.closed_form(d["lhs"], d["rhs"], d["gamma"])
    cfgs = kl.legal_configs("rmsnorm_matmul", 256, 256, 512)
    assert len(cfgs) > 50
    for cfg in cfgs:
        out = kl.rmsnorm_matmul(x, w, g, cfg=cfg)
        rep = rms_check(_host(out), expected)
        assert _ok(rep), (cfg, rep)


def test_no_gamma_is_reference_kernel(gpu):
    """gamma=None is rmsnorm_matmul_online's contract (no weight, EPS=1e-6)."""
    import kernel_library as kl

    d = rms_inputs(128, 256, 192, seed=1, with_gamma=False)
    out = kl.rmsnorm_matmul_online(_dev(d["lhs"], gpu), _dev(d["rhs"], gpu))
    rep = rms_check(_host(out), orms.closed_form(d["lhs"], d["rhs"]))
    assert _ok(rep), rep


@pytest.mark.parametrize("variant", VARIANTS)
def test_no_gamma_every_variant(gpu, variant):
    """gamma=None takes each kernel's no-gamma instance; K = 576 is not a multiple of 64."""
    import kernel_library as kl

    d = rms_inputs(256, 576, 512, seed=5, with_gamma=False)
    x, w = _dev(d["lhs"], gpu), _dev(d["rhs"], gpu)
    expected = orms.closed_form(d["lhs"], d["rhs"])
    cfgs = [c for c in kl.legal_configs("rmsnorm_matmul", 256, 512, 576) if c.variant == variant]
    assert cfgs
    for cfg in cfgs[:: max(1, len(cfgs) // 4)]:
        rep = rms_check(_host(kl.rmsnorm_matmul(x, w, None, cfg=cfg)), expected)
        assert _ok(rep), (cfg, rep)


@pytest.mark.parametrize("variant", VARIANTS)
def test_ragged_and_special_rows(gpu, variant):
    """Edge tiles (M, N not multiples of the block), K not a multiple of block_k; a zero row gives 0."""
    import torch

    import kernel_library as kl

    M, K, N = 200, 264, 136
    d = rms_inputs(M, K, N, seed=2)
    x = d["lhs"].copy()
    x[7] = 0.0           # zero row: out row is exactly 0 (0 * finite rsqrt(eps))
    x[11] = 0.25         # constant row: normalises to 1 -> gamma @ W
    cfgs = [c for c in kl.legal_configs("rmsnorm_matmul", M, N, K) if c.variant == variant]
    for cfg in cfgs[:: max(1, len(cfgs) // 8)]:
        out = kl.rmsnorm_matmul(_dev(x, gpu), _dev(d["rhs"], gpu), _dev(d["gamma"], gpu), cfg=cfg)
        host = _host(out)
        rep = rms_check(host, orms.closed_form(x, d["rhs"], d["gamma"]))
        assert _ok(rep), (cfg, rep)
        assert np.all(host[7] == 0.0)
        torch.cuda.synchronize()


def test_scale_invariance_and_identity_weight(gpu):
    """f(c x) = f(x) for c = 4 (exact in bf16, eps negligible); W = I gives rmsnorm(x) * gamma."""
    import kernel_library as kl

    d = rms_inputs(64, 128, 128, seed=4)
    x, g, w = _dev(d["lhs"], gpu), _dev(d["gamma"], gpu), _dev(d["rhs"], gpu)
    a = _host(kl.rmsnorm_matmul(x, w, g))
    b = _host(kl.rmsnorm_matmul(x * 4, w, g))
    assert np.max(np.abs(a - b)) <= 1e-2 * np.sqrt(np.mean(a * a))
    eye = _dev(np.eye(128, dtype=np.float32), gpu)
    y = _host(kl.rmsnorm_matmul(x, eye, g))
    ref = d["lhs"] * orms.inv_rms(d["lhs"])[:, None] * d["gamma"][None, :]
    rep = rms_check(y, ref)
    assert _ok(rep), rep


def test_baseline_c3_full_size(gpu):
    """Benchmark config C3 (M=K=N=4096, gamma, eps=1e-6), every variant family
    and the configs the C3 sweep ships (the one-pass bm128_bn512_bk32_w8_s3_v4,
    the two-pass v13 blocks, the library default): all 16.7 M outputs against
    a float64 evaluation of the closed form on the GPU, and sampled rows
    against the CPU oracle."""
    import torch

    import kernel_library as kl

    print("C3 4096^3 rmsnorm_matmul", flush=True)
    d = rms_inputs(4096, 4096, 4096, seed=0)
    x, g, w = _dev(d["lhs"], gpu), _dev(d["gamma"], gpu), _dev(d["rhs"], gpu)
    exp_full = rms_closed_form_gpu(x, w, g)
    rng = np.random.default_rng(7)
    rows = np.unique(np.concatenate([[0, 4095], rng.integers(0, 4096, size=24)]))
    expected = orms.closed_form(d["lhs"][rows], d["rhs"], d["gamma"])
    cfgs = [kl.TileConfig(256, 256, 64, 8, 2, variant=0), kl.TileConfig(256, 256, 64, 8, 2, variant=1),
            kl.TileConfig(256, 256, 32, 8, 3, variant=4), kl.TileConfig(256, 256, 64, 4, 2, variant=4),
            kl.TileConfig(256, 256, 32, 8, 3, variant=5), kl.TileConfig(256, 256, 32, 8, 2, variant=5),
            kl.TileConfig(128, 512, 32, 8, 3, variant=4), kl.TileConfig(128, 512, 32, 8, 3, variant=5),
            kl.TileConfig(256, 256, 32, 4, 3, variant=13), kl.TileConfig(256, 256, 32, 4, 4, variant=13),
            kl.TileConfig(128, 512, 32, 8, 3, variant=13), kl.TileConfig(256, 256, 32, 8, 3, variant=13),
            kl.TileConfig(256, 256, 32, 4, 3, variant=15), kl.TileConfig(256, 256, 32, 8, 3, variant=15),
            kl.TileConfig(128, 512, 32, 8, 3, variant=15),
            kl.default_config("rmsnorm_matmul", 4096, 4096, 4096)]
    for cfg in cfgs:
        out_dev = torch.full((4096, 4096), float("nan"), dtype=torch.bfloat16, device=gpu)
        kl.rmsnorm_matmul(x, w, g, cfg=cfg, out=out_dev)
        full = rms_check_full(out_dev, exp_full)
        print(cfg.name, "all outputs vs float64 on the GPU:", full, flush=True)
        assert full["ok"], (cfg, full)
        rep = rms_check(_host(out_dev)[rows], expected)
        print(cfg.name, "sampled rows vs oracle:", rep, flush=True)
        assert _ok(rep), (cfg, rep)


@pytest.mark.parametrize("M,K,N,with_gamma", [(200, 264, 136, True), (200, 264, 136, False), (4096, 4096, 4096, True)])
def test_two_pass_kinds_give_the_same_bits(gpu, M, K, N, with_gamma):
    """Variant 15 (x*gamma packed in x's layout, the paired-load K-contiguous
    core) against variant 13 (packed transposed, the lhsT core): the MFMAs see
    the same bf16 operands in the same K order and the row sums of squares
    are added in the same order, so every config of either gives the same
    bits; all against the float64 closed form too."""
    import torch

    import kernel_library as kl

    print(f"two-pass kinds M={M} K={K} N={N} gamma={with_gamma}", flush=True)
    d = rms_inputs(M, K, N, seed=17, with_gamma=with_gamma)
    x, w = _dev(d["lhs"], gpu), _dev(d["rhs"], gpu)
    g = _dev(d["gamma"], gpu) if with_gamma else None
    ref = kl.rmsnorm_matmul(x, w, g, cfg=kl.TileConfig(256, 256, 32, 4, 3, variant=13))
    full = rms_check_full(ref, rms_closed_form_gpu(x, w, g))
    assert full["ok"], full
    cfgs = [c for c in kl.legal_configs("rmsnorm_matmul", M, N, K) if c.variant in (13, 15) and c.split_k == 1]
    assert len([c for c in cfgs if c.variant == 15]) >= 6
    for cfg in cfgs:
        out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu)
        kl.rmsnorm_matmul(x, w, g, cfg=cfg, out=out)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), cfg


@pytest.mark.parametrize("shape,with_gamma", [((4096, 4096, 4096), True), ((2048, 2048, 2048), False)])
def test_error_within_reference_bf16_semantics(gpu, shape, with_gamma):
    """The kernel's error is no larger than that of the reference kernel's own
    bf16 arithmetic on the same rows: the online recurrence with the scaled
    tile and O rounded to bf16 (kernel_hand_online.py:139-149, 165-192;
    oracle.rmsnorm.online(tile_dtype="bfloat16")), both against the float64
    closed form.  Checked for the configs the benchmark ships (C3 with gamma;
    the reference's 2048^3 without), the library default and the two-pass
    variant; the ratio of the two errors is printed."""
    import kernel_library as kl

    M, N, K = shape
    print(f"reference-semantics bound M={M} N={N} K={K} gamma={with_gamma}", flush=True)
    d = rms_inputs(M, K, N, seed=0, with_gamma=with_gamma)
    gam = d.get("gamma")
    x, w = _dev(d["lhs"], gpu), _dev(d["rhs"], gpu)
    g = _dev(gam, gpu) if with_gamma else None
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(11).integers(0, M, size=30)]))
    closed = orms.closed_form(d["lhs"][rows], d["rhs"], gam)
    ref_bf16 = orms.online(d["lhs"][rows], d["rhs"], gam, tile_dtype="bfloat16")
    ref_err = float(np.max(np.abs(ref_bf16.astype(np.float64) - closed)))
    if with_gamma:
        shipped = [kl.TileConfig.from_name("bm128_bn512_bk32_w8_s3_v4")]
    else:
        shipped = [kl.TileConfig.from_name("bm128_bn128_bk64_w4_s2_v4"),
                   kl.TileConfig.from_name("bm128_bn128_bk64_w4_s3_v14"),
                   kl.TileConfig.from_name("bm256_bn256_bk32_w8_s3_v14"),
                   kl.TileConfig.from_name("bm128_bn128_bk32_w4_s4_v16"),
                   kl.TileConfig.from_name("bm256_bn256_bk32_w8_s3_v16")]
    cfgs = shipped + [kl.TileConfig(256, 256, 32, 4, 3, variant=13)]
    if with_gamma:
        cfgs.append(kl.default_config("rmsnorm_matmul", M, N, K))
    exp_full = rms_closed_form_gpu(x, w, g)
    for cfg in cfgs:
        out_dev = kl.rmsnorm_matmul(x, w, g, cfg=cfg)
        full = rms_check_full(out_dev, exp_full)
        print(cfg.name, "all outputs vs float64 on the GPU:", full, flush=True)
        assert full["ok"], (cfg, full)
        out = _host(out_dev)[rows]
        rep = rms_check(out, closed)
        err = float(np.max(np.abs(out.astype(np.float64) - closed)))
        print(cfg.name, f"max|hip-closed| {err:.4g}  max|reference bf16 - closed| {ref_err:.4g}  "
              f"ratio {err / ref_err:.3f}", rep, flush=True)
        assert _ok(rep), (cfg, rep)
        assert err <= ref_err, (cfg, err, ref_err)


@pytest.mark.parametrize("variant", [14, 16])
def test_no_gamma_variant14_every_config_ragged(gpu, variant):
    """Variants 14 and 16 (no gamma; the rows' sums of squares taken from the
    MFMA A fragments, on the per-tile and the paired-load K-contiguous core):
    every prebuilt config at ragged M, N, K (K not a multiple of block_k, so
    the last K tile's zero-filled chunks must add nothing; an odd number of K
    tiles, so the paired loads end on a half pair), with a zero row (exactly
    0), a constant row and a row of large values, every output against the
    closed form."""
    import kernel_library as kl

    M, K, N = 200, 264, 136
    d = rms_inputs(M, K, N, seed=12, with_gamma=False)
    x = d["lhs"].copy()
    x[7] = 0.0
    x[11] = 0.25
    x[13] *= 64.0
    expected = orms.closed_form(x, d["rhs"])
    xd, wd = _dev(x, gpu), _dev(d["rhs"], gpu)
    cfgs = [c for c in kl.legal_configs("rmsnorm_matmul", M, N, K, with_gamma=False) if c.variant == variant]
    assert len(cfgs) >= 8
    for cfg in cfgs:
        print(f"v{variant} ragged", cfg.name, flush=True)
        host = _host(kl.rmsnorm_matmul(xd, wd, None, cfg=cfg))
        rep = rms_check(host, expected)
        assert _ok(rep), (cfg, rep)
        assert np.all(host[7] == 0.0)


@pytest.mark.parametrize("names", [("bm128_bn128_bk64_w4_s3_v14", "bm64_bn64_bk64_w4_s4_v14", "bm256_bn128_bk64_w8_s3_v14"),
                                   ("bm128_bn128_bk32_w4_s4_v16", "bm256_bn128_bk32_w8_s3_v16",
                                    "bm128_bn256_bk64_w4_s2_v16", "bm256_bn256_bk32_w8_s3_v16")], ids=["v14", "v16"])
def test_no_gamma_variant14_identity_weight(gpu, names):
    """W = I isolates the row statistics: out = bf16(x / rms(x)) for every
    row, at K = 1024 (16 or 32 K tiles, both halves of every A fragment
    used; with 8 waves the row sums come from two or four wave columns)."""
    import kernel_library as kl

    M, K = 256, 1024
    d = rms_inputs(M, K, K, seed=13, with_gamma=False)
    x = d["lhs"]
    eye = _dev(np.eye(K, dtype=np.float32), gpu)
    ref = x * orms.inv_rms(x)[:, None]
    for name in names:
        y = _host(kl.rmsnorm_matmul(_dev(x, gpu), eye, None, cfg=kl.TileConfig.from_name(name)))
        rep = rms_check(y, ref)
        print("identity", name, rep, flush=True)
        assert _ok(rep), (name, rep)


@pytest.mark.parametrize("M,K,N", [(1024, 1024, 1024), (512, 4096, 4096), (200, 264, 136)])
def test_no_gamma_default_calls(gpu, M, K, N):
    """Calls without gamma and without a config: the Python host's default
    (rmsnorm_matmul_online) and the C ABI's own (cfg = NULL, gamma = NULL:
    mi_default_config_no_gamma: variant 16 or 14 at these shapes), every output
    against the closed form; both defaults run the same config, so the two
    outputs are bitwise equal."""
    import ctypes

    import torch

    import kernel_library as kl
    from kernel_library import _lib

    d = rms_inputs(M, K, N, seed=21, with_gamma=False)
    x, w = _dev(d["lhs"], gpu), _dev(d["rhs"], gpu)
    a = kl.rmsnorm_matmul_online(x, w)
    b = torch.empty_like(a)
    rc = _lib.lib().mi_rmsnorm_matmul_bf16(x.data_ptr(), None, w.data_ptr(), b.data_ptr(), M, N, K,
                                           ctypes.c_float(kl.EPS), None,
                                           torch.cuda.current_stream(gpu).cuda_stream)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    rep = rms_check(_host(a), orms.closed_form(d["lhs"], d["rhs"]))
    print(M, K, N, kl.default_config("rmsnorm_matmul_online", M, N, K).name, rep, flush=True)
    assert _ok(rep), rep
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_skinny_decode_shape(gpu):
    """Decode-sized M (16 rows) against an 8192 x 28672 W: the non-temporal-W
    variants 11 / 12 and the default config, every row vs the closed form."""
    import kernel_library as kl

    M, K, N = 16, 8192, 28672
    print("skinny rmsnorm_matmul", M, K, N, flush=True)
    d = rms_inputs(M, K, N, seed=3)
    x, g, w = _dev(d["lhs"], gpu), _dev(d["gamma"], gpu), _dev(d["rhs"], gpu)
    expected = orms.closed_form(d["lhs"], d["rhs"], d["gamma"])
    cfgs = [kl.default_config("rmsnorm_matmul", M, N, K), kl.TileConfig(128, 128, 32, 4, 3, variant=11),
            kl.TileConfig(64, 128, 64, 4, 2, variant=11), kl.TileConfig(128, 128, 32, 4, 3, variant=12),
            kl.TileConfig(32, 128, 128, 4, 3, variant=11), kl.TileConfig(32, 128, 64, 4, 3, variant=11)]
    for cfg in cfgs:
        rep = rms_check(_host(kl.rmsnorm_matmul(x, w, g, cfg=cfg)), expected)
        assert _ok(rep), (cfg, rep)
