"""GPU parity of matmul_lhsT_rhs (bf16 and fp32) against the CPU oracle.

Every call goes through the C ABI of libmi_kernels.so (kernel_library.ops
wraps mi_matmul_lhsT_rhs_*).  Small shapes compare the whole output with the
oracle's float64 closed form; the full benchmark sizes use sampled rows
against the closed form plus size-independent properties (all tile configs
bitwise equal, exact linearity under power-of-two scaling).
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import F32_ATOL, F32_RTOL, mm_check, mm_inputs
from oracle import matmul as omm
from oracle import metrics

pytestmark = pytest.mark.gpu


def _dev(a: np.ndarray, dtype, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(device)


def _host(t) -> np.ndarray:
    import torch

    return t.to(torch.float32).cpu().numpy()


def _kl():
    import kernel_library

    return kernel_library


def test_c1_fp32_matches_closed_form(gpu):
    """benchmark config C1: lhsT[512,256] . rhs[512,512], fp32 N(0,1), seed 0."""
    import torch

    d = mm_inputs(512, 256, 512, seed=0, dist="normal", dtype="float32")
    out = _kl().matmul_lhsT_rhs(_dev(d["lhs_T"], torch.float32, gpu), _dev(d["rhs"], torch.float32, gpu))
    expected = omm.closed_form(d["lhs_T"], d["rhs"])
    rep = metrics.report(_host(out), expected, atol=F32_ATOL, rtol=F32_RTOL)
    print("c1", rep)
    np.testing.assert_allclose(_host(out), expected, atol=F32_ATOL, rtol=F32_RTOL)


@pytest.mark.parametrize("name", ["bm64_bn64_bk16_w4_s1", "bm64_bn64_bk32_w4_s1", "bm64_bn64_bk16_w4_s1_v1",
                                  "bm128_bn128_bk16_w4_s1_v1"])
@pytest.mark.parametrize("M,N,K", [(256, 512, 512), (37, 53, 129), (200, 136, 1000), (1, 1, 1), (130, 70, 2)])
def test_fp32_variants_match_closed_form(gpu, name, M, N, K):
    """Both fp32 kernels (0: sequential FMAs; 1: the fp32 MFMA, two K values
    per step) at C1 and at ragged shapes (odd K, edges in M and N, a single
    element), against the float64 product within C1's tolerance."""
    import torch

    kl = _kl()
    d = mm_inputs(K, M, N, seed=3, dist="normal", dtype="float32")
    out = kl.matmul_lhsT_rhs(_dev(d["lhs_T"], torch.float32, gpu), _dev(d["rhs"], torch.float32, gpu),
                             cfg=kl.TileConfig.from_name(name))
    expected = d["lhs_T"].astype(np.float64).T @ d["rhs"].astype(np.float64)
    np.testing.assert_allclose(_host(out), expected, atol=F32_ATOL, rtol=F32_RTOL)


def test_fp32_mfma_128cube_within_1e4(gpu):
    """The fp32 MFMA kernel on the reference's own 128^3 check (atol=rtol=1e-4)."""
    import torch

    kl = _kl()
    rng = np.random.default_rng(0)
    lhs_T = rng.standard_normal((128, 128)).astype(np.float32)
    rhs = rng.standard_normal((128, 128)).astype(np.float32)
    for name in ("bm64_bn64_bk16_w4_s1_v1", "bm128_bn128_bk16_w4_s1_v1"):
        out = kl.matmul_lhsT_rhs(_dev(lhs_T, torch.float32, gpu), _dev(rhs, torch.float32, gpu),
                                 cfg=kl.TileConfig.from_name(name))
        np.testing.assert_allclose(_host(out), lhs_T.T @ rhs, atol=1e-4, rtol=1e-4)


def test_128cube_fp32_reference_procedure(gpu):
    """test/ops/test_direct_numpy_call.py:32-38: seed 0, 128^3, atol=rtol=1e-4."""
    import torch

    rng = np.random.default_rng(0)
    lhs_T = rng.standard_normal((128, 128)).astype(np.float32)
    rhs = rng.standard_normal((128, 128)).astype(np.float32)
    out = _kl().matmul_lhsT_rhs(_dev(lhs_T, torch.float32, gpu), _dev(rhs, torch.float32, gpu))
    np.testing.assert_allclose(_host(out), lhs_T.T @ rhs, atol=1e-4, rtol=1e-4)


def _streamk_key(cfg, M, N, K, cus):
    """K offsets at which the stream-K plan cuts every output tile (mi_streamk.hpp: unit u = t*KT + kt,
    workgroup w takes units [w*total//grid, (w+1)*total//grid)), as the split-K key; a config whose
    tiles are cut differently gets a key of its own."""
    kt = -(-K // cfg.block_k)
    tiles = -(-M // cfg.block_m) * -(-N // cfg.block_n)
    total = tiles * kt
    grid = min(cus, total)
    starts = {w * total // grid for w in range(grid)}
    cuts = {tuple(u - t * kt for u in range(t * kt, t * kt + kt) if u in starts) for t in range(tiles)}
    if len(cuts) != 1:
        return ("streamk", cfg.name)
    offs = tuple(c * cfg.block_k for c in sorted(cuts.pop()))
    return () if offs == (0,) else offs


def test_bf16_every_config_small_fixture(gpu):
    """The reference's small fixture shape (K=256, M=256, N=512), every compiled config."""
    import torch

    kl = _kl()
    d = mm_inputs(256, 256, 512, seed=0)
    a, b = _dev(d["lhs_T"], torch.bfloat16, gpu), _dev(d["rhs"], torch.bfloat16, gpu)
    expected = omm.closed_form(d["lhs_T"], d["rhs"])
    first = {}
    K = 256
    for cfg in kl.legal_configs("matmul_lhsT_rhs", 256, 512, K):
        out = kl.matmul_lhsT_rhs(a, b, cfg=cfg)
        torch.cuda.synchronize()
        rep = mm_check(_host(out), expected)
        assert rep["ok"], (cfg, rep)
        bits = out.view(torch.int16).cpu().numpy()
        # Same K order in every config (ascending, 16 per MFMA): bitwise equal.
        # Split-K sums fp32 partials over K ranges, so configs are bitwise
        # equal when they split K at the same boundaries.  Variant 4 sums
        # each wave's K sub-steps, then the waves: equal when its split of
        # every K tile into waves' sub-steps is the same.
        # Stream-K (variants 5, 6) sums its parts in K order as split-K does,
        # so it joins the split configs with the same boundaries when every
        # tile is cut at the same K offsets (else it stands alone).
        kts = -(-(-(-K // cfg.block_k)) // cfg.split_k) * cfg.block_k
        key = tuple(range(0, K, kts)) if cfg.split_k > 1 else ()
        if cfg.variant == 4:
            key += ("kw", cfg.block_k // 16 // cfg.waves, cfg.waves)
        if cfg.variant in (5, 6):
            key = _streamk_key(cfg, 256, 512, K, torch.cuda.get_device_properties(gpu).multi_processor_count)
        if key not in first:
            first[key] = (cfg, bits)
        else:
            assert np.array_equal(bits, first[key][1]), (cfg, first[key][0])
    assert () in first and len(first) > 1


@pytest.mark.parametrize("M,N,K", [(264, 520, 100), (8, 8, 7), (40, 136, 33), (16, 1024, 512), (128, 96, 1000)])
def test_bf16_ragged_shapes(gpu, M, N, K):
    """Edge tiles in M, N and K (K not a multiple of block_k): masked stores, zero-filled K tail."""
    import torch

    kl = _kl()
    d = mm_inputs(K, M, N, seed=3)
    a, b = _dev(d["lhs_T"], torch.bfloat16, gpu), _dev(d["rhs"], torch.bfloat16, gpu)
    expected = omm.closed_form(d["lhs_T"], d["rhs"])
    cfgs = kl.legal_configs("matmul_lhsT_rhs", M, N, K)
    assert cfgs
    for cfg in cfgs[:: max(1, len(cfgs) // 12)]:
        out = kl.matmul_lhsT_rhs(a, b, cfg=cfg)
        rep = mm_check(_host(out), expected)
        assert rep["ok"], (M, N, K, cfg, rep)


@pytest.mark.parametrize("M,N,K", [(200, 136, 1040), (8, 8, 7), (264, 520, 100), (1024, 512, 14336)])
def test_kw_variant_ragged_and_deterministic(gpu, M, N, K):
    """Matmul variant 4 (K sub-steps split over the waves, the waves' blocks
    summed in the epilogue) at ragged and long-K shapes, every prebuilt
    config: against the oracle, two runs bitwise equal, and configs that
    split each K tile over the waves the same way bitwise equal."""
    import torch

    kl = _kl()
    d = mm_inputs(K, M, N, seed=11)
    a, b = _dev(d["lhs_T"], torch.bfloat16, gpu), _dev(d["rhs"], torch.bfloat16, gpu)
    expected = omm.closed_form(d["lhs_T"], d["rhs"])
    cfgs = [c for c in kl.legal_configs("matmul_lhsT_rhs", M, N, K) if c.variant == 4 and c.split_k == 1]
    assert cfgs
    first = {}
    for cfg in cfgs:
        print("variant 4", cfg.name, M, N, K, flush=True)
        out = kl.matmul_lhsT_rhs(a, b, cfg=cfg)
        again = kl.matmul_lhsT_rhs(a, b, cfg=cfg)
        torch.cuda.synchronize()
        rep = mm_check(_host(out), expected)
        assert rep["ok"], (M, N, K, cfg, rep)
        assert torch.equal(out, again), cfg
        key = (cfg.block_k // 16 // cfg.waves, cfg.waves)
        bits = out.view(torch.int16).cpu().numpy()
        if key in first:
            assert np.array_equal(bits, first[key][1]), (cfg, first[key][0])
        else:
            first[key] = (cfg, bits)


def test_bf16_identity_and_brute_force(gpu):
    """lhs_T = I gives rhs exactly; a tiny case against the brute-force loop."""
    import torch

    kl = _kl()
    K = 64
    rhs = mm_inputs(K, 8, 96, seed=5)["rhs"]
    out = kl.matmul_lhsT_rhs(_dev(np.eye(K, dtype=np.float32), torch.bfloat16, gpu), _dev(rhs, torch.bfloat16, gpu))
    assert np.array_equal(_host(out), rhs)
    d = mm_inputs(24, 16, 32, seed=6)
    out = kl.matmul_lhsT_rhs(_dev(d["lhs_T"], torch.bfloat16, gpu), _dev(d["rhs"], torch.bfloat16, gpu))
    rep = mm_check(_host(out), omm.brute_force(d["lhs_T"], d["rhs"]))
    assert rep["ok"], rep


def _sampled_check(out_host: np.ndarray, lhs_T: np.ndarray, rhs: np.ndarray, rows: np.ndarray) -> dict:
    exp = omm.closed_form(lhs_T[:, rows], rhs)
    return mm_check(out_host[rows], exp)


@pytest.mark.parametrize(
    "M,N,K,dist",
    [
        (8192, 8192, 8192, "uniform"),  # C2
        (2048, 1024, 8192, "uniform"),  # C4a
        (4096, 14336, 1024, "uniform"),  # C4b
        (1024, 4096, 14336, "uniform"),  # C4c
        (16, 28672, 8192, ("normal", 0.02)),  # C5
        (64, 28672, 8192, ("normal", 0.02)),
        (128, 28672, 8192, ("normal", 0.02)),
    ],
)
def test_bf16_baseline_shapes(gpu, M, N, K, dist):
    """Benchmark shapes (C2, C4, C5) with the default (tuned) config and, at
    C2, every config the benchmark's autotune sweep has shipped or can ship
    (the 256x256 and 128x512 pipelined configs, 2..4 stages, 4 or 8 waves).

    Sampled rows against the oracle's float64 closed form; the whole output
    against a float64 torch product of the same bf16 inputs on the GPU; and
    exact linearity (scaling rhs by 2 scales every output by exactly 2).
    """
    import torch

    kl = _kl()
    print(f"shape M={M} N={N} K={K}", flush=True)
    d = mm_inputs(K, M, N, seed=0, dist=dist)
    a, b = _dev(d["lhs_T"], torch.bfloat16, gpu), _dev(d["rhs"], torch.bfloat16, gpu)
    cfgs = [kl.default_config("matmul_lhsT_rhs", M, N, K)]
    if (M, N, K) == (8192, 8192, 8192):
        cfgs += [kl.TileConfig.from_name(n) for n in C2_SHIPPABLE]
    rng = np.random.default_rng(1)
    rows = np.unique(np.concatenate([[0, M - 1], rng.integers(0, M, size=min(M, 24))]))
    ref = (a.double().t() @ b.double()).cpu().numpy()
    for cfg in cfgs:
        out = kl.matmul_lhsT_rhs(a, b, cfg=cfg)
        host = _host(out)
        rep = _sampled_check(host, d["lhs_T"], d["rhs"], rows)
        print(cfg.name, "sampled rows vs oracle", rep, flush=True)
        assert rep["ok"], (cfg, rep)
        full = mm_check(host, ref)
        print(cfg.name, "full output vs fp64 torch", full, flush=True)
        assert full["ok"], (cfg, full)
        out2 = kl.matmul_lhsT_rhs(a, b * 2, cfg=cfg)
        assert torch.equal(out2, out * 2), cfg


# Configs the C2 sweep has picked on some box (bench.py runs the sweep), and
# their neighbours in the same family.
C2_SHIPPABLE = ("bm256_bn256_bk32_w4_s3_v1", "bm256_bn256_bk32_w4_s4_v1", "bm256_bn256_bk32_w4_s2_v1",
                "bm256_bn256_bk32_w8_s3_v1", "bm256_bn256_bk64_w4_s2_v1", "bm256_bn256_bk64_w8_s2_v1",
                "bm128_bn512_bk32_w8_s3_v1")


def test_empty_contraction_writes_zeros(gpu):
    """K = 0: every family writes an all-zero output (a fill kernel, also for odd M*N)."""
    import torch

    kl = _kl()
    for M, N in ((3, 5), (64, 96)):
        for dt in (torch.bfloat16, torch.float32):
            out = torch.full((M, N), float("nan"), dtype=dt, device=gpu)
            kl.matmul_lhsT_rhs(torch.empty((0, M), dtype=dt, device=gpu), torch.empty((0, N), dtype=dt, device=gpu),
                               out=out)
            torch.cuda.synchronize()
            assert torch.count_nonzero(out).item() == 0, (M, N, dt)
        out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu)
        kl.matmul_lhs_rhs(torch.empty((M, 0), dtype=torch.bfloat16, device=gpu),
                          torch.empty((0, N), dtype=torch.bfloat16, device=gpu), out=out)
        torch.cuda.synchronize()
        assert torch.count_nonzero(out).item() == 0, (M, N)


def test_operands_on_another_device_are_refused(gpu):
    """Every operand must be on the first operand's device: the kernels read raw pointers there."""
    import torch

    kl = _kl()
    a = torch.zeros((64, 32), dtype=torch.bfloat16, device=gpu)
    b = torch.zeros((64, 48), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError, match="device"):
        kl.matmul_lhsT_rhs(a, b, out=torch.empty((32, 48), dtype=torch.bfloat16))
    x = torch.zeros((32, 64), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError, match="device"):
        kl.matmul_lhs_rhs(x, b, out=torch.empty((32, 48), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="device"):
        kl.rmsnorm_matmul(x, b, torch.ones(64, dtype=torch.bfloat16), out=torch.empty((32, 48), dtype=torch.bfloat16,
                                                                                      device=gpu))
