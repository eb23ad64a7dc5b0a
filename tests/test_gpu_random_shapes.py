"""Seeded random shapes x random legal tile configs, for every kernel family, against the oracle.

Each case draws a shape, (M, N) multiples of 8 up to 776 and K from 1 (8 where
the family needs it) to 2056. So there are edge tiles in M and N, and K tails
that are no multiple of block_k. The case then draws one config from
``legal_configs`` at that shape. That list holds split-K copies and, for
lhsT.rhs, the stream-K variants wherever the grid is small. The config runs
twice through the C ABI, and the test checks:

* the whole output against the float64 closed form, within the family's
  tolerance: ``oracle.matmul.closed_form`` (out = lhsT^T . rhs, reference
  kernel_hand_90.92mfu.py:101-131), ``closed_form_lhs`` for the K-contiguous
  lhs, and ``oracle.rmsnorm.closed_form`` (the two-pass form of
  kernel_hand_online.py:5-8);
* both runs bitwise equal, since no kernel's result may depend on how its
  workgroups were scheduled.

Shapes and configs come from ``numpy.random.default_rng(seed)``, so a failing
case replays from the printed line.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import F32_ATOL, F32_RTOL, mm_check, mm_inputs, rms_check, rms_inputs
from oracle import inputs as oinputs
from oracle import matmul as omm
from oracle import metrics
from oracle import rmsnorm as orms

CASES = 24


def _dev(a: np.ndarray, dtype, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(device)


def _host(t) -> np.ndarray:
    import torch

    return t.to(torch.float32).cpu().numpy()


def _shape(rng, k_mult: int) -> tuple[int, int, int]:
    M = 8 * int(rng.integers(1, 98))
    N = 8 * int(rng.integers(1, 98))
    K = k_mult * int(rng.integers(1, 2056 // k_mult + 1))
    return M, N, K


def _pick(rng, cfgs):
    assert cfgs
    return cfgs[int(rng.integers(0, len(cfgs)))]


def _twice(fn):
    """Two runs of ``fn`` into fresh outputs; asserts they are bitwise equal and returns the first."""
    import torch

    a = fn()
    b = fn()
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a.view(torch.int32),
                       b.view(torch.int16) if b.dtype == torch.bfloat16 else b.view(torch.int32))
    return a


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(CASES))
def test_lhsT_rhs_bf16(gpu, seed):
    import torch

    import kernel_library as kl

    rng = np.random.default_rng(1000 + seed)
    M, N, K = _shape(rng, 1)
    cfg = _pick(rng, kl.legal_configs("matmul_lhsT_rhs", M, N, K))
    print(f"[random] matmul_lhsT_rhs bf16 seed={seed} M={M} N={N} K={K} {cfg.name}", flush=True)
    d = mm_inputs(K, M, N, seed=seed)
    a, b = _dev(d["lhs_T"], torch.bfloat16, gpu), _dev(d["rhs"], torch.bfloat16, gpu)
    out = _twice(lambda: kl.matmul_lhsT_rhs(a, b, cfg=cfg))
    rep = mm_check(_host(out), omm.closed_form(d["lhs_T"], d["rhs"]))
    assert rep["ok"], (M, N, K, cfg, rep)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(CASES))
def test_lhs_rhs_bf16(gpu, seed):
    import torch

    import kernel_library as kl

    rng = np.random.default_rng(2000 + seed)
    M, N, K = _shape(rng, 8)
    cfg = _pick(rng, kl.legal_configs("matmul_lhs_rhs", M, N, K))
    print(f"[random] matmul_lhs_rhs bf16 seed={seed} M={M} N={N} K={K} {cfg.name}", flush=True)
    d = oinputs.generate({"lhs": ((M, K), "bfloat16"), "rhs": ((K, N), "bfloat16")}, seed,
                         {"lhs": "uniform", "rhs": "uniform"})
    a, b = _dev(d["lhs"], torch.bfloat16, gpu), _dev(d["rhs"], torch.bfloat16, gpu)
    out = _twice(lambda: kl.matmul_lhs_rhs(a, b, cfg=cfg))
    rep = mm_check(_host(out), omm.closed_form_lhs(d["lhs"], d["rhs"]))
    assert rep["ok"], (M, N, K, cfg, rep)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(CASES))
def test_lhsT_rhs_f32(gpu, seed):
    import torch

    import kernel_library as kl

    rng = np.random.default_rng(3000 + seed)
    M, N, K = _shape(rng, 1)
    cfg = _pick(rng, kl.legal_configs("matmul_lhsT_rhs_f32", M, N, K))
    print(f"[random] matmul_lhsT_rhs fp32 seed={seed} M={M} N={N} K={K} {cfg.name}", flush=True)
    d = mm_inputs(K, M, N, seed=seed, dist="normal", dtype="float32")
    a, b = _dev(d["lhs_T"], torch.float32, gpu), _dev(d["rhs"], torch.float32, gpu)
    out = _twice(lambda: kl.matmul_lhsT_rhs(a, b, cfg=cfg))
    rep = metrics.report(_host(out), omm.closed_form(d["lhs_T"], d["rhs"]), atol=F32_ATOL, rtol=F32_RTOL)
    assert rep["allclose"] and rep["nonfinite"] == 0, (M, N, K, cfg, rep)


@pytest.mark.gpu
@pytest.mark.parametrize("gamma", [True, False], ids=["gamma", "no_gamma"])
@pytest.mark.parametrize("seed", range(CASES))
def test_rmsnorm_matmul(gpu, seed, gamma):
    """With gamma, and without it (the reference's contract, where the no-gamma variant 14 is in the draw)."""
    import torch

    import kernel_library as kl

    rng = np.random.default_rng((4000 if gamma else 5000) + seed)
    M, N, K = _shape(rng, 8)
    cfg = _pick(rng, kl.legal_configs("rmsnorm_matmul", M, N, K, with_gamma=gamma))
    print(f"[random] rmsnorm_matmul gamma={gamma} seed={seed} M={M} N={N} K={K} {cfg.name}", flush=True)
    d = rms_inputs(M, K, N, seed=seed, with_gamma=gamma)
    x, w = _dev(d["lhs"], torch.bfloat16, gpu), _dev(d["rhs"], torch.bfloat16, gpu)
    g = _dev(d["gamma"], torch.bfloat16, gpu) if gamma else None
    out = _twice(lambda: kl.rmsnorm_matmul(x, w, g, cfg=cfg))
    rep = rms_check(_host(out), orms.closed_form(d["lhs"], d["rhs"], d.get("gamma")))
    assert rep["ok"], (M, N, K, cfg, rep)


def test_draws_cover_the_variant_families():
    """The seeded draws above reach split-K and more than one variant per family (CPU: legality only)."""
    import kernel_library as kl

    seen: dict[str, set] = {}
    for fam, base, k_mult, kw in [("matmul_lhsT_rhs", 1000, 1, {}), ("matmul_lhs_rhs", 2000, 8, {}),
                                  ("rmsnorm_matmul", 4000, 8, {"with_gamma": True}),
                                  ("rmsnorm_matmul", 5000, 8, {"with_gamma": False})]:
        for seed in range(CASES):
            rng = np.random.default_rng(base + seed)
            M, N, K = _shape(rng, k_mult)
            cfg = _pick(rng, kl.legal_configs(fam, M, N, K, **kw))
            seen.setdefault(fam, set()).add((cfg.variant, cfg.split_k > 1))
    for fam, s in seen.items():
        assert len({v for v, _ in s}) > 1, (fam, s)
    assert any(split for s in seen.values() for _, split in s)
