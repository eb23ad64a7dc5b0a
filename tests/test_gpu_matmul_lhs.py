"""GPU parity of matmul_lhs_rhs (lhs[M,K] K-contiguous . rhs[K,N], bf16) against the CPU oracle.

Every call goes through the C ABI (mi_matmul_lhs_rhs_bf16).  Small shapes
compare the whole output with the oracle's float64 closed form; every
config must also be bitwise equal to the lhsT.rhs kernel on the transposed
operand (same tile config, variant 1): the two kernels feed identical MFMA
operands in the same K order and differ only in how the A panel is laid
out in LDS.  The full benchmark shape uses sampled rows against the closed
form, the whole output against a float64 product, and exact linearity.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import mm_check
from oracle import inputs as oinputs
from oracle import matmul as omm

pytestmark = pytest.mark.gpu


def _kl():
    import kernel_library

    return kernel_library


def _inputs(M: int, K: int, N: int, seed: int, dist="uniform") -> dict:
    return oinputs.generate({"lhs": ((M, K), "bfloat16"), "rhs": ((K, N), "bfloat16")}, seed,
                            {"lhs": dist, "rhs": dist})


def _dev(a: np.ndarray, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).to(device)


def _host(t) -> np.ndarray:
    import torch

    return t.to(torch.float32).cpu().numpy()


def _as_lhsT_cfg(cfg):
    """The lhsT.rhs kernel's pipelined variant at the same tile config."""
    kl = _kl()
    return kl.TileConfig(cfg.block_m, cfg.block_n, cfg.block_k, cfg.waves, cfg.lds_stages, cfg.split_k,
                         cfg.group_m, 1)


@pytest.mark.parametrize("M,N,K", [(256, 512, 256), (512, 256, 1024)])
def test_every_config_matches_oracle_and_lhsT_kernel(gpu, M, N, K):
    import torch

    kl = _kl()
    d = _inputs(M, K, N, seed=0)
    a, b = _dev(d["lhs"], gpu), _dev(d["rhs"], gpu)
    aT = a.t().contiguous()
    expected = omm.closed_form_lhs(d["lhs"], d["rhs"])
    cfgs = kl.legal_configs("matmul_lhs_rhs", M, N, K)
    assert len(cfgs) >= 10 and {c.variant for c in cfgs} == {0, 1, 2}
    for cfg in cfgs:
        print("cfg", cfg.name, flush=True)
        out = kl.matmul_lhs_rhs(a, b, cfg=cfg)
        rep = mm_check(_host(out), expected)
        assert rep["ok"], (cfg, rep)
        twin = _as_lhsT_cfg(cfg)
        if kl.check("matmul_lhsT_rhs", twin, M, N, K)[0] == 0:
            ref = kl.matmul_lhsT_rhs(aT, b, cfg=twin)
            assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), cfg


@pytest.mark.parametrize("M,N,K", [(264, 520, 104), (8, 8, 8), (40, 136, 40), (200, 136, 264), (128, 96, 1000)])
def test_ragged_shapes_and_k_tail(gpu, M, N, K):
    """Edge tiles in M and N, and K not a multiple of block_k: the last K tile
    reads zeros past K (never the next row's values)."""
    kl = _kl()
    d = _inputs(M, K, N, seed=3)
    expected = omm.closed_form_lhs(d["lhs"], d["rhs"])
    a, b = _dev(d["lhs"], gpu), _dev(d["rhs"], gpu)
    cfgs = kl.legal_configs("matmul_lhs_rhs", M, N, K)
    assert cfgs
    for cfg in cfgs[:: max(1, len(cfgs) // 8)]:
        print("shape", M, N, K, "cfg", cfg.name, flush=True)
        rep = mm_check(_host(kl.matmul_lhs_rhs(a, b, cfg=cfg)), expected)
        assert rep["ok"], (M, N, K, cfg, rep)


def test_k_tail_never_reads_the_next_row(gpu):
    """With K = 40 (one full 32-column tile plus 8), row r's tail chunk past K
    would be row r+1's first values.  Put inf there: row r must stay finite
    and exact, only row r+1 sees the inf."""
    import torch

    kl = _kl()
    M, N, K = 64, 64, 40
    d = _inputs(M, K, N, seed=4)
    lhs = d["lhs"].copy()
    lhs[1, :8] = np.inf
    keep = np.ones(M, dtype=bool)
    keep[1] = False
    expected = omm.closed_form_lhs(lhs[keep], d["rhs"])
    a, b = _dev(lhs, gpu), _dev(d["rhs"], gpu)
    cfgs = kl.legal_configs("matmul_lhs_rhs", M, N, K)
    assert any(c.block_k == 32 for c in cfgs) and any(c.block_k == 64 for c in cfgs)
    for cfg in cfgs:
        print("cfg", cfg.name, flush=True)
        host = _host(kl.matmul_lhs_rhs(a, b, cfg=cfg))
        torch.cuda.synchronize()
        assert np.all(np.isfinite(host[keep])), cfg
        rep = mm_check(host[keep], expected)
        assert rep["ok"], (cfg, rep)
        assert not np.all(np.isfinite(host[1])), cfg


def test_identity_and_brute_force(gpu):
    kl = _kl()
    K = 64
    rhs = _inputs(8, K, 96, seed=5)["rhs"]
    out = kl.matmul_lhs_rhs(_dev(np.eye(K, dtype=np.float32), gpu), _dev(rhs, gpu))
    assert np.array_equal(_host(out), rhs)
    d = _inputs(16, 24, 32, seed=6)
    out = kl.matmul_lhs_rhs(_dev(d["lhs"], gpu), _dev(d["rhs"], gpu))
    rep = mm_check(_host(out), omm.brute_force(np.ascontiguousarray(d["lhs"].T), d["rhs"]))
    assert rep["ok"], rep


def test_rejects_k_not_multiple_of_8(gpu):
    kl = _kl()
    d = _inputs(64, 36, 64, seed=7)
    with pytest.raises(Exception, match="multiple of 8"):
        kl.matmul_lhs_rhs(_dev(d["lhs"], gpu), _dev(d["rhs"], gpu))


@pytest.mark.parametrize("M,N,K", [(8192, 8192, 8192), (4096, 4096, 4096)])
def test_full_size(gpu, M, N, K):
    """Sampled rows against the oracle, the whole output against a float64
    product on the GPU, exact linearity, and bitwise equality with the
    lhsT.rhs kernel on the transposed operand at the default config."""
    import torch

    kl = _kl()
    print(f"shape M={M} N={N} K={K}", flush=True)
    d = _inputs(M, K, N, seed=0)
    a, b = _dev(d["lhs"], gpu), _dev(d["rhs"], gpu)
    cfg = kl.default_config("matmul_lhs_rhs", M, N, K)
    out = kl.matmul_lhs_rhs(a, b, cfg=cfg)
    host = _host(out)
    rng = np.random.default_rng(1)
    rows = np.unique(np.concatenate([[0, M - 1], rng.integers(0, M, size=24)]))
    rep = mm_check(host[rows], omm.closed_form_lhs(d["lhs"][rows], d["rhs"]))
    print("sampled rows vs oracle", rep)
    assert rep["ok"], rep
    ref = (a.double() @ b.double()).cpu().numpy()
    full = mm_check(host, ref)
    print("full output vs fp64 torch", full)
    assert full["ok"], full
    del ref
    assert torch.equal(kl.matmul_lhs_rhs(a, b * 2, cfg=cfg), out * 2)
    same = kl.matmul_lhsT_rhs(a.t().contiguous(), b, cfg=_as_lhsT_cfg(cfg))
    assert torch.equal(same.view(torch.int16), out.view(torch.int16))
