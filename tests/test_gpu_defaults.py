"""GPU parity of calls that pass no config, at shapes without a tuned entry.

Such a call runs the library default (``mi_default_config``): a block chosen
by its estimated rounds-of-tiles time, split-K when the grid leaves CUs
idle, the paired-load lhs blocks, the two-pass fused kernel, and for skinny M
the non-temporal blocks (256-wide and split over a long K, or the block with
the most tiles).  Each case checks that the default is the config the estimate is
meant to pick (so the case exercises that path), then the whole output
against a float64 product of the same bf16 inputs on the GPU and sampled
rows against the CPU oracle.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import mm_check, mm_inputs, rms_check, rms_inputs
from oracle import matmul as omm
from oracle import rmsnorm as orms

pytestmark = pytest.mark.gpu


def _dev(a: np.ndarray, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).to(device)


def _host(t) -> np.ndarray:
    import torch

    return t.to(torch.float32).cpu().numpy()


def _rows(M: int) -> np.ndarray:
    return np.unique(np.concatenate([[0, M - 1], np.random.default_rng(5).integers(0, M, size=min(M, 16))]))


@pytest.mark.parametrize("fam,shape,expect", [
    ("matmul_lhsT_rhs", (1000, 2000, 3000), "bm64_bn128_bk64_w4_s4_v1"),
    ("matmul_lhsT_rhs", (512, 512, 32768), "bm128_bn128_bk32_w4_s4_v1_k16"),
    ("matmul_lhsT_rhs", (96, 4544, 16256), "bm128_bn256_bk32_w4_s3_v3_k8"),
    ("matmul_lhsT_rhs", (3072, 3072, 3072), "bm256_bn256_bk32_w4_s3_v1"),
    ("matmul_lhsT_rhs", (200, 4096, 4096), "bm128_bn128_bk32_w4_s4_v1_k4"),
    ("matmul_lhsT_rhs", (1088, 3712, 8000), "bm64_bn256_bk64_w4_s3_v1"),
    ("matmul_lhsT_rhs", (512, 960, 4096), "bm64_bn64_bk64_w4_s4_v1_k2"),
    ("matmul_lhsT_rhs", (16, 8192, 8192), "bm32_bn128_bk64_w4_s4_v3_k4"),
    ("matmul_lhsT_rhs", (32, 2048, 16384), "bm64_bn64_bk64_w4_s4_v3_k8"),
    ("matmul_lhsT_rhs", (640, 10240, 2048), "bm128_bn256_bk32_w4_s3_v1"),
    ("matmul_lhsT_rhs", (8, 9344, 6336), "bm32_bn256_bk64_w4_s4_v3_k4"),
    ("matmul_lhs_rhs", (2048, 4096, 1024), "bm128_bn256_bk32_w4_s3_v1"),
    ("matmul_lhs_rhs", (512, 4096, 4096), "bm64_bn128_bk64_w4_s4"),
    ("matmul_lhs_rhs", (1536, 1536, 6144), "bm128_bn128_bk32_w4_s4_v1"),
    ("matmul_lhs_rhs", (256, 9216, 16384), "bm256_bn128_bk64_w8_s3_k2"),
    ("matmul_lhs_rhs", (48, 2880, 14912), "bm64_bn128_bk64_w4_s4_v2_k8"),
])
def test_matmul_without_config(gpu, fam, shape, expect):
    import torch

    import kernel_library as kl

    M, N, K = shape
    print(fam, shape, flush=True)
    assert kl.default_config(fam, M, N, K).name == expect
    d = mm_inputs(K, M, N, seed=4, dist="uniform")
    a, b = _dev(d["lhs_T"], gpu), _dev(d["rhs"], gpu)
    if fam == "matmul_lhs_rhs":
        out = kl.matmul_lhs_rhs(a.t().contiguous(), b)
    else:
        out = kl.matmul_lhsT_rhs(a, b)
    host = _host(out)
    full = mm_check(host, (a.double().t() @ b.double()).cpu().numpy())
    print("full output vs fp64 torch", full, flush=True)
    assert full["ok"], full
    rows = _rows(M)
    rep = mm_check(host[rows], omm.closed_form(d["lhs_T"][:, rows], d["rhs"]))
    print("sampled rows vs oracle", rep, flush=True)
    assert rep["ok"], rep


@pytest.mark.parametrize("shape,expect", [
    ((256, 8192, 4096), "bm64_bn128_bk64_w4_s4_v13"),
    ((128, 4096, 4096), "bm64_bn128_bk64_w4_s3_v11_k4"),
    ((256, 4096, 4096), "bm64_bn128_bk64_w4_s4_v13_k2"),
    ((256, 2048, 2048), "bm64_bn128_bk64_w4_s4_v13_k4"),
    ((512, 4096, 8192), "bm128_bn256_bk32_w4_s3_v5_k4"),
    ((1024, 4096, 4096), "bm128_bn128_bk32_w4_s4_v15"),
    ((48, 5504, 704), "bm32_bn128_bk64_w4_s3_v11"),
    ((8, 4096, 3072), "bm32_bn128_bk64_w4_s3_v11_k8"),
    ((768, 8064, 12992), "bm256_bn128_bk64_w4_s3_v13"),
    ((384, 4096, 16384), "bm128_bn512_bk32_w8_s3_v4_k8"),
    ((128, 1792, 11008), "bm64_bn128_bk64_w4_s3_v11_k8"),
    ((16, 9088, 9536), "bm32_bn128_bk128_w4_s3_v11_k2"),
    ((128, 7552, 5952), "bm128_bn128_bk64_w4_s3_v11_k4"),
    ((640, 2048, 1024), None),
])
def test_rmsnorm_matmul_without_config(gpu, shape, expect):
    import kernel_library as kl

    M, N, K = shape
    print("rmsnorm_matmul", shape, flush=True)
    if expect is not None:
        assert kl.default_config("rmsnorm_matmul", M, N, K).name == expect
    d = rms_inputs(M, K, N, seed=6)
    x, g, w = _dev(d["lhs"], gpu), _dev(d["gamma"], gpu), _dev(d["rhs"], gpu)
    out = kl.rmsnorm_matmul(x, w, g)
    host = _host(out)
    xd, gd, wd = x.double(), g.double(), w.double()
    exp = ((xd * (xd * xd).mean(dim=1, keepdim=True).add(1e-6).rsqrt()) * gd[None, :]) @ wd
    full = rms_check(host, exp.cpu().numpy())
    print("full output vs fp64 torch", full, flush=True)
    assert full["ok"], full
    rows = _rows(M)
    rep = rms_check(host[rows], orms.closed_form(d["lhs"][rows], d["rhs"], d["gamma"]))
    print("sampled rows vs oracle", rep, flush=True)
    assert rep["ok"], rep
