"""GPU parity against the committed golden fixtures (tests/golden/), through the C ABI."""

from __future__ import annotations

import numpy as np
import pytest

from golden import make_golden
from helpers import F32_ATOL, F32_RTOL, mm_check, rms_check
from oracle import metrics

pytestmark = pytest.mark.gpu


def _dev(a, dtype, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(device).to(dtype)


@pytest.mark.parametrize("name", sorted(n for n in make_golden.FIXTURES if n.startswith("mm_")))
def test_matmul_golden(gpu, name):
    import torch

    import kernel_library as kl

    d = make_golden.load(name)
    dt = torch.float32 if "f32" in name else torch.bfloat16
    a, b = _dev(d["lhs_T"], dt, gpu), _dev(d["rhs"], dt, gpu)
    cfgs = kl.legal_configs("matmul_lhsT_rhs_f32" if dt == torch.float32 else "matmul_lhsT_rhs", a.shape[1],
                            b.shape[1], a.shape[0])
    assert cfgs
    for cfg in cfgs:
        out = kl.matmul_lhsT_rhs(a, b, cfg=cfg).float().cpu().numpy()
        if dt == torch.float32:
            rep = metrics.report(out, d["expected"], atol=F32_ATOL, rtol=F32_RTOL)
            assert rep["allclose"], (name, cfg, rep)
        else:
            rep = mm_check(out, d["expected"])
            assert rep["ok"], (name, cfg, rep)


@pytest.mark.parametrize("name", sorted(n for n in make_golden.FIXTURES if n.startswith("lhs_")))
def test_matmul_lhs_golden(gpu, name):
    import torch

    import kernel_library as kl

    d = make_golden.load(name)
    a, b = _dev(d["lhs"], torch.bfloat16, gpu), _dev(d["rhs"], torch.bfloat16, gpu)
    cfgs = kl.legal_configs("matmul_lhs_rhs", a.shape[0], b.shape[1], a.shape[1])
    assert cfgs
    for cfg in cfgs:
        rep = mm_check(kl.matmul_lhs_rhs(a, b, cfg=cfg).float().cpu().numpy(), d["expected"])
        assert rep["ok"], (name, cfg, rep)


@pytest.mark.parametrize("name", sorted(n for n in make_golden.FIXTURES if n.startswith("rms_")))
def test_rmsnorm_golden(gpu, name):
    import torch

    import kernel_library as kl

    d = make_golden.load(name)
    x, w = _dev(d["lhs"], torch.bfloat16, gpu), _dev(d["rhs"], torch.bfloat16, gpu)
    g = _dev(d["gamma"], torch.bfloat16, gpu) if "gamma" in d else None
    M, K = x.shape
    # Without gamma every variant runs, the gamma-free variant 14 included.
    for cfg in kl.legal_configs("rmsnorm_matmul", M, w.shape[1], K, with_gamma=g is not None):
        out = kl.rmsnorm_matmul(x, w, g, cfg=cfg).float().cpu().numpy()
        rep = rms_check(out, d["expected"])
        assert rep["ok"], (name, cfg, rep)
