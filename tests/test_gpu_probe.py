"""GPU checks of the measurement probes bench.py reports (libmi_probe.so).

The probes are not part of the kernel_library ABI, but the default bench
line depends on them: the clocked twin of the shipped kernel gives the line's
clock, the MFMA probes its ``mfma_ceiling``, and the panel-stream probe the
L2 / fabric ceilings of the profiling workloads.  These tests run each on a
small case: the twin must compute exactly what the product kernel computes
(it is the same body plus two counter reads per workgroup), and every probe
must report a positive rate at a clock inside the chip's range.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import mm_inputs

pytestmark = pytest.mark.gpu


def _dev(a: np.ndarray, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).to(device)


@pytest.mark.parametrize("name", ["bm256_bn256_bk32_w4_s3_v1", "bm64_bn128_bk64_w4_s4_v1"])
def test_clocked_twin_is_bitwise_the_product_kernel(gpu, name):
    import torch

    import kernel_library as kl
    from kernel_library import _probe

    cfg = kl.TileConfig.from_name(name)
    d = mm_inputs(776, 520, 1000, seed=3, dist="uniform")  # K, M, N: ragged against both tiles
    a, b = _dev(d["lhs_T"], gpu), _dev(d["rhs"], gpu)
    ref = kl.matmul_lhsT_rhs(a, b, cfg=cfg)
    out = torch.full_like(ref, float("nan"))
    r = _probe.clocked_lhsT_rhs(a, b, out, cfg, launches=3, warmup=1)
    torch.cuda.synchronize()
    print(name, r)
    assert r is not None
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert 500.0 < r["clock_mhz"] < 2600.0 and r["us"] > 0


def test_mfma_probes_report_a_rate_and_clock(gpu):
    import torch

    from kernel_library import _probe

    src = torch.empty(1 << 20, dtype=torch.bfloat16, device=gpu).uniform_(-1, 1)
    for mode in (0, 1):
        r = _probe.mfma_ceiling(src, mode, iters=16, launches=2, warmup=1)
        print("mfma probe", mode, r)
        assert 0 < r["tflops"] < 2600.0 and 500.0 < r["clock_mhz"] < 2600.0


@pytest.mark.parametrize("row_bytes,pitch", [(1024, 1024), (128, 4096), (256, 57344)])
def test_panel_stream_reports_a_rate(gpu, row_bytes, pitch):
    import torch

    from kernel_library import _probe

    buf = torch.ones(1 << 24, dtype=torch.float32, device=gpu)  # 64 MiB
    region = (2 << 20) // (pitch * (1024 // row_bytes)) * (pitch * (1024 // row_bytes))
    r = _probe.panel_stream(buf, region, 4, 8, rounds=4, row_bytes=row_bytes, pitch=pitch, launches=2, warmup=1)
    print(r)
    assert r["gbs"] > 0 and 500.0 < r["clock_mhz"] < 2600.0
    assert r["bytes_per_clk_per_cu"] < 256.0
