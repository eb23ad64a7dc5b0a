"""bench.py's host-side pieces, on the CPU: the seeded shape sets of the default-config study."""

from __future__ import annotations

import importlib.util
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_random_default_shapes_are_seeded_and_in_bounds():
    """Each seed gives the same 30 shapes every time: 14 lhsT.rhs, 6 lhs.rhs and 10 rmsnorm_matmul, every size
    a multiple of 8 that the C ABI accepts, at most 5e11 FLOP each; different seeds give different shapes."""
    b = _bench()
    a1, a2, c = b.random_default_shapes(2028), b.random_default_shapes(2028), b.random_default_shapes(2026)
    assert a1 == a2 and a1 != c and len(a1) == 30
    fams = [f for f, _ in a1]
    assert (fams.count("matmul_lhsT_rhs"), fams.count("matmul_lhs_rhs"), fams.count("rmsnorm_matmul")) == (14, 6, 10)
    for _, (m, n, k) in a1 + c:
        assert m % 8 == 0 and n % 8 == 0 and k % 8 == 0
        assert 8 <= m <= 8192 and 512 <= n <= 14336 and 512 <= k <= 16384
        assert 2.0 * m * n * k <= 5e11
    skinny = sum(1 for _, (m, _, _) in a1 if m <= 128)
    assert 2 <= skinny <= 24  # 1/4 of the draws, more after the FLOP cap's redraws


def test_timed_region_found_between_twin_readings(tmp_path):
    """The rocprof summary of the default bench command takes the timed
    region's dispatches: the one run of exactly --steps product-kernel
    dispatches with a clocked-twin dispatch on each side (settle runs and
    the --warmup run are other lengths).  Checked on a synthetic
    kernel_trace.csv laid out as bench.py launches."""
    import csv

    from autotune.runner.trace import read_kernel_trace, timed_region

    prod = "void mi::mm_lhsT_rhs_bf16_pipe_kernel<256, 256, 32, 4, 3, false, false>(unsigned short const*)"
    twin = "void mi::clocked_lhsT_rhs_kernel<256, 256, 32, 4, 3>(unsigned short const*)"
    rows, t = [], 0
    fill = "void at::native::vectorized_elementwise_kernel<4, at::native::FillFunctor<long>>(int)"
    for name, count, ns in [(prod, 64, 800), (fill, 1, 5), (twin, 11, 900), (prod, 70, 790), (fill, 1, 5),
                            (twin, 11, 900), (prod, 5, 780), (fill, 1, 5), (twin, 11, 900), (prod, 20, 740),
                            (fill, 1, 5), (twin, 11, 900), (prod, 1340, 750)]:
        for _ in range(count):
            rows.append({"Kernel_Name": name, "Start_Timestamp": t, "End_Timestamp": t + ns})
            t += ns + 10
    path = tmp_path / "run_kernel_trace.csv"
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        w.writerows(rows)
    res = timed_region(read_kernel_trace(str(path)), 20)
    assert res["dispatches"] == 20 and res["avg_us"] == 0.74 and "pipe_kernel<256, 256" in res["kernel"]
    with pytest.raises(ValueError):
        timed_region(read_kernel_trace(str(path)), 7)
