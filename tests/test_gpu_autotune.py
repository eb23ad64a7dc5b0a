"""GPU end-to-end of the autotune loop: profile() -> results.json -> selection.

Mirrors the reference's driver contract (autotune/src/autotune/runner/api.py:24-75,
output.py:218-271): per-kernel failures become result rows, never
exceptions; results.json names the fastest kernel; a config that is not
prebuilt is built by hipcc and then timed like the others; the detailed
profile keeps a rocprofv3 kernel trace per kernel.  The JIT-built library's
output is checked against the oracle, so the generated unit is the same
kernel as the prebuilt one.
"""

from __future__ import annotations

import json
import os

import pytest

from helpers import mm_check
from oracle import matmul as omm

pytestmark = pytest.mark.gpu


def test_profile_sweep_selection_failures_and_traces(gpu, tmp_path):
    import torch

    from autotune.runner.api import profile
    from autotune.runner.benchmark import generate_tensors
    from autotune.tune import default_dists, input_specs, make_jobs
    from kernel_library import _lib
    from kernel_library.config import TileConfig

    M = N = K = 512
    prebuilt = [TileConfig(128, 128, 64, 4, 2, variant=1), TileConfig(256, 256, 32, 4, 3, variant=1)]
    jit = TileConfig(512, 128, 32, 8, 1)                       # legal, not prebuilt: built by hipcc here
    illegal = TileConfig(256, 256, 128, 8, 2)                  # 256 KiB of LDS panels
    jobs = make_jobs("matmul_lhsT_rhs", M, N, K, prebuilt + [jit, illegal])
    cache = str(tmp_path / "cache")
    print("profiling", list(jobs), flush=True)
    out = profile(jobs, cache, 0, "gfx950", True, warmup=2, reps=5)
    by = {r.kernel_name: r for r in out.results}
    assert len(by) == 4
    assert not by[f"{illegal.name}.hip"].hardware_output.startswith("[")
    assert "LDS" in by[f"{illegal.name}.hip"].hardware_output
    ok = [r for r in out.results if r.hardware_output.startswith("[")]
    assert len(ok) == 3
    assert by[f"{jit.name}.hip"].profiler_summary["library"] != str(_lib.LIB_PATH)

    doc = json.load(open(os.path.join(cache, "results.json")))
    times = {k["kernel_name"]: k for k in doc["kernels"]}
    assert doc["metadata"]["num_kernels"] == 4
    best = min(ok, key=lambda r: r.profiler_summary["total_time"])
    assert doc["metrics"]["best_kernel"] == best.kernel_name
    assert doc["metrics"]["best_total_time_s"] == pytest.approx(best.profiler_summary["total_time"])
    assert len(times) == 4

    for r in ok:
        stem = r.kernel_name[:-len(".hip")]
        folder = os.path.join(cache, stem)
        assert os.path.exists(os.path.join(folder, f"{stem}.hip"))
        assert os.path.exists(os.path.join(folder, "profile_summary.json"))
        detailed = json.load(open(os.path.join(folder, "profile.json")))
        assert len(detailed["times_s"]) == 5
        row = detailed["rocprof"]
        print(stem, row.get("avg_ns"), row.get("error"), flush=True)
        assert "error" not in row, row
        assert row["calls"] == 2 + 5 and row["avg_ns"] > 0
        assert os.path.exists(os.path.join(folder, "rocprof", "run_kernel_stats.csv"))

    # the JIT-built library computes the same product
    specs = input_specs("matmul_lhsT_rhs", M, N, K)
    host = generate_tensors(specs, 0, default_dists("matmul_lhsT_rhs", K))
    lib = _lib.load(by[f"{jit.name}.hip"].profiler_summary["library"])
    a = torch.from_numpy(host["lhs_T"]).to(torch.bfloat16).to(gpu)
    b = torch.from_numpy(host["rhs"]).to(torch.bfloat16).to(gpu)
    o = torch.empty((M, N), dtype=torch.bfloat16, device=gpu)
    import ctypes

    c = jit.to_c()
    rc = lib.mi_matmul_lhsT_rhs_bf16(a.data_ptr(), b.data_ptr(), o.data_ptr(), M, N, K, ctypes.byref(c),
                                     torch.cuda.current_stream(gpu).cuda_stream)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    # the oracle takes the bf16-rounded values the kernel sees
    rep = mm_check(o.float().cpu().numpy(), omm.closed_form(a.float().cpu().numpy(), b.float().cpu().numpy()))
    assert rep["ok"], rep


def test_tune_picks_a_passing_winner(gpu):
    from autotune.tune import tune

    res = tune("matmul_lhs_rhs", 1024, 1024, 1024, reps=5, warmup=2, finalists=3, rounds=2)
    assert res.best is not None and res.check["pass"], res.check
    assert res.best_time_s > 0
