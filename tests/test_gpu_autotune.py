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
        # counter passes: measured MFMA busy, engine clock and HBM-side bytes
        c = detailed["counters"]
        print(stem, {k: c.get(k) for k in ("mfma_busy_percent", "engine_clock_mhz", "hbm_gbps", "error")},
              flush=True)
        assert "error" not in c, c
        compulsory = (M * K + K * N + M * N) * 2
        assert 0.5 * compulsory < c["hbm_bytes"] < 64 * compulsory, (c["hbm_bytes"], compulsory)
        assert times[r.kernel_name]["hbm_gbps_measured"] == pytest.approx(c["hbm_gbps"])
        assert "engine_clock_mhz" not in c and "note" in c     # 512^3 calls are too short to clock
        # the compiled artifact and the trace, base64 (the reference's neff_b64 / ntff_b64)
        import base64

        co = base64.b64decode(r.neff_b64)
        assert co[:4] == b"\x7fELF", stem
        trace = base64.b64decode(r.ntff_b64).decode()
        assert trace.splitlines()[0].count(",") > 3 and "mi::" in trace, trace[:300]
    assert by[f"{illegal.name}.hip"].neff_b64 is None and by[f"{illegal.name}.hip"].ntff_b64 is None

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


def test_counters_of_a_long_kernel(gpu, tmp_path):
    """The counter passes on a call long enough to clock (4096^3, ~100 us):
    MFMA busy, engine clock and HBM bytes in physical ranges, and in
    results.json beside the timing."""
    from autotune.runner.api import profile
    from autotune.tune import make_jobs
    from kernel_library.config import TileConfig

    M = N = K = 4096
    jobs = make_jobs("matmul_lhsT_rhs", M, N, K, [TileConfig(256, 256, 32, 4, 3, variant=1)])
    cache = str(tmp_path / "cache")
    out = profile(jobs, cache, 0, "gfx950", True, warmup=3, reps=10)
    r = out.results[0]
    assert r.hardware_output.startswith("["), r.hardware_output
    c = r.profile_detailed["counters"]
    print("4096^3 counters", {k: c.get(k) for k in ("mfma_busy_percent", "engine_clock_mhz", "hbm_gbps")},
          flush=True)
    assert "error" not in c, c
    assert 20.0 < c["mfma_busy_percent"] <= 100.0
    assert 500.0 < c["engine_clock_mhz"] <= 2450.0
    compulsory = 3 * M * N * 2
    assert 0.9 * compulsory < c["hbm_bytes"] < 16 * compulsory
    doc = json.load(open(os.path.join(cache, "results.json")))
    assert doc["kernels"][0]["mfma_busy_percent"] == pytest.approx(c["mfma_busy_percent"])
    assert doc["kernels"][0]["engine_clock_mhz"] == pytest.approx(c["engine_clock_mhz"])
    assert "busy" in str(out) and "MHz" in str(out)


def test_tune_picks_a_passing_winner(gpu):
    from autotune.tune import tune

    res = tune("matmul_lhs_rhs", 1024, 1024, 1024, reps=5, warmup=2, finalists=3, rounds=2)
    assert res.best is not None and res.check["pass"], res.check
    assert res.best_time_s > 0


@pytest.mark.parametrize("M,N,K", [(2048, 1024, 8192), (1024, 4096, 14336)])
def test_tune_at_c4_shapes(gpu, M, N, K):
    """The autotune sweep BASELINE's config 4 asks for, at two of its shapes:
    every legal prebuilt config (split-K and stream-K copies included at
    C4a) through the numerics gate, the winner re-checked, and the winner no
    slower than the shipped tuned-table config timed in the same way."""
    import statistics

    import torch

    import kernel_library as kl
    from autotune.runner.benchmark import Launcher, generate_tensors, time_launches, upload
    from autotune.tune import default_dists, input_specs, tune
    from kernel_library import _lib

    print(f"tune matmul_lhsT_rhs {M}x{N}x{K}", flush=True)
    res = tune("matmul_lhsT_rhs", M, N, K, reps=10, warmup=3, finalists=4, rounds=3)
    assert res.best is not None and res.check["pass"], res.check
    assert len(res.output.successes) >= 40
    shipped = kl.default_config("matmul_lhsT_rhs", M, N, K)
    specs = input_specs("matmul_lhsT_rhs", M, N, K)
    d = upload(generate_tensors(specs, 0, default_dists("matmul_lhsT_rhs", K)), specs, torch.device(gpu))
    out = torch.empty((M, N), dtype=torch.bfloat16, device=gpu)
    # The two configs are timed in alternating rounds, so that neither sees
    # only the clock state the sweep left behind.
    launches = {cfg.name: Launcher(_lib.lib(), "matmul_lhsT_rhs", cfg, d, out, M, N, K) for cfg in (res.best, shipped)}
    rounds: dict[str, list[float]] = {name: [] for name in launches}
    for _ in range(5):
        for name, launch in launches.items():
            rounds[name].append(statistics.median(time_launches(launch, 5, 20)))
    t = {name: statistics.median(v) for name, v in rounds.items()}
    print(f"winner {res.best.name} {t[res.best.name] * 1e6:.1f} us, tuned table {shipped.name} "
          f"{t[shipped.name] * 1e6:.1f} us", flush=True)
    # One box's timing noise between two near-equal configs, not a ranking.
    assert t[res.best.name] <= 1.10 * t[shipped.name]


def test_vendor_baseline_matches_oracle(gpu):
    """The vendor rows (hipBLASLt for the matmuls; torch's unfused rmsnorm then
    hipBLASLt for the fused kernel) compute the same function as the kernels:
    their outputs against the oracle's float64 closed forms."""
    import torch

    from autotune.runner.baseline import profile_torch_baseline
    from autotune.runner.benchmark import generate_tensors
    from autotune.tune import default_dists, input_specs
    from helpers import rms_check
    from oracle import rmsnorm as orms

    M, N, K = 256, 384, 512
    for fam in ("matmul_lhsT_rhs", "matmul_lhs_rhs", "rmsnorm_matmul"):
        print("vendor baseline", fam, flush=True)
        dists = default_dists(fam, K)
        out = torch.empty((M, N), dtype=torch.bfloat16, device=gpu)
        r = profile_torch_baseline(M, N, K, seed=3, warmup=2, reps=5, dists=dists, func_name=fam, out=out,
                                   lhs_layout="MK" if fam == "matmul_lhs_rhs" else "KM")
        assert r.hardware_output.startswith("["), r.hardware_output
        assert r.profiler_summary["numerics"]["pass"], r.profiler_summary["numerics"]
        host = {k: torch.from_numpy(v).to(torch.bfloat16).float().numpy()
                for k, v in generate_tensors(input_specs(fam, M, N, K), 3, dists).items()}
        got = out.float().cpu().numpy()
        if fam == "matmul_lhsT_rhs":
            rep = mm_check(got, omm.closed_form(host["lhs_T"], host["rhs"]))
        elif fam == "matmul_lhs_rhs":
            rep = mm_check(got, omm.closed_form(host["lhs"].T, host["rhs"]))
        else:
            rep = rms_check(got, orms.closed_form(host["lhs"], host["rhs"], host["gamma"]))
        assert rep["ok"], (fam, rep)


def test_tune_from_frontier_sample_and_gate(gpu, tmp_path):
    """The frontier sampler's configs (prebuilt and just-in-time built) go
    through tune(): none is a compile error, every success passed the
    numerics gate, the winner matches the oracle, and the vendor row is in
    results.json beside them."""
    import numpy as np
    import torch

    import kernel_library as kl
    from autotune.runner.benchmark import Launcher, generate_tensors, upload
    from autotune.search import TileMDP, frontier_sample
    from autotune.tune import default_dists, input_specs, tune
    from kernel_library import _lib

    M, N, K = 512, 768, 1024
    cfgs = frontier_sample(TileMDP("matmul_lhsT_rhs", M, N, K), 10, seed=3)
    print("frontier sample", [c.name for c in cfgs], flush=True)
    cache = str(tmp_path / "tune")
    res = tune("matmul_lhsT_rhs", M, N, K, cfgs, cache_dir=cache, warmup=2, reps=5, finalists=3, rounds=2,
               baseline=True)
    for r in res.output.results:
        assert "hipcc failed" not in r.hardware_output and "illegal config" not in r.hardware_output, r
    assert res.best is not None and res.check["pass"], res.check
    for r in res.output.results:
        if r.profiler_summary:
            assert r.profiler_summary["numerics"]["pass"]
    doc = json.load(open(os.path.join(cache, "results.json")))
    assert doc["baseline"]["kernel_name"] == "vendor_matmul_lhsT_rhs"
    assert doc["baseline"]["numerics"]["pass"]
    assert doc["metrics"]["best_speedup_vs_baseline"] > 0
    winner = next(r for r in res.output.results if r.profiler_summary and
                  kl.TileConfig(**r.profiler_summary["config"]) == res.best)
    specs = input_specs("matmul_lhsT_rhs", M, N, K)
    host = generate_tensors(specs, 0, default_dists("matmul_lhsT_rhs", K))
    dev = upload(host, specs, gpu)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=gpu)
    Launcher(_lib.load(winner.profiler_summary["library"]), "matmul_lhsT_rhs", res.best, dev, out, M, N, K)()
    torch.cuda.synchronize()
    a = dev["lhs_T"].float().cpu().numpy()
    b = dev["rhs"].float().cpu().numpy()
    rep = mm_check(out.float().cpu().numpy(), omm.closed_form(a, b))
    assert rep["ok"], rep
    assert np.isfinite(out.float().cpu().numpy()).all()


def test_gate_turns_a_wrong_output_into_a_failure_row(gpu):
    """A candidate whose output disagrees with the golden is a failure row
    with its report, not a success.  The mistake is planted in the golden
    (the host-side expected values, doubled); the kernel is correct."""
    import torch

    from autotune.runner import golden
    from autotune.runner.benchmark import benchmark_one, generate_tensors, upload
    from autotune.runner.types import OutputSpec
    from autotune.tune import default_dists, input_specs
    from kernel_library import _lib
    from kernel_library.config import TileConfig

    M = N = K = 256
    specs = input_specs("matmul_lhsT_rhs", M, N, K)
    dev = upload(generate_tensors(specs, 0, default_dists("matmul_lhsT_rhs", K)), specs, gpu)
    exp, atol = golden.expected_output("matmul_lhsT_rhs", dev)
    cfg = TileConfig(128, 128, 64, 4, 2, variant=1)
    spec = OutputSpec("out", (M, N), "bfloat16")
    good = benchmark_one("good.hip", str(_lib.LIB_PATH), "matmul_lhsT_rhs", cfg, dev, spec, M, N, K, 1, 3,
                         golden=(exp, atol))
    assert good.hardware_output.startswith("[") and good.profiler_summary["numerics"]["pass"]
    bad = benchmark_one("bad.hip", str(_lib.LIB_PATH), "matmul_lhsT_rhs", cfg, dev, spec, M, N, K, 1, 3,
                        golden=(exp * 2, atol))
    assert bad.profiler_summary is None and bad.hardware_output.startswith("numerics check failed")
    torch.cuda.synchronize()
