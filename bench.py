"""Benchmark of the kernel_library hot path on one MI355X: prints ONE JSON line.

Workload (the configuration the metric is quoted on): the square bf16
``lhsT . rhs`` matmul at 8192^3, inputs U(-1,1) from seed 0 rounded to bf16,
fp32 accumulation, bf16 output, with the tile config chosen by the autotune
sweep (every legal prebuilt config, hipEvent-timed, fastest kept).  A step is
one launch of that kernel on inputs resident in HBM.

* ``value``: whole-job TFLOP/s = steps * 2*M*N*K / wall seconds of the timed
  region (bracketed by device synchronisation).
* ``roofline``: the same kernel's algorithmic FLOPs per launch over its
  average launch duration from HIP events recorded on the launch stream
  around the timed region, against MI355X's dense bf16 MFMA peak
  (2.5 PFLOP/s).  ``traffic`` is the HBM bytes per launch measured with
  rocprofv3 PMC counters (FETCH_SIZE + WRITE_SIZE, scaled by a copy-kernel
  calibration) when that measurement for the same config is recorded in
  ``profiles/traffic.json``; otherwise null.
* ``fused``: the rmsnorm_matmul kernel at 4096^3 (benchmark config C3) beside
  the plain matmul at the same shape, each with its autotuned config; the
  matmul both on its own U(-1,1) inputs and on the fused kernel's operands
  (normalised x, W).
* ``fused_reference_contract``: the same pair at the reference kernel's own
  shape and contract (2048^3, no gamma: rmsnorm_matmul_online).
* ``data_sensitivity``: the C2 kernel on all-zero and all-one inputs
  (diagnostic: the chip's clock under MFMA load depends on operand data).
* ``other_configs``: C4's three shapes (TFLOP/s), each autotuned by a sweep
  in this run (its winner, configs timed and numerics under ``sweep``), and
  C5's three plus the fused kernel at C5's shapes (HBM GB/s) with their
  tuned configs.
* ``cpu_baseline``: the CPU oracle's tile-faithful emulation of the
  reference kernel's loop nest (fp32, numpy/BLAS) on a bounded column slice
  of the same workload, rank 0 only.
* ``config.sweep_winner`` / ``config.pinned``: the sweep's fastest config
  and whether the shipped one is instead the tuned-table config because it
  was within 2 % of the winner in interleaved re-timing (so the line's
  config is the one the committed profiles cover whenever the two tie).
* ``clock``: the engine clock the shipped kernel runs at, measured right
  before the timed region (after its warm-up steps) and right after it by
  its clocked twin (the same
  kernel reading the engine-cycle and 100 MHz real-time counters around each
  workgroup: ``kernel_library._probe``), with the twin's launch time beside
  the product kernel's, and the share of the peak at that clock it reaches.
  ``clock.settle`` records how the timed region's start was reached: the
  kernel runs back to back until two successive twin readings agree within
  1 % (settle()), so the short timed region measures the kernel at its
  steady clock, not the clock's ramp after an idle gap.
* ``sustained``: the same kernel over at least one second of back-to-back
  launches after the timed region, with the twin's clock after it.
* ``mfma_ceiling``: the rate of the MFMA work alone on the benchmark's data
  (operands from registers; then with the kernel's LDS operand reads), with
  no global traffic: what any kernel running those instructions reaches
  under the chip's power limit.
* ``vendor``: hipBLASLt (``torch.matmul(lhs_T.t(), rhs)``) on the same
  inputs, and per shape in ``fused`` / ``other_configs``.

Flags: ``--gpus N`` (only 1 is supported: this build runs on one GPU),
``--steps``, ``--warmup``, ``--no-tune`` (use the tuned-config table /
library default), ``--only-kernel`` (skip the sweep, the fused pair and the
CPU baseline: the command profiled under rocprofv3 PMC runs),
``--calibrate-copy-mib N`` (run one device copy of N MiB first, the PMC
scale reference), ``--cpu-seconds`` (CPU baseline budget), ``--config NAME``
(time this tile config instead of sweeping), ``--workload c3`` (time the
fused rmsnorm_matmul at 4096^3 instead of the C2 matmul: the command the C3
kernel profiles are taken with; the default line is always C2),
``--workload c5 --m M`` / ``--workload decode --m M`` (the skinny matmul or
the fused kernel at (M, 28672, 8192), HBM-bound: the commands their profiles
are taken with), ``--workload c4a|c4b|c4c|c3-matmul`` (the plain lhsT.rhs
matmul at one C4 shape or at 4096^3, tuned config or ``--config``: the
commands their profiles are taken with), ``--workload c2-clock`` (the clock study: engine clock
against data movement at 8192^3, printed as a line of its own; see
clock_study()).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "nki-autotune_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

M = N = K = 8192
PEAK_BF16_TFLOPS = 2500.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description="kernel_library hot-path benchmark (one MI355X)")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-tune", action="store_true")
    ap.add_argument("--only-kernel", action="store_true")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--sweep-reps", type=int, default=20)
    ap.add_argument("--config", default="", help="tile config name (e.g. bm256_bn256_bk32_w4_s3_v1) instead of the sweep")
    ap.add_argument("--workload", choices=["c2", "c2-clock", "c3", "c3-matmul", "c4a", "c4b", "c4c", "c5", "decode",
                                           "panel-stream", "defaults", "defaults-random", "split-host", "online-pair"],
                    default="c2",
                    help="c2: lhsT.rhs matmul 8192^3 (the metric); c3: rmsnorm_matmul 4096^3; c3-matmul: the plain "
                         "lhsT.rhs matmul at 4096^3; c4a/b/c: the C4 "
                         "lhsT.rhs shapes; c5: skinny lhsT.rhs (--m) x 28672 x 8192; decode: rmsnorm_matmul at the "
                         "c5 shape; panel-stream: the K-panel loads alone from L2, MALL and HBM; defaults: the "
                         "library's default config against the autotune sweep's best at 83 shapes; "
                         "defaults-random: the same at 30 seeded random shapes the default was not fitted to; "
                         "split-host: back-to-back calls of workspace configs through the allocating entry point "
                         "and the no-alloc one; online-pair: the fused kernel without gamma beside the matmul at "
                         "2048^3, the reference kernel's shape and contract (all but c2: profiling workloads)")
    ap.add_argument("--settle-s", type=float, default=2.0,
                    help="GPU idle time before the timed region's warm-up (see settle())")
    ap.add_argument("--m", type=int, default=16, choices=[16, 64, 128], help="M of the c5 / decode workloads")
    ap.add_argument("--random-seed", type=int, default=2026, help="seed of the defaults-random shapes")
    return ap.parse_args()


def sweep(func_name: str, m: int, n: int, k: int, reps: int, no_tune: bool, with_gamma: bool = True):
    """Autotuned config of ``func_name`` at (m, n, k) (or the table/default one with ``no_tune``)."""
    import kernel_library as kl
    from autotune.tune import tune

    if no_tune:
        return kl.default_config(func_name, m, n, k), None
    res = tune(func_name, m, n, k, check=True, warmup=max(3, reps // 4), reps=reps, with_gamma=with_gamma)
    if res.best is None:
        raise RuntimeError(f"autotune sweep found no working config for {func_name} {m}x{n}x{k}:\n{res.output}")
    if res.check is not None and not res.check["pass"]:
        raise RuntimeError(f"autotuned {func_name} config {res.best.name} fails numerics: {res.check}")
    log(f"sweep {func_name} {m}x{n}x{k}: {len(res.output.successes)} configs, best {res.best.name} "
        f"{res.best_time_s * 1e6:.1f} us; numerics {res.check}")
    return res.best, res


def time_calls(launch, reps: int = 50) -> float:
    """Median per-launch seconds (HIP events around each launch) of ``launch``."""
    import torch

    from autotune.runner.benchmark import time_launches

    times = time_launches(launch, 5, reps)
    torch.cuda.synchronize()
    return sorted(times)[len(times) // 2]


def c_launchers(dev):
    """Launch closures that call the C ABI with arguments built once: the
    Python wrappers' ~10 us of host work per call would otherwise leave the
    GPU idle between 20 us kernels and be timed with them."""
    import ctypes

    import torch

    from kernel_library import _lib

    lib = _lib.lib()
    stream = torch.cuda.current_stream(dev).cuda_stream
    held = []

    def mm(lhs_t, rhs, out, cfg):
        c = cfg.to_c()
        held.append(c)
        k, m = lhs_t.shape
        args = (lhs_t.data_ptr(), rhs.data_ptr(), out.data_ptr(), m, rhs.shape[1], k, ctypes.byref(c), stream)
        _lib.check_rc(lib.mi_matmul_lhsT_rhs_bf16(*args), "matmul_lhsT_rhs")
        return lambda: lib.mi_matmul_lhsT_rhs_bf16(*args)

    def rms(x, w, g, out, cfg, eps=1e-6):
        c = cfg.to_c()
        held.append(c)
        m, k = x.shape
        args = (x.data_ptr(), g.data_ptr() if g is not None else None, w.data_ptr(), out.data_ptr(), m, w.shape[1], k,
                ctypes.c_float(eps), ctypes.byref(c), stream)
        _lib.check_rc(lib.mi_rmsnorm_matmul_bf16(*args), "rmsnorm_matmul")
        return lambda: lib.mi_rmsnorm_matmul_bf16(*args)

    return mm, rms


def fused_pair(reps: int, no_tune: bool, s: int = 4096, gamma: bool = True) -> dict:
    """rmsnorm_matmul vs plain matmul at s^3, each autotuned: C3 (4096^3 with
    gamma), or without gamma the reference kernel's own contract
    (rmsnorm_matmul_online, tuned under that name)."""
    import torch

    from autotune.runner.benchmark import generate_tensors, upload
    from autotune.tune import default_dists, input_specs

    dev = torch.device("cuda:0")
    fam_r = "rmsnorm_matmul" if gamma else "rmsnorm_matmul_online"
    cfg_r, _ = sweep(fam_r, s, s, s, reps, no_tune, with_gamma=gamma)
    cfg_m, _ = sweep("matmul_lhsT_rhs", s, s, s, reps, no_tune)
    spec_r = input_specs("rmsnorm_matmul", s, s, s, with_gamma=gamma)
    r = upload(generate_tensors(spec_r, 0, default_dists("rmsnorm_matmul", s)), spec_r, dev)
    g = r.get("gamma")
    spec_m = input_specs("matmul_lhsT_rhs", s, s, s)
    mm = upload(generate_tensors(spec_m, 0, default_dists("matmul_lhsT_rhs", s)), spec_m, dev)
    out_r = torch.empty((s, s), dtype=torch.bfloat16, device=dev)
    out_m = torch.empty((s, s), dtype=torch.bfloat16, device=dev)
    c_mm, c_rms = c_launchers(dev)
    fused = c_rms(r["lhs"], r["rhs"], g, out_r, cfg_r)
    plain = c_mm(mm["lhs_T"], mm["rhs"], out_m, cfg_m)
    # Interleaved rounds: both kernels see the same clock and power states.
    tr, tm = [], []
    for _ in range(5):
        tr.append(time_calls(fused, 40))
        tm.append(time_calls(plain, 40))
    # The same matmul on the fused kernel's own operands: lhsT = the
    # normalised, gamma-scaled x (bf16), rhs = W.  MI355X's clock under MFMA
    # load depends on the operand data, so this is the like-for-like pair.
    xf = r["lhs"].float()
    xhat = xf * torch.rsqrt(xf.pow(2).mean(1, keepdim=True) + 1e-6)
    xhat = (xhat * g.float() if gamma else xhat).bfloat16()
    same = {"lhs_T": xhat.t().contiguous(), "rhs": r["rhs"]}
    del xf, xhat
    same_launch = c_mm(same["lhs_T"], same["rhs"], out_m, cfg_m)
    ts = []
    for _ in range(5):
        ts.append(time_calls(same_launch, 40))
    t_r, t_m, t_s = sorted(tr)[2], sorted(tm)[2], sorted(ts)[2]
    fl = 2.0 * s ** 3
    x, w = r["lhs"], r["rhs"]

    def unfused():
        xf = x.float()
        xn = xf * torch.rsqrt(xf.pow(2).mean(1, keepdim=True) + 1e-6)
        torch.matmul((xn * g.float() if gamma else xn).to(torch.bfloat16), w, out=out_r)

    t_v = vendor_time(unfused)
    return {
        "shape": [s, s, s],
        "gamma": gamma,
        "rmsnorm_matmul_tflops": round(fl / t_r / 1e12, 1),
        "rmsnorm_matmul_config": cfg_r.name,
        "matmul_tflops": round(fl / t_m / 1e12, 1),
        "matmul_config": cfg_m.name,
        "fused_over_matmul_time": round(t_r / t_m, 4),
        "matmul_same_operands_tflops": round(fl / t_s / 1e12, 1),
        "fused_over_same_operand_matmul_time": round(t_r / t_s, 4),
        "vendor_unfused": {"library": "torch eager rmsnorm, then torch.matmul (hipBLASLt)",
                           "tflops": round(fl / t_v / 1e12, 1), "fused_speedup": round(t_v / t_r, 3)},
    }


def data_sensitivity(cfg, steps: int = 20) -> dict:
    """The C2 kernel and config on constant inputs (zeros, ones) instead of U(-1,1).

    Same launches, same work; only the operand values differ.  MI355X lowers
    its clock under MFMA load as the power the operand data draws rises, so
    the constant-input rate shows what the kernel's issue rate reaches when
    power does not limit it.  Diagnostic only: the metric is the U(-1,1)
    figure."""
    import torch

    import kernel_library as kl
    from autotune.runner.benchmark import time_launches

    dev = torch.device("cuda:0")
    out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    res = {}
    for name, fill in (("zeros", 0.0), ("ones", 1.0)):
        a = torch.full((K, M), fill, dtype=torch.bfloat16, device=dev)
        b = torch.full((K, N), fill, dtype=torch.bfloat16, device=dev)
        times = time_launches(lambda: kl.matmul_lhsT_rhs(a, b, cfg=cfg, out=out), 3, steps)
        t = sorted(times)[len(times) // 2]
        res[f"{name}_inputs_tflops"] = round(2.0 * M * N * K / t / 1e12, 1)
        del a, b
    torch.cuda.synchronize()
    return res


SKINNY_N, SKINNY_K = 28672, 8192
# Benchmark config C4: (M, K, N) of the non-square sweeps.
C4_SHAPES = {"c4a": (2048, 8192, 1024), "c4b": (4096, 1024, 14336), "c4c": (1024, 14336, 4096)}
# Plain lhsT.rhs shapes timed by shape_main: C4's three, and the C3 shape (the
# fused kernel's like-for-like matmul).
PLAIN_SHAPES = {**C4_SHAPES, "c3-matmul": (4096, 4096, 4096)}
HBM_PEAK_GBS = 8000.0


def skinny_bytes(fam: str, m: int) -> int:
    """Compulsory HBM bytes of one launch at (m, 28672, 8192): both operands read once, out written once."""
    b = (m * SKINNY_K + SKINNY_K * SKINNY_N + m * SKINNY_N) * 2
    return b + (2 * SKINNY_K if fam == "rmsnorm_matmul" else 0)


def skinny_inputs(fam: str, m: int, dev):
    """C5 inputs (N(0, 0.02)) for the matmul; the C3 distributions for the fused kernel."""
    from autotune.runner.benchmark import generate_tensors, upload
    from autotune.tune import default_dists, input_specs

    specs = input_specs(fam, m, SKINNY_N, SKINNY_K)
    dists = ({"lhs_T": ("normal", 0.02), "rhs": ("normal", 0.02)} if fam == "matmul_lhsT_rhs"
             else default_dists(fam, SKINNY_K))
    return upload(generate_tensors(specs, 0, dists), specs, dev)


SETTLE_TOL = 0.01      # two successive clock readings this close: the clock has settled
SETTLE_CAP_S = 6.0     # give up waiting for a steady clock after this much load
SETTLE_STEP_S = 0.25   # back-to-back launches between two readings


def settle(launch, idle_s: float, reading=None) -> dict:
    """Bring the GPU to the steady clock of ``launch`` before a timed region; returns what it took.

    A long run of back-to-back GEMMs (the sweep before the timed region: ~10 s)
    drives the engine clock down under the power limit (the shipped config
    timed 11 % slower right after the sweep than inside it), and a GPU that
    has been idle starts below its working clock and takes more than half a
    second of load to reach it.  So: idle ``idle_s`` seconds, then run the
    timed kernel back to back in steps of ``SETTLE_STEP_S`` seconds,
    reading the engine clock after each step with ``reading`` (the kernel's
    clocked twin, 10 launches), until two successive readings agree within
    ``SETTLE_TOL`` -- or ``SETTLE_CAP_S`` seconds of load have passed.
    Without a ``reading`` (no clocked twin for the kernel) it is half a
    second of load."""
    if idle_s > 0:
        time.sleep(idle_s)
    t0 = time.perf_counter()
    warm(launch, SETTLE_STEP_S)
    readings: list[float] = []
    steady = False
    if reading is None:
        warm(launch, 0.5 - SETTLE_STEP_S)
    else:
        while True:
            r = reading()
            if not r or "error" in r:
                break
            readings.append(r["clock_mhz"])
            if len(readings) >= 2 and abs(readings[-1] - readings[-2]) <= SETTLE_TOL * readings[-1]:
                steady = True
                break
            if time.perf_counter() - t0 >= SETTLE_CAP_S:
                break
            warm(launch, SETTLE_STEP_S)
    return {"idle_s": idle_s, "load_s": round(time.perf_counter() - t0, 2), "readings_mhz": readings,
            "steady": steady if reading is not None else None,
            "rule": f"idle, then the timed kernel back to back; its clocked twin read every {SETTLE_STEP_S} s of "
                    f"load until two successive readings agree within {100 * SETTLE_TOL:.0f} % "
                    f"(at most {SETTLE_CAP_S} s)"}


def sustained(launch, flop: float, reading=None, seconds: float = 1.0) -> dict:
    """Throughput of at least ``seconds`` of back-to-back launches (HIP events around the whole run), then the
    clock read by ``reading`` right after: the kernel under sustained load, beside the short timed region."""
    import torch

    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    n = 0
    t0 = time.perf_counter()
    ev0.record(stream)
    while time.perf_counter() - t0 < seconds:
        for _ in range(20):
            launch()
        n += 20
        torch.cuda.synchronize()
    ev1.record(stream)
    torch.cuda.synchronize()
    s = ev0.elapsed_time(ev1) * 1e-3
    out = {"launches": n, "seconds": round(s, 3), "us_per_launch": round(s / n * 1e6, 1),
           "tflops": round(flop * n / s / 1e12, 1), "pct_mfma_peak": round(100 * flop * n / s / 1e12 / PEAK_BF16_TFLOPS, 2)}
    if reading is not None:
        r = reading()
        if r and "error" not in r:
            out["clock_after_mhz"] = r["clock_mhz"]
    return out


def warm(launch, seconds: float = 0.5) -> None:
    """Launch back to back for ``seconds``: the engine clock rises over the
    first few hundred milliseconds of sustained load, and a short burst of
    launches after an idle gap is timed at the lower clock (10-15 % slower
    for the C4 shapes)."""
    import torch

    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(10):
            launch()
        torch.cuda.synchronize()


def other_configs(reps: int = 30, sweep_reps: int = 20, no_tune: bool = False) -> dict:
    """C4 (TFLOP/s) and C5 plus the fused kernel at C5's shapes (HBM GB/s).

    C4 is the autotune sweep BASELINE's config 4 asks for: each shape is
    swept in this run (every legal prebuilt config with its numerics gate,
    then the finalists re-timed in interleaved rounds; ``no_tune`` takes the
    tuned-table config instead), and the winner is timed through the C ABI
    with arguments built once.  C5 and the fused decode shapes take their
    tuned configs.  Each shape is timed after half a second of back-to-back
    launches of the same kernel.  C5 and the fused decode shapes are timed
    with a 512 MiB buffer overwritten before every launch, so W streams from
    HBM, not from the 256 MB MALL."""
    import torch

    import kernel_library as kl
    from autotune.runner.benchmark import generate_tensors, time_launches, upload
    from autotune.tune import default_dists, input_specs

    dev = torch.device("cuda:0")
    c_mm, _ = c_launchers(dev)
    res = {}
    for m, k, n in ((2048, 8192, 1024), (4096, 1024, 14336), (1024, 14336, 4096)):
        cfg, tuned = sweep("matmul_lhsT_rhs", m, n, k, sweep_reps, no_tune)
        specs = input_specs("matmul_lhsT_rhs", m, n, k)
        d = upload(generate_tensors(specs, 0, default_dists("matmul_lhsT_rhs", k)), specs, dev)
        out = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        launch = c_mm(d["lhs_T"], d["rhs"], out, cfg)
        warm(launch)
        t = sorted(time_launches(launch, 5, reps))
        tf = 2.0 * m * n * k / t[len(t) // 2] / 1e12
        a_t = d["lhs_T"].t()
        tv = vendor_time(lambda: torch.matmul(a_t, d["rhs"], out=out))  # noqa: B023
        row = {"config": cfg.name, "tflops": round(tf, 1), "pct_mfma_peak": round(100 * tf / PEAK_BF16_TFLOPS, 1),
               "hipblaslt_tflops": round(2.0 * m * n * k / tv / 1e12, 1)}
        if tuned is not None:
            row["sweep"] = {"configs_timed": len(tuned.output.successes), "failures": len(tuned.output.failures),
                            "winner_sweep_us": round(tuned.best_time_s * 1e6, 2),
                            "numerics_pass": bool(tuned.check and tuned.check["pass"]),
                            "tuned_table_config": kl.default_config("matmul_lhsT_rhs", m, n, k).name}
        res[f"C4 (M,K,N)=({m},{k},{n})"] = row
        del d, out
    scratch = torch.empty((512 << 20) // 4, dtype=torch.float32, device=dev)
    for fam, label in (("matmul_lhsT_rhs", "C5"), ("rmsnorm_matmul", "fused decode")):
        for m in (16, 64, 128):
            d = skinny_inputs(fam, m, dev)
            cfg = kl.default_config(fam, m, SKINNY_N, SKINNY_K)
            out = torch.empty((m, SKINNY_N), dtype=torch.bfloat16, device=dev)
            if fam == "matmul_lhsT_rhs":
                launch = lambda: kl.matmul_lhsT_rhs(d["lhs_T"], d["rhs"], cfg=cfg, out=out)  # noqa: E731
            else:
                launch = lambda: kl.rmsnorm_matmul(d["lhs"], d["rhs"], d["gamma"], cfg=cfg, out=out)  # noqa: E731
            warm(launch)
            t = sorted(time_launches(launch, 5, reps, flush=scratch.zero_))
            gbs = skinny_bytes(fam, m) / t[len(t) // 2] / 1e9
            if fam == "matmul_lhsT_rhs":
                a_t = d["lhs_T"].t()
                vendor = lambda: torch.matmul(a_t, d["rhs"], out=out)  # noqa: E731,B023
            else:
                def vendor(x=d["lhs"], g=d["gamma"], w=d["rhs"], out=out):
                    xf = x.float()
                    y = (xf * torch.rsqrt(xf.pow(2).mean(1, keepdim=True) + 1e-6) * g.float()).to(torch.bfloat16)
                    torch.matmul(y, w, out=out)
            warm(vendor, 0.3)
            tv = sorted(time_launches(vendor, 5, reps, flush=scratch.zero_))
            res[f"{label} M={m}"] = {"config": cfg.name, "us": round(t[len(t) // 2] * 1e6, 1),
                                     "hbm_gbs": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
                                     "vendor_hbm_gbs": round(skinny_bytes(fam, m) / tv[len(tv) // 2] / 1e9, 1)}
            del d, out
    del scratch
    torch.cuda.synchronize()
    return res


PIN_WITHIN = 1.02


def pin_to_table(fam: str, s: int, best, reps: int):
    """Ship the tuned-table config instead of the sweep's winner when the two
    are within 2 % in interleaved re-timing (box-to-box noise is larger), so
    the line's config is the one the committed profiles cover."""
    import kernel_library as kl
    from autotune.tune import refine
    from kernel_library.config import table_key, tuned_table

    table = tuned_table().get(table_key(fam, s, s, s))
    if table is None:
        return best, {"sweep_winner": best.name, "pinned": False}
    table_cfg = kl.TileConfig(**table)
    if table_cfg == best:
        return best, {"sweep_winner": best.name, "pinned": False}
    times = refine(fam, s, s, s, [best, table_cfg], reps=max(10, reps // 2), rounds=5)
    ratio = times[table_cfg.name] / times[best.name]
    log(f"sweep winner {best.name} {times[best.name] * 1e6:.1f} us vs table {table_cfg.name} "
        f"{times[table_cfg.name] * 1e6:.1f} us (ratio {ratio:.4f})")
    if ratio <= PIN_WITHIN:
        return table_cfg, {"sweep_winner": best.name, "pinned": True, "table_over_winner_time": round(ratio, 4)}
    return best, {"sweep_winner": best.name, "pinned": False, "table_over_winner_time": round(ratio, 4)}


def twin_clock(d: dict, out, cfg, launches: int = 10):
    """Clock and launch time of the shipped kernel's clocked twin (None: no twin; dict with "error")."""
    from kernel_library import _probe

    try:
        return _probe.clocked_lhsT_rhs(d["lhs_T"], d["rhs"], out, cfg, launches=launches, warmup=1)
    except ImportError as exc:
        return {"error": str(exc)}


def clock_of(before, after, cfg, achieved_tflops: float) -> dict:
    """The engine clock around the timed region: the clocked twin of the
    shipped kernel (10 launches) right before the timed steps and right after."""
    from kernel_library import _probe

    if before is None or after is None:
        return {"error": f"no clocked twin of {cfg.name}"}
    if "error" in before or "error" in after:
        return {"error": before.get("error") or after.get("error")}
    mhz = (before["clock_mhz"] + after["clock_mhz"]) / 2
    at_clock = PEAK_BF16_TFLOPS * mhz / _probe.PEAK_CLOCK_MHZ
    return {"clock_mhz": round(mhz, 1), "before": before, "after": after,
            "source": "clocked twin of the shipped kernel (s_memtime / s_memrealtime per workgroup), 10 launches "
                      "after the warm-up steps, right before the timed steps, and 10 right after them",
            "peak_at_that_clock_tflops": round(at_clock, 1),
            "frac_of_peak_at_that_clock": round(achieved_tflops / at_clock, 4)}


def mfma_ceiling(src) -> dict:
    """The MFMA probe on the benchmark's own U(-1,1) operands: registers only, then with LDS operand reads."""
    from autotune.runner.driver import warm_clock
    from kernel_library import _probe

    warm_clock(src.device, 0.3)
    return {"regs_only": _probe.mfma_ceiling(src, 0), "with_lds_operand_reads": _probe.mfma_ceiling(src, 1),
            "data": "U(-1,1) bf16 operands (the C2 lhsT), 1024 waves x 32768 MFMA 32x32x16 each"}


def vendor_time(launch, reps: int = 20) -> float:
    from autotune.runner.benchmark import time_launches

    warm(launch, 0.3)
    t = sorted(time_launches(launch, 3, reps))
    return t[len(t) // 2]


def vendor_matmul(lhs_T, rhs, kernel_s: float) -> dict:
    """hipBLASLt (torch.matmul of the transposed lhs_T view) on the C2 inputs, beside the kernel's launch time."""
    import torch

    out = torch.empty((lhs_T.shape[1], rhs.shape[1]), dtype=lhs_T.dtype, device=lhs_T.device)
    a = lhs_T.t()
    t = vendor_time(lambda: torch.matmul(a, rhs, out=out))
    k, m = lhs_T.shape
    flop = 2.0 * m * rhs.shape[1] * k
    del out
    return {"library": "torch.matmul (hipBLASLt)", "us": round(t * 1e6, 1), "tflops": round(flop / t / 1e12, 1),
            "kernel_speedup": round(t / kernel_s, 3)}


def cpu_baseline(budget_s: float) -> dict:
    """The oracle's tile-faithful emulation of the reference loop nest, timed on a bounded column slice."""
    import numpy as np
    from threadpoolctl import threadpool_info

    from oracle import matmul as omm

    rng = np.random.default_rng(0)
    lhs_T = rng.uniform(-1.0, 1.0, (K, M)).astype(np.float32)
    # Double the slice until one emulation run takes >= budget/4 (total CPU time ~ budget/2).
    cols = 64
    while True:
        rhs = rng.uniform(-1.0, 1.0, (K, cols)).astype(np.float32)
        t0 = time.perf_counter()
        omm.tiled(lhs_T, rhs, out_dtype="float32")
        dt = time.perf_counter() - t0
        flops = 2.0 * M * cols * K
        if dt >= budget_s / 4 or cols >= N:
            break
        cols = min(N, cols * 2)
    threads = max([i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"] or [1])
    return {
        "value": round(flops / dt / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": int(threads),
        "kind": "port",
        "sample": f"oracle.matmul.tiled (fp32 tile-faithful emulation of kernel_hand_90.92mfu.py:101-131) on "
                  f"lhsT[{K},{M}] x rhs[{K},{cols}] (a {cols}-column slice of the 8192^3 workload), "
                  f"{dt:.2f} s, BLAS threads {threads}, host cpus {len(os.sched_getaffinity(0))}",
    }


def recorded_traffic(fam: str, shape, cfg_name: str):
    """HBM bytes per launch recorded for (family, shape, config), or None; ``shape`` is s (s^3) or "MxNxK"."""
    try:
        with open(TRAFFIC_FILE) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    key = shape if isinstance(shape, str) else f"{shape}x{shape}x{shape}"
    entry = rec.get(f"{fam}:{key}:{cfg_name}")
    return None if entry is None else entry.get("hbm_bytes_per_launch")


def main() -> int:
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py runs on exactly one GPU: this build has no multi-GPU path (use --gpus 1)", file=sys.stderr)
        return 2
    import torch

    import kernel_library as kl
    from autotune.runner.benchmark import generate_tensors, upload
    from autotune.tune import default_dists, input_specs

    if not torch.cuda.is_available():
        print("bench.py needs an MI355X (no HIP device visible)", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    if args.calibrate_copy_mib:
        nb = args.calibrate_copy_mib << 20
        src = torch.ones(nb // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration copy of {args.calibrate_copy_mib} MiB done")
        del src, dst

    if args.workload in ("c5", "decode"):
        return skinny_main(args, dev)
    if args.workload == "c2-clock":
        return clock_study(args, dev)
    if args.workload == "panel-stream":
        return panel_stream_study(args, dev)
    if args.workload == "defaults":
        return defaults_study(args, dev, [(f, sh) for f, shapes in (
            ("matmul_lhsT_rhs", DEFAULTS_MM + DEFAULTS_SKINNY), ("matmul_lhs_rhs", DEFAULTS_LHS),
            ("rmsnorm_matmul", DEFAULTS_RMS)) for sh in shapes], "defaults")
    if args.workload == "defaults-random":
        return defaults_study(args, dev, random_default_shapes(args.random_seed), f"defaults-random:{args.random_seed}")
    if args.workload == "split-host":
        return split_host_study(args, dev)
    if args.workload == "online-pair":
        print(json.dumps({"workload": "online-pair", **fused_pair(args.sweep_reps, args.no_tune, s=2048, gamma=False)}),
              flush=True)
        return 0
    if args.workload in PLAIN_SHAPES:
        return shape_main(args, dev, *PLAIN_SHAPES[args.workload])
    fam, s = ("matmul_lhsT_rhs", M) if args.workload == "c2" else ("rmsnorm_matmul", 4096)
    pin = {}
    if args.config:
        cfg = kl.TileConfig.from_name(args.config)
    else:
        cfg, res = sweep(fam, s, s, s, args.sweep_reps, args.no_tune or args.only_kernel)
        if res is not None:
            cfg, pin = pin_to_table(fam, s, cfg, args.sweep_reps)
    specs = input_specs(fam, s, s, s)
    d = upload(generate_tensors(specs, 0, default_dists(fam, s)), specs, dev)
    out = torch.empty((s, s), dtype=torch.bfloat16, device=dev)

    if fam == "matmul_lhsT_rhs":
        def step():
            kl.matmul_lhsT_rhs(d["lhs_T"], d["rhs"], cfg=cfg, out=out)
    else:
        def step():
            kl.rmsnorm_matmul(d["lhs"], d["rhs"], d["gamma"], cfg=cfg, out=out)

    clock_twin = fam == "matmul_lhsT_rhs" and not args.only_kernel
    reading = (lambda: twin_clock(d, out, cfg)) if clock_twin else None
    settled = settle(step, args.settle_s, reading)
    log(f"settle: {settled}")
    for _ in range(args.warmup):
        step()
    before = twin_clock(d, out, cfg) if clock_twin else None
    stream = torch.cuda.current_stream(dev)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    after = twin_clock(d, out, cfg) if clock_twin else None
    kern_s = ev0.elapsed_time(ev1) * 1e-3 / args.steps
    flop = 2.0 * s * s * s
    value = flop * args.steps / wall / 1e12
    achieved = flop / kern_s / 1e12
    log(f"timed {args.steps} steps: wall {wall * 1e3:.1f} ms, {value:.1f} TFLOP/s; kernel avg {kern_s * 1e6:.1f} us")

    line = {
        "metric": "bf16 TFLOP/s + % MFMA peak, lhsT·rhs matmul 8192³ and rmsnorm_matmul, 1 GPU",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: lhsT, rhs ~ U(-1,1) seed 0 rounded to bf16, resident in HBM" if fam == "matmul_lhsT_rhs"
        else "synthetic: x ~ N(0,1), gamma = 1 + 0.1 N(0,1), W ~ N(0, 1/64), seed 0, bf16, resident in HBM",
        "config": {
            "workload": "lhsT[8192,8192]·rhs[8192,8192] bf16 matmul, fp32 accumulate, bf16 out (benchmark config C2)"
            if fam == "matmul_lhsT_rhs" else
            "rmsnorm(x[4096,4096])*gamma[4096] . W[4096,4096] bf16, fp32 accumulate (benchmark config C3)",
            "kernel": "mm_lhsT_rhs_bf16" if fam == "matmul_lhsT_rhs" else "rmsnorm_matmul_bf16",
            "tile_config": cfg.name,
            "autotuned": not (args.no_tune or args.only_kernel or args.config),
            **pin,
            "pct_mfma_peak": round(100.0 * value / PEAK_BF16_TFLOPS, 2),
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": recorded_traffic(fam, s, cfg.name),
        },
    }
    if not args.only_kernel and fam == "matmul_lhsT_rhs":
        line["clock"] = clock_of(before, after, cfg, achieved)
        line["clock"]["settle"] = settled
        log(f"clock: {line['clock']}")
        line["sustained"] = sustained(step, flop, reading)
        log(f"sustained: {line['sustained']}")
        line["mfma_ceiling"] = mfma_ceiling(d["lhs_T"])
        log(f"MFMA ceiling: {line['mfma_ceiling']}")
        line["vendor"] = vendor_matmul(d["lhs_T"], d["rhs"], kern_s)
        log(f"vendor: {line['vendor']}")
        line["data_sensitivity"] = data_sensitivity(cfg)
        log(f"data sensitivity: {line['data_sensitivity']}")
        line["fused"] = fused_pair(args.sweep_reps, args.no_tune)
        log(f"fused pair: {line['fused']}")
        line["fused_reference_contract"] = fused_pair(args.sweep_reps, args.no_tune, s=2048, gamma=False)
        log(f"fused pair, 2048^3 without gamma: {line['fused_reference_contract']}")
        line["other_configs"] = other_configs(sweep_reps=args.sweep_reps, no_tune=args.no_tune)
        log(f"other configs: {line['other_configs']}")
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(line, ensure_ascii=False), flush=True)
    return 0


# Configs of the clock study: tiles from 256x256 down to 64x128, so LDS
# bytes read per MFMA and fabric bytes per launch both span about 3x.
CLOCK_STUDY_CONFIGS = ("bm256_bn256_bk32_w4_s3_v1", "bm256_bn256_bk32_w8_s3_v1", "bm128_bn512_bk32_w8_s3_v1",
                       "bm128_bn256_bk32_w4_s3_v1", "bm128_bn128_bk64_w4_s3_v1", "bm64_bn128_bk64_w4_s4_v1")


def lds_bytes_per_mfma(cfg) -> int:
    """LDS bytes a wave reads per 32x32x16 MFMA: its (tm + tn) x 16 bf16 operand slice per tm/32 x tn/32 MFMAs.

    The wave tile (tm, tn) follows the kernels' wave split: the most square
    power-of-two split of the workgroup tile into ``waves`` tiles of at
    least 32x32."""
    best = None
    wm = 1
    while wm <= cfg.waves:
        wn = cfg.waves // wm
        tm, tn = cfg.block_m // wm, cfg.block_n // wn
        if wm * wn == cfg.waves and tm >= 32 and tn >= 32 and tm % 32 == 0 and tn % 32 == 0:
            if best is None or abs(tm - tn) < abs(best[0] - best[1]):
                best = (tm, tn)
        wm *= 2
    tm, tn = best
    return (tm + tn) * 16 * 2 // ((tm // 32) * (tn // 32))


def clock_study(args, dev) -> int:
    """--workload c2-clock: does the engine clock rise as data movement falls?

    The C2 workload (8192^3, U(-1,1) bf16) on the clocked twins of lhsT.rhs
    configs whose tiles span 256x256 to 64x128, beside the two MFMA probes
    that run the same MFMA count with no global traffic (operands from LDS,
    then from registers).  Rounds interleave every row, so each row sees the
    same power and thermal history; a row reports its median clock and
    launch time over the rounds.  The fabric bytes of each row come from a
    rocprofv3 FETCH_SIZE / WRITE_SIZE pass of this same command."""
    import statistics

    import torch

    import kernel_library as kl
    from autotune.runner.benchmark import generate_tensors, upload
    from autotune.tune import default_dists, input_specs
    from kernel_library import _probe

    fam, s = "matmul_lhsT_rhs", M
    specs = input_specs(fam, s, s, s)
    d = upload(generate_tensors(specs, 0, default_dists(fam, s)), specs, dev)
    out = torch.empty((s, s), dtype=torch.bfloat16, device=dev)
    flop = 2.0 * s * s * s
    cfgs = [kl.TileConfig.from_name(n) for n in CLOCK_STUDY_CONFIGS]
    rounds = max(1, args.steps // 10)
    rows = {c.name: [] for c in cfgs}
    probes = {"mfma_lds_probe": [], "mfma_regs_probe": []}
    settle(lambda: kl.matmul_lhsT_rhs(d["lhs_T"], d["rhs"], cfg=cfgs[0], out=out), args.settle_s)
    for r in range(rounds):
        for c in cfgs:
            rows[c.name].append(_probe.clocked_lhsT_rhs(d["lhs_T"], d["rhs"], out, c, launches=10, warmup=2))
        probes["mfma_lds_probe"].append(_probe.mfma_ceiling(d["lhs_T"], 1))
        probes["mfma_regs_probe"].append(_probe.mfma_ceiling(d["lhs_T"], 0))
        log(f"clock study round {r + 1}/{rounds} done")
    table = []
    for c in cfgs:
        us = statistics.median(x["us"] for x in rows[c.name])
        mhz = statistics.median(x["clock_mhz"] for x in rows[c.name])
        tf = flop / (us * 1e-6) / 1e12
        table.append({"config": c.name, "lds_bytes_per_mfma": lds_bytes_per_mfma(c), "us": round(us, 1),
                      "tflops": round(tf, 1), "clock_mhz": round(mhz, 1),
                      "frac_of_peak": round(tf / PEAK_BF16_TFLOPS, 4),
                      "frac_of_peak_at_that_clock": round(tf / (PEAK_BF16_TFLOPS * mhz / _probe.PEAK_CLOCK_MHZ), 4)})
    for name, lst in probes.items():
        tf = statistics.median(x["tflops"] for x in lst)
        mhz = statistics.median(x["clock_mhz"] for x in lst)
        table.append({"config": name, "lds_bytes_per_mfma": 512 if name == "mfma_lds_probe" else 0,
                      "tflops": tf, "clock_mhz": mhz, "frac_of_peak": round(tf / PEAK_BF16_TFLOPS, 4),
                      "frac_of_peak_at_that_clock": round(tf / (PEAK_BF16_TFLOPS * mhz / _probe.PEAK_CLOCK_MHZ), 4)})
    for row in table:
        log(json.dumps(row))
    print(json.dumps({"workload": "c2-clock", "shape": [s, s, s], "rounds": rounds,
                      "data": "lhsT, rhs ~ U(-1,1) seed 0 rounded to bf16", "rows": table}), flush=True)
    return 0


def panel_stream_study(args, dev) -> int:
    """--workload panel-stream: how fast can a CU's LDS-direct K-panel loads run with nothing else to do?

    The kernels' panel loads (1 KiB per wave instruction, straight into LDS)
    with no LDS reads and no MFMA, one workgroup per CU, at 4 or 8 waves and
    4..16 loads in flight per wave.  Each launch moves 1 GiB.  Rows:

    * consecutive 1 KiB chunks of a 2 MiB region (held in every XCD's L2
      after the first pass), a 64 MiB one (from the MALL) and a 1 GiB one
      (from HBM);
    * the panel shapes of the benchmark kernels from a 2 MiB region: K rows
      of 64, 128 or 256 bf16 columns (128, 256, 512 bytes) out of matrix
      rows 2048 to 16384 bytes long (the lhsT / rhs pitches of C2, C4a, C4c);
    * the skinny weight panel (128 columns of a 28672-column rhs) over a
      896 MiB region (HBM).

    The L2 rows bound every kernel whose panels are L2 hits: its panel
    bytes per CU over the L2 rows' bytes per clock per CU is the fewest
    clocks it can take."""
    import torch

    from kernel_library import _probe

    buf = torch.ones(1 << 28, dtype=torch.float32, device=dev)  # 1 GiB
    cases = [("L2 contiguous", 2 << 20, 1024, 1024), ("MALL contiguous", 64 << 20, 1024, 1024),
             ("HBM contiguous", 1 << 30, 1024, 1024),
             ("L2 C4a lhsT panel (64 of 2048 cols)", 2 << 20, 128, 4096),
             ("L2 C4a rhs panel (128 of 1024 cols)", 2 << 20, 256, 2048),
             ("L2 C4c panel (128 of 4096 cols)", 2 << 20, 256, 8192),
             ("L2 C2 panel (256 of 8192 cols)", 2 << 20, 512, 16384),
             ("L2 64-col panel of 8192 cols", 2 << 20, 128, 16384),
             ("HBM skinny rhs panel (128 of 28672 cols)", 57344 * 4 * 4096, 256, 57344)]
    rows = []
    for label, region, rb, pitch in cases:
        for w, inf in ((4, 8), (4, 16), (8, 8)):
            rounds = max(1, (1 << 30) // (256 * w * inf * 1024))
            r = dict(case=label, **_probe.panel_stream(buf, region, w, inf, rounds, row_bytes=rb, pitch=pitch))
            log(json.dumps(r))
            rows.append(r)
    print(json.dumps({"workload": "panel-stream", "wgs": 256, "bytes_per_launch": 1 << 30, "rows": rows}),
          flush=True)
    return 0


# (M, N, K) shapes of the default-config study, beside the benchmark's own.
DEFAULTS_MM = [(1024, 1024, 1024), (2048, 2048, 2048), (3072, 3072, 3072), (4096, 4096, 4096), (6144, 6144, 6144),
               (4096, 11008, 4096), (4096, 4096, 11008), (2048, 1024, 4096), (1024, 2048, 8192),
               (8192, 1024, 8192), (512, 4096, 4096), (256, 14336, 4096), (1000, 2000, 3000), (8192, 8192, 1024),
               (1024, 8192, 16384), (96, 8192, 8192), (4096, 14336, 1024), (2048, 1024, 8192),
               (1536, 1536, 6144), (2048, 4096, 1024), (768, 3072, 3072), (4096, 1024, 2048), (12288, 4096, 4096),
               (136, 4096, 4096), (6144, 2048, 2048), (2560, 2560, 10240), (512, 512, 32768), (16, 4096, 8192),
               (64, 14336, 4096), (2048, 2048, 8192), (1280, 5120, 5120), (4608, 4608, 2304), (640, 10240, 2048),
               (32, 2048, 16384), (3584, 1024, 4096), (1024, 3584, 14336), (200, 4096, 4096), (8192, 2048, 4096),
               (6144, 768, 6144)]
DEFAULTS_SKINNY = [(128, 16384, 8192), (64, 12288, 16384), (32, 8192, 16384), (16, 28672, 8192), (128, 28672, 8192),
                   (16, 8192, 8192), (32, 14336, 4096), (64, 4096, 4096), (128, 4096, 14336), (128, 8192, 4096),
                   (64, 28672, 8192), (8, 11008, 4096)]
DEFAULTS_LHS = [(1024, 1024, 1024), (2048, 2048, 2048), (3072, 3072, 3072), (4096, 4096, 4096), (8192, 1024, 8192),
                (2048, 1024, 4096), (512, 4096, 4096), (1024, 8192, 16384), (96, 8192, 8192), (4096, 14336, 1024),
                (16, 28672, 8192), (1536, 1536, 6144), (512, 512, 32768), (8192, 8192, 8192)]
DEFAULTS_RMS = [(4096, 4096, 4096), (2048, 8192, 2048), (8192, 4096, 4096), (1024, 14336, 4096), (512, 4096, 8192),
                (2048, 2048, 2048), (1024, 4096, 4096), (3072, 3072, 3072), (256, 8192, 4096), (1024, 1024, 4096),
                (1536, 6144, 2048), (640, 8192, 4096), (4096, 2048, 4096), (128, 4096, 4096), (768, 6144, 4096),
                (2560, 4096, 2048), (384, 8192, 8192), (1024, 8192, 1024)]


SPLIT_HOST_CASES = [((2048, 2048, 1024), "bm128_bn128_bk64_w4_s3_v1_k2"), ((2048, 2048, 1024), "bm64_bn64_bk64_w4_s4_v1_k2"),
                    ((2048, 2048, 1024), "bm128_bn128_bk64_w4_s3_v1"), ((2048, 2048, 1024), "bm64_bn128_bk64_w4_s4_v5"),
                    ((2048, 1024, 8192), "bm128_bn128_bk64_w4_s3_v1_k2"),
                    ((2048, 1024, 8192), "bm256_bn128_bk64_w8_s3_v1_k4"),
                    ((2048, 1024, 8192), "bm64_bn128_bk64_w4_s4_v1")]


def split_host_study(args, dev) -> int:
    """--workload split-host: what does a workspace config cost per call beyond its kernels?

    Each (M, N, K), config of ``SPLIT_HOST_CASES`` (split-K, stream-K, and an
    unsplit control) is called back to back on torch's current stream through
    ``mi_matmul_lhsT_rhs_bf16`` (which keeps a workspace per stream) and
    through ``mi_matmul_lhsT_rhs_bf16_noalloc`` (a static device array: no
    allocation of any kind), the two in alternating rounds.  Per entry point:
    the wall time per call of 400 back-to-back calls with one synchronisation
    (best of 5 rounds), and the host time to issue 200 calls without waiting.
    Equal back-to-back times mean the allocating entry point adds nothing the
    GPU waits for."""
    import ctypes

    import torch

    import kernel_library as kl
    from kernel_library import _lib

    lib = _lib.lib()
    stream = torch.cuda.current_stream(dev).cuda_stream
    rows = []
    for (m, n, k), name in SPLIT_HOST_CASES:
        a = torch.empty((k, m), dtype=torch.bfloat16, device=dev).uniform_(-1, 1)
        b = torch.empty((k, n), dtype=torch.bfloat16, device=dev).uniform_(-1, 1)
        out = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        c = kl.TileConfig.from_name(name).to_c()
        fns = {e: getattr(lib, e) for e in ("mi_matmul_lhsT_rhs_bf16", "mi_matmul_lhsT_rhs_bf16_noalloc")}
        call_args = (a.data_ptr(), b.data_ptr(), out.data_ptr(), m, n, k, ctypes.byref(c), stream)
        for e, fn in fns.items():
            for _ in range(50):
                rc = fn(*call_args)
                if rc != 0:
                    raise RuntimeError(f"{e} {name}: {_lib.last_error()}")
        torch.cuda.synchronize()
        b2b = {e: float("inf") for e in fns}
        issue = {e: float("inf") for e in fns}
        for _ in range(5):
            for e, fn in fns.items():
                t0 = time.perf_counter()
                for _ in range(400):
                    fn(*call_args)
                torch.cuda.synchronize()
                b2b[e] = min(b2b[e], (time.perf_counter() - t0) / 400)
                t0 = time.perf_counter()
                for _ in range(200):
                    fn(*call_args)
                issue[e] = min(issue[e], (time.perf_counter() - t0) / 200)
                torch.cuda.synchronize()
        r = {"shape": [m, n, k], "config": name}
        for e in fns:
            r[e] = {"back_to_back_us": round(b2b[e] * 1e6, 2), "host_issue_us": round(issue[e] * 1e6, 2)}
        log(json.dumps(r))
        rows.append(r)
        del a, b, out
    print(json.dumps({"workload": "split-host", "rows": rows}), flush=True)
    return 0


def random_default_shapes(seed: int = 2026, count: int = 30) -> list:
    """Shapes the default config was not fitted to: 14 lhsT.rhs, 6 lhs.rhs and 10 rmsnorm_matmul shapes,
    drawn from a fixed seed.  Each draw is skinny (M from 8 to 128) with probability 1/4; the others have M of
    256 to 8192, N of 512 to 14336 and K of 512 to 16384, in steps of 64.  A draw over 5e11 FLOP is redrawn (so
    the sweep stays short), which leaves more skinny shapes than a quarter: 9, 9 and 17 of 30 for seeds 2026,
    2027 and 2028."""
    import numpy as np

    rng = np.random.default_rng(seed)
    fams = ["matmul_lhsT_rhs"] * 14 + ["matmul_lhs_rhs"] * 6 + ["rmsnorm_matmul"] * 10
    out = []
    for fam in fams[:count]:
        while True:
            skinny = rng.random() < 0.25
            m = int(rng.choice([8, 16, 32, 48, 64, 96, 128])) if skinny else int(rng.integers(4, 129)) * 64
            n = int(rng.integers(8, 225)) * 64
            k = int(rng.integers(8, 257)) * 64
            if 2.0 * m * n * k <= 5e11:
                break
        out.append((fam, (m, n, k)))
    return out


def defaults_study(args, dev, jobs: list, name: str) -> int:
    """--workload defaults / defaults-random: how close does a call without a config come to the autotuned best?

    For each (kernel, shape) of ``jobs``: the library default (``mi_default_config``, not the
    tuned table) and the autotune sweep over every legal prebuilt config
    (10 reps each, numerics-gated, the 4 fastest re-timed), then the default
    and the sweep's winner re-timed together in 5 interleaved rounds.  Skinny
    shapes (M <= 128) overwrite a 512 MiB buffer before every launch, so the
    weight streams from HBM as it does in decode.  One JSON row per shape on
    stderr, the whole table as one line on stdout."""
    import ctypes
    import statistics

    import kernel_library as kl
    from autotune.tune import refine, tune
    from kernel_library import _lib
    from kernel_library.config import kernel_id

    rows = []
    for fam, (m, n, k) in jobs:
        c = _lib.MiTileCfg()
        _lib.check_rc(_lib.lib().mi_default_config(kernel_id(fam), m, n, k, ctypes.byref(c)), "mi_default_config")
        dflt = kl.TileConfig.from_c(c)
        # Skinny M (decode): the weight streams from HBM, as in the C5
        # measurements (a 512 MiB buffer overwritten before every launch).
        flush = 512 << 20 if m <= 128 else 0
        res = tune(fam, m, n, k, check=True, warmup=3, reps=10, allow_jit=False, finalists=4, rounds=3,
                   flush_bytes=flush)
        if res.best is None:
            raise RuntimeError(f"no working config for {fam} {m}x{n}x{k}")
        cfgs = [dflt] if res.best.name == dflt.name else [dflt, res.best]
        t = refine(fam, m, n, k, cfgs, rounds=5, reps=20, flush_bytes=flush)
        row = {"kernel": fam, "shape": [m, n, k], "default": dflt.name, "default_us": round(t[dflt.name] * 1e6, 1),
               "best": res.best.name, "best_us": round(t[res.best.name] * 1e6, 1),
               "default_over_best": round(t[dflt.name] / t[res.best.name], 3),
               "best_tflops": round(2.0 * m * n * k / t[res.best.name] / 1e12, 1)}
        log(json.dumps(row))
        rows.append(row)
    ratios = [r["default_over_best"] for r in rows]
    print(json.dumps({"workload": name, "shapes": len(rows), "median_default_over_best": statistics.median(ratios),
                      "max_default_over_best": max(ratios), "rows": rows}), flush=True)
    return 0


def shape_main(args, dev, m: int, k: int, n: int) -> int:
    """--workload c4a|c4b|c4c|c3-matmul: the lhsT.rhs matmul at one shape with its tuned config (or --config).

    The command the C4 profiles (and the fused kernel's like-for-like matmul
    profile) are taken with; prints a line of its own."""
    import torch

    import kernel_library as kl
    from autotune.runner.benchmark import generate_tensors, upload
    from autotune.tune import default_dists, input_specs

    fam = "matmul_lhsT_rhs"
    cfg = kl.TileConfig.from_name(args.config) if args.config else kl.default_config(fam, m, n, k)
    specs = input_specs(fam, m, n, k)
    d = upload(generate_tensors(specs, 0, default_dists(fam, k)), specs, dev)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=dev)

    def step():
        kl.matmul_lhsT_rhs(d["lhs_T"], d["rhs"], cfg=cfg, out=out)

    settle(step, args.settle_s)
    for _ in range(args.warmup):
        step()
    stream = torch.cuda.current_stream(dev)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record(stream)
    for _ in range(args.steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    kern_s = ev0.elapsed_time(ev1) * 1e-3 / args.steps
    tf = 2.0 * m * n * k / kern_s / 1e12
    log(f"timed {args.steps} steps of {fam} M={m} K={k} N={n} {cfg.name}: avg {kern_s * 1e6:.1f} us")
    print(json.dumps({
        "metric": f"bf16 TFLOP/s, {fam} (M,K,N)=({m},{k},{n}) (profiling workload, not the headline metric)",
        "value": round(tf, 1), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(kern_s * 1e3, 5), "higher_is_better": True, "dtype": "bf16",
        "config": {"workload": f"{fam} M={m}, K={k}, N={n}", "tile_config": cfg.name},
        "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tf / PEAK_BF16_TFLOPS, 4), "traffic": None},
    }, ensure_ascii=False), flush=True)
    return 0


def skinny_main(args, dev) -> int:
    """--workload c5 / decode: one HBM-bound kernel at (--m, 28672, 8192), back-to-back launches.

    The command the skinny kernel profiles are taken with; the line's
    roofline is HBM bytes (compulsory, algorithmic) over the launch time."""
    import torch

    import kernel_library as kl

    fam = "matmul_lhsT_rhs" if args.workload == "c5" else "rmsnorm_matmul"
    m = args.m
    cfg = kl.TileConfig.from_name(args.config) if args.config else kl.default_config(fam, m, SKINNY_N, SKINNY_K)
    d = skinny_inputs(fam, m, dev)
    out = torch.empty((m, SKINNY_N), dtype=torch.bfloat16, device=dev)
    if fam == "matmul_lhsT_rhs":
        def step():
            kl.matmul_lhsT_rhs(d["lhs_T"], d["rhs"], cfg=cfg, out=out)
    else:
        def step():
            kl.rmsnorm_matmul(d["lhs"], d["rhs"], d["gamma"], cfg=cfg, out=out)
    settle(step, args.settle_s)
    for _ in range(args.warmup):
        step()
    stream = torch.cuda.current_stream(dev)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kern_s = ev0.elapsed_time(ev1) * 1e-3 / args.steps
    nbytes = skinny_bytes(fam, m)
    log(f"timed {args.steps} steps of {fam} {m}x{SKINNY_N}x{SKINNY_K} {cfg.name}: kernel avg {kern_s * 1e6:.1f} us")
    print(json.dumps({
        "metric": f"HBM GB/s, {fam} {m}x{SKINNY_N}x{SKINNY_K} (profiling workload, not the headline metric)",
        "value": round(nbytes * args.steps / wall / 1e9, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 5),
        "higher_is_better": True,
        "dtype": "bf16",
        "config": {"workload": f"{fam} M={m}, N={SKINNY_N}, K={SKINNY_K}", "tile_config": cfg.name},
        "roofline": {"bound": "hbm", "achieved": round(nbytes / kern_s / 1e9, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(nbytes / kern_s / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": recorded_traffic(fam, f"{m}x{SKINNY_N}x{SKINNY_K}", cfg.name)},
    }, ensure_ascii=False), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
