"""rocprofv3 kernel traces for detailed profiles.

The reference captures ``profile.json`` plus the NEFF/NTFF trace of each
kernel when ``collect_detailed_profile=True``
(autotune/src/autotune/runner/benchmark.py:90-113; output.py:143-215).  The
MI355X analogue is a rocprofv3 kernel trace of the same instance:

* :func:`write_replay_job` writes ``<cache>/<stem>/replay.json``, everything
  a fresh process needs to re-run that instance (library, family, tile
  config, shape, input specs and distributions, seed, timing schedule);
* :func:`trace_kernel` runs ``rocprofv3 --kernel-trace --stats`` over
  ``python -m autotune.runner.replay replay.json`` as a child process into
  ``<cache>/<stem>/rocprof/`` and returns the instance's row of the stats
  (calls, average / min / max duration).  It never raises: a missing
  profiler, a timeout or a failed run is returned as an ``error`` string,
  like every other per-kernel failure of the profiler;
* :func:`collect_counters` runs two rocprofv3 counter passes over the same
  replay (``rocprofv3 --pmc`` takes at most 4 TCC counters per run, and
  FETCH_SIZE alone uses 3) and derives, per call of the instance: the MFMA
  busy fraction, the engine clock and the HBM-side bytes and GB/s -- the
  profiler-measured counterparts of the reference's neuron-profile fields
  (benchmark.py:58-87).  The byte counters are scaled by what they read for
  a device copy of known size made by the same replay just before.

Traces run in their own processes because rocprofv3 has to start the
program it profiles; the profiling process itself keeps its GPU context.
"""

from __future__ import annotations

import csv
import json
import os
import shutil
import signal
import subprocess
import sys
from pathlib import Path

TRACE_TIMEOUT_S = 180
COUNTER_TIMEOUT_S = 120
# MI355X: 8 XCDs of 32 CUs, 4 SIMDs per CU.
NUM_XCDS = 8
NUM_SIMDS = 1024
CALIBRATE_MIB = 256
# GRBM_GUI_ACTIVE covers the counter window around a dispatch, not only the
# kernel: shorter calls than this get no clock or MFMA-busy figure.
MIN_CLOCKED_NS = 50_000
# One counter pass per entry, each within rocprofv3's per-block limits
# (8 SQ, 4 TCC -- FETCH_SIZE takes 3, WRITE_SIZE 2 --, 2 GRBM).
COUNTER_PASSES = (("SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE", "FETCH_SIZE"), ("WRITE_SIZE", "GRBM_GUI_ACTIVE"))
_PKG_DIR = Path(__file__).resolve().parents[2]   # nki-autotune_amd/


def write_replay_job(variant_dir: str, kernel_name: str, func_name: str, library_path: str, config: dict,
                     shape: tuple[int, int, int], input_specs: dict, input_dists: dict | None, seed: int,
                     warmup: int, reps: int, flush_bytes: int = 0) -> str:
    os.makedirs(variant_dir, exist_ok=True)
    job = {
        "kernel_name": kernel_name,
        "func_name": func_name,
        "library_path": library_path,
        "config": config,
        "shape": list(shape),
        "input_specs": {k: [list(s), d] for k, (s, d) in input_specs.items()},
        "input_dists": {k: (list(v) if isinstance(v, tuple) else v) for k, v in (input_dists or {}).items()},
        "seed": seed,
        "warmup": warmup,
        "reps": reps,
        "flush_bytes": flush_bytes,
    }
    path = os.path.join(variant_dir, "replay.json")
    with open(path, "w") as f:
        json.dump(job, f, indent=2)
    return path


def rocprof_command(out_dir: str, replay_path: str) -> list[str]:
    """The profiler command: the program itself follows ``--`` (no shell, no launcher)."""
    return [shutil.which("rocprofv3") or "rocprofv3", "--kernel-trace", "--stats", "--output-format", "csv", "-d",
            out_dir, "-o", "run", "--", sys.executable, "-u", "-m", "autotune.runner.replay", replay_path]


def parse_kernel_stats(stats_csv: str, match: str = "mi::") -> dict:
    """The rows of rocprofv3's kernel_stats.csv whose kernel name contains ``match``.

    The longest-running one gives the top-level fields; ``kernels`` lists
    every match (a split-K config launches its main kernel and a summing
    kernel per call)."""
    rows = []
    with open(stats_csv) as f:
        for row in csv.DictReader(f):
            if match in row["Name"]:
                rows.append({
                    "kernel": row["Name"],
                    "calls": int(row["Calls"]),
                    "avg_ns": float(row["AverageNs"]),
                    "min_ns": float(row["MinNs"]),
                    "max_ns": float(row["MaxNs"]),
                    "total_ns": float(row["TotalDurationNs"]),
                })
    if not rows:
        raise ValueError(f"no kernel matching {match!r} in {stats_csv}")
    main = dict(max(rows, key=lambda r: r["total_ns"]))
    main["kernels"] = rows
    return main


def trace_kernel(variant_dir: str, replay_path: str, timeout_s: int = TRACE_TIMEOUT_S) -> dict:
    """Run the replay under rocprofv3; return the stats row or ``{"error": ...}``."""
    if shutil.which("rocprofv3") is None:
        return {"error": "rocprofv3 not found on PATH"}
    out_dir = os.path.join(variant_dir, "rocprof")
    shutil.rmtree(out_dir, ignore_errors=True)
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join([str(_PKG_DIR), str(_PKG_DIR.parent), env.get("PYTHONPATH", "")])
    cmd = rocprof_command(out_dir, os.path.abspath(replay_path))
    try:
        proc = subprocess.Popen(cmd, cwd=str(_PKG_DIR), env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                                text=True, start_new_session=True)
        try:
            log, _ = proc.communicate(timeout=timeout_s)
        except subprocess.TimeoutExpired:
            os.killpg(proc.pid, signal.SIGKILL)
            proc.communicate()
            return {"error": f"rocprofv3 trace timed out after {timeout_s} s", "command": cmd}
        with open(os.path.join(variant_dir, "rocprof.log"), "w") as f:
            f.write(log)
        stats = os.path.join(out_dir, "run_kernel_stats.csv")
        if not os.path.exists(stats):
            tail = log.strip().splitlines()[-1] if log.strip() else ""
            return {"error": f"rocprofv3 exited with {proc.returncode} and wrote no kernel stats: {tail}",
                    "command": cmd}
        row = parse_kernel_stats(stats)
        row["command"] = cmd
        row["trace_dir"] = out_dir
        return row
    except Exception as exc:  # per-kernel failures are data, never raised
        return {"error": f"{type(exc).__name__}: {exc}", "command": cmd}


def _run_profiler(cmd: list[str], log_path: str, timeout_s: int) -> tuple[int | None, str]:
    """Run a profiler command in its own process group; (return code or None on timeout, log)."""
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join([str(_PKG_DIR), str(_PKG_DIR.parent), env.get("PYTHONPATH", "")])
    proc = subprocess.Popen(cmd, cwd=str(_PKG_DIR), env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                            text=True, start_new_session=True)
    try:
        log, _ = proc.communicate(timeout=timeout_s)
    except subprocess.TimeoutExpired:
        os.killpg(proc.pid, signal.SIGKILL)
        proc.communicate()
        return None, ""
    with open(log_path, "w") as f:
        f.write(log)
    return proc.returncode, log


def counter_command(out_dir: str, replay_path: str, counters: tuple[str, ...], reps: int) -> list[str]:
    return [shutil.which("rocprofv3") or "rocprofv3", "--pmc", *counters, "--output-format", "csv", "-d", out_dir,
            "-o", "run", "--", sys.executable, "-u", "-m", "autotune.runner.replay", replay_path, "--warmup", "1",
            "--reps", str(reps), "--calibrate-copy-mib", str(CALIBRATE_MIB)]


def read_counter_csv(path: str) -> list[dict]:
    """Dispatches of a rocprofv3 counter_collection.csv in order: name, duration (ns), counters (summed)."""
    by_id: dict[int, dict] = {}
    with open(path) as f:
        for row in csv.DictReader(f):
            d = by_id.setdefault(int(row["Dispatch_Id"]), {
                "name": row["Kernel_Name"],
                "ns": float(row["End_Timestamp"]) - float(row["Start_Timestamp"]),
                "counters": {},
            })
            d["counters"][row["Counter_Name"]] = d["counters"].get(row["Counter_Name"], 0.0) + float(
                row["Counter_Value"])
    return [by_id[i] for i in sorted(by_id)]


def per_call_counters(dispatches: list[dict], calls: int, calibrate_bytes: int, match: str = "mi::") -> dict:
    """Counters of the median timed call of the instance, and the copy calibration.

    A call is ``len(kernel dispatches) / calls`` consecutive dispatches (a
    split-K or two-pass config launches more than one kernel per call); the
    first call is the warm-up.  The calibration is the last device copy
    before the first kernel dispatch: its FETCH_SIZE / WRITE_SIZE (KiB) for
    ``calibrate_bytes`` moved give the byte scale of each counter."""
    first = next((i for i, d in enumerate(dispatches) if match in d["name"]), None)
    if first is None:
        raise ValueError(f"no dispatch matching {match!r}")
    kern = [d for d in dispatches if match in d["name"]]
    per = len(kern) // calls
    if per < 1 or per * calls != len(kern):
        raise ValueError(f"{len(kern)} kernel dispatches for {calls} calls")
    groups = []
    for c in range(1, calls):  # call 0 is the warm-up
        g = kern[c * per:(c + 1) * per]
        tot = {}
        for d in g:
            for k, v in d["counters"].items():
                tot[k] = tot.get(k, 0.0) + v
        groups.append({"ns": sum(d["ns"] for d in g), "counters": tot})
    groups.sort(key=lambda g: g["ns"])
    med = groups[len(groups) // 2]
    copies = [d for d in dispatches[:first] if "copyBuffer" in d["name"]]
    scale = {}
    if copies:
        cal = copies[-1]["counters"]
        for name in ("FETCH_SIZE", "WRITE_SIZE"):
            if cal.get(name):
                scale[name] = calibrate_bytes / (cal[name] * 1024.0)
    return {"ns": med["ns"], "counters": med["counters"], "scale": scale,
            "kernels": sorted({d["name"].split("(")[0] for d in kern})}


def derive(passes: list[dict]) -> dict:
    """MFMA busy %, engine clock (MHz) and HBM bytes / GB/s of one call from the counter passes."""
    out: dict = {"passes": passes}
    c0 = passes[0]["counters"]
    grbm = c0.get("GRBM_GUI_ACTIVE")
    ns = passes[0]["ns"]
    if grbm and ns >= MIN_CLOCKED_NS:
        cycles = grbm / NUM_XCDS
        out["engine_clock_mhz"] = cycles / ns * 1e3
        if "SQ_VALU_MFMA_BUSY_CYCLES" in c0:
            out["mfma_busy_percent"] = 100.0 * c0["SQ_VALU_MFMA_BUSY_CYCLES"] / NUM_SIMDS / cycles
    elif grbm:
        out["note"] = (f"call of {ns / 1e3:.1f} us: GRBM_GUI_ACTIVE also counts the counter window around the "
                       f"dispatch, so clock and MFMA busy are derived for calls of at least "
                       f"{MIN_CLOCKED_NS / 1e3:.0f} us only")
    fetch = c0.get("FETCH_SIZE")
    write = passes[1]["counters"].get("WRITE_SIZE") if len(passes) > 1 else None
    if fetch is not None and write is not None:
        fs = passes[0]["scale"].get("FETCH_SIZE")
        ws = passes[1]["scale"].get("WRITE_SIZE")
        if fs and ws:
            out["fetch_bytes"] = fetch * 1024.0 * fs
            out["write_bytes"] = write * 1024.0 * ws
            out["hbm_bytes"] = out["fetch_bytes"] + out["write_bytes"]
            out["hbm_gbps"] = out["hbm_bytes"] / ns
    return out


def collect_counters(variant_dir: str, replay_path: str, reps: int = 5, timeout_s: int = COUNTER_TIMEOUT_S) -> dict:
    """Counter passes over the replay; the derived figures, or ``{"error": ...}`` (never raises)."""
    if shutil.which("rocprofv3") is None:
        return {"error": "rocprofv3 not found on PATH"}
    passes = []
    try:
        for i, counters in enumerate(COUNTER_PASSES):
            out_dir = os.path.join(variant_dir, f"counters{i}")
            shutil.rmtree(out_dir, ignore_errors=True)
            cmd = counter_command(out_dir, os.path.abspath(replay_path), counters, reps)
            rc, log = _run_profiler(cmd, os.path.join(variant_dir, f"counters{i}.log"), timeout_s)
            if rc is None:
                return {"error": f"counter pass {i} timed out after {timeout_s} s", "command": cmd}
            found = [os.path.join(dp, f) for dp, _, fs in os.walk(out_dir) for f in fs
                     if f.endswith("counter_collection.csv")]
            if not found:
                tail = log.strip().splitlines()[-1] if log.strip() else ""
                return {"error": f"counter pass {i} exited with {rc} and wrote no counters: {tail}", "command": cmd}
            passes.append({**per_call_counters(read_counter_csv(found[0]), 1 + reps, CALIBRATE_MIB << 20),
                           "counter_names": list(counters)})
        return derive(passes)
    except Exception as exc:  # per-kernel failures are data, never raised
        return {"error": f"{type(exc).__name__}: {exc}"}


def read_kernel_trace(path: str) -> list[dict]:
    """Dispatches of a rocprofv3 kernel_trace.csv in start order: name and duration (ns)."""
    rows = []
    with open(path) as f:
        for row in csv.DictReader(f):
            start, end = float(row["Start_Timestamp"]), float(row["End_Timestamp"])
            rows.append({"name": row["Kernel_Name"], "start": start, "ns": end - start})
    rows.sort(key=lambda r: r["start"])
    return rows


def timed_region(dispatches: list[dict], steps: int, product: str = "mm_lhsT_rhs_bf16_pipe_kernel",
                 bracket: str = "clocked_lhsT_rhs_kernel") -> dict:
    """The dispatches of a bench.py timed region in a kernel trace of the whole run.

    bench.py reads the engine clock with the kernel's clocked twin right
    before and right after its ``steps`` timed launches, so the timed region
    is the one run of exactly ``steps`` consecutive dispatches of the
    product kernel with a twin dispatch on each side (the warm-up run before
    the first twin reading has ``--warmup`` dispatches, the settle runs
    more).  Dispatches of other libraries (torch's buffer fills around a
    twin reading) are skipped.  Returns their kernel name and duration
    statistics (us)."""
    ours = [d for d in dispatches if "mi::" in d["name"]]
    runs, i = [], 0
    while i < len(ours):
        if product in ours[i]["name"]:
            j = i
            while j < len(ours) and ours[j]["name"] == ours[i]["name"]:
                j += 1
            before = i > 0 and bracket in ours[i - 1]["name"]
            after = j < len(ours) and bracket in ours[j]["name"]
            if j - i == steps and before and after:
                runs.append(ours[i:j])
            i = j
        else:
            i += 1
    if len(runs) != 1:
        raise ValueError(f"{len(runs)} runs of {steps} {product} dispatches between clocked-twin dispatches")
    ns = sorted(d["ns"] for d in runs[0])
    return {"kernel": runs[0][0]["name"].split("(")[0], "dispatches": len(ns),
            "avg_us": round(sum(ns) / len(ns) / 1e3, 2), "median_us": round(ns[len(ns) // 2] / 1e3, 2),
            "min_us": round(ns[0] / 1e3, 2), "max_us": round(ns[-1] / 1e3, 2)}


def _main() -> int:
    import argparse

    ap = argparse.ArgumentParser(description="rocprofv3 trace summaries")
    sub = ap.add_subparsers(dest="cmd", required=True)
    tr = sub.add_parser("timed-region", help="the bench.py timed region in a kernel_trace.csv of the whole run")
    tr.add_argument("--csv", required=True)
    tr.add_argument("--steps", type=int, required=True)
    tr.add_argument("--flop", type=float, default=2.0 * 8192 ** 3, help="algorithmic FLOP per launch")
    tr.add_argument("--peak-tflops", type=float, default=2500.0)
    args = ap.parse_args()
    res = timed_region(read_kernel_trace(args.csv), args.steps)
    res["tflops_from_avg"] = round(args.flop / (res["avg_us"] * 1e-6) / 1e12, 1)
    res["frac_from_avg"] = round(res["tflops_from_avg"] / args.peak_tflops, 4)
    print(json.dumps(res))
    return 0


if __name__ == "__main__":
    sys.exit(_main())
