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
  like every other per-kernel failure of the profiler.

The trace runs in its own process because rocprofv3 has to start the
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
