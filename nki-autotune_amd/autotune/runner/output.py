"""Profile output: result table, selection, and the cache-directory layout.

Follows reference autotune/src/autotune/runner/output.py: ``SuccessRow``
(:18-25), ``ProfileOutput`` with ``successes`` / ``failures`` / ``__str__``
(:52-85), per-kernel folders ``<cache>/<stem>/`` holding the kernel source
and ``profile_summary.json`` (:143-215), and ``results.json`` with metadata,
metrics and a naturally sorted kernel index (:218-271).  Differences, all
additive: the source file is ``<stem>.hip`` (the kernel instance), the
compile log is ``log-hipcc.txt``, each row also carries TFLOP/s and the
tile config, and the failure counters classify LDS/legality rejections
instead of SBUF/PSUM out-of-memory.
"""

from __future__ import annotations

import json
import os
from dataclasses import dataclass
from pathlib import Path
from typing import NamedTuple

from autotune.runner.types import KernelJob, ProfileResult, profiler_percent

_PROFILE_SUMMARY_FILE = "profile_summary.json"
_PROFILE_DETAILED_FILE = "profile.json"
_COMPILE_LOG_FILE = "log-hipcc.txt"


class SuccessRow(NamedTuple):
    """Kernel result narrowed to the fields of the table (reference output.py:18-25)."""

    kernel_name: str
    total_time_s: float
    mfu: float
    mbu: float | None
    roofline_ceiling: float | None
    tflops: float | None = None
    config: str = ""


def _collect_successes(results: list[ProfileResult]) -> list[SuccessRow]:
    """Kernels that resolved, ran on the GPU and produced a timing summary."""
    rows: list[SuccessRow] = []
    for r in results:
        if not r.hardware_output.startswith("["):
            continue
        summary = r.profiler_summary or {}
        total = summary.get("total_time")
        if not isinstance(total, (int, float)):
            continue
        mfu = profiler_percent(summary, "mfu_estimated_percent")
        if mfu is None:
            continue
        cfg = summary.get("config") or {}
        rows.append(
            SuccessRow(
                kernel_name=r.kernel_name,
                total_time_s=float(total),
                mfu=mfu,
                mbu=profiler_percent(summary, "mbu_estimated_percent"),
                roofline_ceiling=profiler_percent(summary, "mfu_max_achievable_estimated_percent"),
                tflops=summary.get("tflops"),
                config=_cfg_name(cfg),
            )
        )
    return rows


def _cfg_name(cfg: dict) -> str:
    if not cfg:
        return ""
    s = f"bm{cfg['block_m']}_bn{cfg['block_n']}_bk{cfg['block_k']}_w{cfg['waves']}_s{cfg['lds_stages']}"
    if cfg.get("group_m", 8) != 8:
        s += f"_g{cfg['group_m']}"
    if cfg.get("variant", 0):
        s += f"_v{cfg['variant']}"
    return s


@dataclass
class ProfileOutput:
    """Results of one profiling run (reference output.py:52-85)."""

    results: list[ProfileResult]
    compiler_logs: dict[str, str]
    elapsed_s: float
    cache_dir: str = ""

    @property
    def successes(self) -> list[SuccessRow]:
        """Kernels that resolved and produced GPU timings."""
        return _collect_successes(self.results)

    @property
    def failures(self) -> list[ProfileResult]:
        """Kernels that failed legality, compilation or execution."""
        return [r for r in self.results if r.profiler_summary is None or not r.hardware_output.startswith("[")]

    @property
    def best(self) -> SuccessRow | None:
        """The selection step: ``min(successes, key=total_time_s)``
        (reference examples/tune_matmul_lhsT_rhs.py:238; output.py:251)."""
        rows = self.successes
        return min(rows, key=lambda s: s.total_time_s) if rows else None

    def __str__(self) -> str:
        lines: list[str] = []
        successes = self.successes
        lines.extend(_format_results_table(successes))
        lines.extend(_format_failures(self.failures))
        lines.extend(_format_summary(successes, self))
        return "\n".join(lines)


def _fmt_pct(value: float | None) -> str:
    return "-" if value is None else f"{value:.2f}%"


def _format_results_table(successes: list[SuccessRow]) -> list[str]:
    lines: list[str] = []
    show_roofline = any(s.mbu is not None or s.roofline_ceiling is not None for s in successes)
    header = f"{'Kernel':<40} {'total_s':>10} {'TFLOP/s':>9} {'mfu':>8}"
    if show_roofline:
        header += f" {'mbu':>8} {'ceiling':>8}"
    for s in sorted(successes, key=lambda s: s.total_time_s):
        if not lines:
            lines.append(header)
            lines.append("-" * len(header))
        tf = "-" if s.tflops is None else f"{s.tflops:.1f}"
        row = f"{s.kernel_name:<40} {s.total_time_s:>10.6f} {tf:>9} {s.mfu:>7.2f}%"
        if show_roofline:
            row += f" {_fmt_pct(s.mbu):>8} {_fmt_pct(s.roofline_ceiling):>8}"
        lines.append(row)
    return lines


def _format_failures(failures: list[ProfileResult]) -> list[str]:
    lines: list[str] = []
    for i, r in enumerate(failures):
        if i == 0:
            lines.append(f"\n{len(failures)} failures:")
        first = r.hardware_output.strip().splitlines()
        lines.append(f"  {r.kernel_name}: {first[-1] if first else r.hardware_output}")
    return lines


def _format_summary(successes: list[SuccessRow], output: ProfileOutput) -> list[str]:
    lines = ["\nSummary:", f"  Succeeded:  {len(successes)}/{len(output.results)}",
             f"  Wallclock:  {output.elapsed_s:.1f}s"]
    if successes:
        best = min(successes, key=lambda s: s.total_time_s)
        lines.append(f"  Best:       {best.total_time_s:.6f} s ({best.kernel_name})")
        lines.append(f"  Worst:      {max(s.total_time_s for s in successes):.6f} s")
    if output.cache_dir:
        lines.append(f"  Cache:      {output.cache_dir}")
    return lines


def write_kernel_sources(cache_dir: str, kernels: dict[str, KernelJob]) -> None:
    """Write each kernel instance source to ``<cache>/<stem>/<stem>.hip``."""
    for kname, job in kernels.items():
        stem = Path(kname).stem
        variant_dir = os.path.join(cache_dir, stem)
        os.makedirs(variant_dir, exist_ok=True)
        with open(os.path.join(variant_dir, f"{stem}.hip"), "w") as f:
            f.write(job.source)


def write_compiler_logs(cache_dir: str, compiler_logs: dict[str, str]) -> None:
    """Write build logs to ``<cache>/<stem>/log-hipcc.txt``."""
    for kname, log_text in compiler_logs.items():
        stem = Path(kname).stem
        variant_dir = os.path.join(cache_dir, stem)
        os.makedirs(variant_dir, exist_ok=True)
        with open(os.path.join(variant_dir, _COMPILE_LOG_FILE), "w") as f:
            f.write(log_text)


def _kernel_sort_key(kernel_name: str) -> tuple[int, int, str]:
    """Natural sort: ``<prefix>_<N>`` by N, then the rest alphabetically (reference output.py:164-176)."""
    stem = Path(kernel_name).stem
    tail = stem.rsplit("_", 1)[-1]
    return (0, int(tail), stem) if tail.isdigit() else (1, 0, stem)


def _write_per_kernel_profiles(cache_dir: str, results: list[ProfileResult]) -> None:
    for r in results:
        stem = Path(r.kernel_name).stem
        variant_dir = os.path.join(cache_dir, stem)
        os.makedirs(variant_dir, exist_ok=True)
        if r.profiler_summary is not None:
            with open(os.path.join(variant_dir, _PROFILE_SUMMARY_FILE), "w") as f:
                json.dump(r.profiler_summary, f, indent=2)
        if r.profile_detailed is not None:
            with open(os.path.join(variant_dir, _PROFILE_DETAILED_FILE), "w") as f:
                json.dump(r.profile_detailed, f)


def _kernel_index_row(r: ProfileResult, total_time_s, mfu, mbu, ceiling) -> dict:
    stem = Path(r.kernel_name).stem
    summary = r.profiler_summary or {}
    return {
        "kernel_name": r.kernel_name,
        "kernel_path": f"{stem}/{stem}.hip",
        "hardware_output": r.hardware_output,
        "total_time_s": total_time_s,
        "tflops": summary.get("tflops"),
        "config": summary.get("config"),
        "mfu_estimated_percent": mfu,
        "mbu_estimated_percent": mbu,
        "mfu_max_achievable_estimated_percent": ceiling,
    }


# Failure classes counted in results.json (the reference counts SBUF/PSUM OOM, output.py:236-239).
_FAILURE_CLASSES = {
    "lds_over_budget": "LDS over budget",
    "illegal_config": "illegal config",
    "compile_error": "hipcc failed",
    "timeout": "timed out",
}


def write_results_json(cache_dir: str, num_kernels: int, results: list[ProfileResult], wallclock_s: float) -> None:
    """Write results.json (index + metrics) and the per-kernel summaries."""
    _write_per_kernel_profiles(cache_dir, results)
    extracted = {}
    counters = {k: 0 for k in _FAILURE_CLASSES}
    success = 0
    for r in results:
        total = (r.profiler_summary or {}).get("total_time")
        total_s = float(total) if isinstance(total, (int, float)) else None
        extracted[r.kernel_name] = (
            total_s,
            profiler_percent(r.profiler_summary, "mfu_estimated_percent"),
            profiler_percent(r.profiler_summary, "mbu_estimated_percent"),
            profiler_percent(r.profiler_summary, "mfu_max_achievable_estimated_percent"),
        )
        if total_s is not None:
            success += 1
            continue
        for key, needle in _FAILURE_CLASSES.items():
            if needle in r.hardware_output:
                counters[key] += 1
                break
    ok = [(r, extracted[r.kernel_name]) for r in results if extracted[r.kernel_name][0] is not None]
    times = [e[0] for _, e in ok]
    mfus = [e[1] for _, e in ok if e[1] is not None]
    mbus = [e[2] for _, e in ok if e[2] is not None]
    best = min(ok, key=lambda s: s[1][0])[0] if ok else None
    worst = max(ok, key=lambda s: s[1][0])[0] if ok else None
    data = {
        "metadata": {"num_kernels": num_kernels, "wallclock_s": wallclock_s},
        "metrics": {
            "best_total_time_s": min(times) if times else None,
            "worst_total_time_s": max(times) if times else None,
            "best_kernel": best.kernel_name if best else None,
            "worst_kernel": worst.kernel_name if worst else None,
            "best_config": (best.profiler_summary or {}).get("config") if best else None,
            "best_tflops": (best.profiler_summary or {}).get("tflops") if best else None,
            "best_mfu": max(mfus) if mfus else None,
            "worst_mfu": min(mfus) if mfus else None,
            "best_mbu": max(mbus) if mbus else None,
            "worst_mbu": min(mbus) if mbus else None,
            "success": success,
            **counters,
        },
        "kernels": [_kernel_index_row(r, *extracted[r.kernel_name])
                    for r in sorted(results, key=lambda r: _kernel_sort_key(r.kernel_name))],
    }
    with open(os.path.join(cache_dir, "results.json"), "w") as f:
        json.dump(data, f, indent=2)
