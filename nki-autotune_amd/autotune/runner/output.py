"""Profile output: one results model, rendered as the table and as results.json.

The reference's callers read a fixed surface, kept here
(reference autotune/src/autotune/runner/output.py): ``SuccessRow`` (:18-25),
``ProfileOutput.successes`` / ``failures`` / ``__str__`` (:52-85), the
per-kernel cache folders ``<cache>/<stem>/`` with ``profile_summary.json``
(:143-215) and ``results.json`` with its ``metadata`` / ``metrics`` /
``kernels`` keys (:218-271).

Behind that surface every ProfileResult is normalised once into a
:class:`KernelRecord` (ran or not, time, utilisation, counters, failure
class), and a :class:`ResultsModel` holds the records plus an optional
vendor-library baseline row.  The text table, the selection (``best``) and
the JSON document are three views of that one model.  Additions to the
reference's fields: TFLOP/s and the tile config per kernel, the measured
counters when a detailed profile took them (MFMA-busy %, HBM GB/s, engine
clock), failure classes for LDS / legality / hipcc / timeout / numerics
instead of SBUF / PSUM out-of-memory, and the baseline row.
"""

from __future__ import annotations

import json
import os
import re
from dataclasses import dataclass, field
from pathlib import Path
from typing import NamedTuple

from autotune.runner.types import KernelJob, ProfileResult, profiler_percent

SUMMARY_FILE = "profile_summary.json"
DETAILED_FILE = "profile.json"
COMPILE_LOG_FILE = "log-hipcc.txt"

# Failure classes counted in results.json: key -> text that marks it in a
# kernel's hardware_output (first match wins).
FAILURE_CLASSES = (
    ("lds_over_budget", "LDS over budget"),
    ("illegal_config", "illegal config"),
    ("compile_error", "hipcc failed"),
    ("timeout", "timed out"),
    ("numerics_mismatch", "numerics check failed"),
)
# The reference's out-of-memory counters of results.json (output.py:225-239,
# :265-266), kept under their names: SBUF is the on-chip scratchpad, whose
# counterpart is LDS ("LDS over budget", the lds_over_budget class above);
# PSUM holds the matmul accumulators, whose counterpart is a wave's
# accumulator registers (the legality check's message for a wave tile whose
# fp32 accumulators exceed its share of the SIMD's 512 registers).
OOM_MARKS = (("sbuf_oom", "LDS over budget"), ("psum_oom", "exceed its share of the 512 registers"))


class SuccessRow(NamedTuple):
    """A kernel that ran, narrowed to the table's fields (reference output.py:18-25)."""

    kernel_name: str
    total_time_s: float
    mfu: float
    mbu: float | None
    roofline_ceiling: float | None
    tflops: float | None = None
    config: str = ""


def config_name(cfg: dict | None) -> str:
    """The tile config's name (kernel_library.TileConfig.name) from its field dict."""
    if not cfg:
        return ""
    name = f"bm{cfg['block_m']}_bn{cfg['block_n']}_bk{cfg['block_k']}_w{cfg['waves']}_s{cfg['lds_stages']}"
    extras = (("_g", cfg.get("group_m", 8), 8), ("_v", cfg.get("variant", 0), 0), ("_k", cfg.get("split_k", 1), 1))
    return name + "".join(f"{tag}{v}" for tag, v, default in extras if v != default)


@dataclass(frozen=True)
class KernelRecord:
    """One ProfileResult, normalised."""

    result: ProfileResult
    time_s: float | None          # median launch time; None when the kernel did not run
    mfu: float | None             # percent of the MFMA peak (algorithmic FLOPs / time)
    mbu: float | None             # percent of the HBM peak (compulsory bytes / time)
    ceiling: float | None         # roofline ceiling of the shape, percent of the MFMA peak
    failure: str | None           # failure class key, None for a success

    @property
    def name(self) -> str:
        return self.result.kernel_name

    @property
    def summary(self) -> dict:
        return self.result.profiler_summary or {}

    @property
    def ok(self) -> bool:
        return self.time_s is not None and self.mfu is not None

    @property
    def counters(self) -> dict:
        """Measured counters of a detailed profile (empty when none were taken)."""
        return (self.result.profile_detailed or {}).get("counters") or {}

    @classmethod
    def of(cls, r: ProfileResult) -> "KernelRecord":
        summary = r.profiler_summary or {}
        t = summary.get("total_time")
        ran = r.hardware_output.startswith("[") and isinstance(t, (int, float))
        failure = None
        if not ran:
            failure = next((key for key, mark in FAILURE_CLASSES if mark in r.hardware_output), "other")
        return cls(result=r, time_s=float(t) if ran else None,
                   mfu=profiler_percent(summary, "mfu_estimated_percent") if ran else None,
                   mbu=profiler_percent(summary, "mbu_estimated_percent") if ran else None,
                   ceiling=profiler_percent(summary, "mfu_max_achievable_estimated_percent") if ran else None,
                   failure=failure)

    def success_row(self) -> SuccessRow:
        return SuccessRow(self.name, self.time_s, self.mfu, self.mbu, self.ceiling, self.summary.get("tflops"),
                          config_name(self.summary.get("config")))

    def index_entry(self) -> dict:
        """This kernel's entry in results.json's ``kernels`` list."""
        stem = Path(self.name).stem
        c = self.counters
        return {
            "kernel_name": self.name,
            "kernel_path": f"{stem}/{stem}.hip",
            "hardware_output": self.result.hardware_output,
            "total_time_s": self.time_s,
            "tflops": self.summary.get("tflops"),
            "config": self.summary.get("config"),
            "mfu_estimated_percent": self.mfu,
            "mbu_estimated_percent": self.mbu,
            "mfu_max_achievable_estimated_percent": self.ceiling,
            "numerics": self.summary.get("numerics"),
            "mfma_busy_percent": c.get("mfma_busy_percent"),
            "hbm_gbps_measured": c.get("hbm_gbps"),
            "engine_clock_mhz": c.get("engine_clock_mhz"),
        }


def natural_key(name: str) -> list:
    """Sort key that orders digit runs by value: ``kernel_2`` before ``kernel_10``."""
    return [(0, int(tok), "") if tok.isdigit() else (1, 0, tok) for tok in re.split(r"(\d+)", Path(name).stem) if tok]


@dataclass
class ResultsModel:
    """The records of one profiling run, plus an optional baseline row."""

    records: list[KernelRecord]
    baseline: KernelRecord | None = None

    @classmethod
    def of(cls, results: list[ProfileResult], baseline: ProfileResult | None = None) -> "ResultsModel":
        return cls([KernelRecord.of(r) for r in results], KernelRecord.of(baseline) if baseline else None)

    @property
    def ran(self) -> list[KernelRecord]:
        return [k for k in self.records if k.ok]

    def fastest(self) -> KernelRecord | None:
        """The selection step: ``min(total_time)`` (reference examples/tune_matmul_lhsT_rhs.py:238)."""
        return min(self.ran, key=lambda k: k.time_s, default=None)

    def slowest(self) -> KernelRecord | None:
        return max(self.ran, key=lambda k: k.time_s, default=None)

    # ---- text view -------------------------------------------------------
    def table_lines(self) -> list[str]:
        ran = sorted(self.ran, key=lambda k: k.time_s)
        if not ran and self.baseline is None:
            return []
        extra = any(k.mbu is not None or k.ceiling is not None for k in ran)
        measured = any(k.counters for k in ran)
        cols = [("Kernel", 40, "<"), ("total_s", 10, ">"), ("TFLOP/s", 9, ">"), ("mfu", 8, ">")]
        if extra:
            cols += [("mbu", 8, ">"), ("ceiling", 8, ">")]
        if measured:
            cols += [("busy", 7, ">"), ("HBM GB/s", 9, ">"), ("MHz", 6, ">")]
        head = " ".join(f"{t:{a}{w}}" for t, w, a in cols)
        lines = [head, "-" * len(head)]
        for k in ran:
            lines.append(self._row(k, extra, measured))
        if self.baseline is not None:
            lines.append("-" * len(head))
            if self.baseline.ok:
                lines.append(self._row(self.baseline, extra, measured))
                best = self.fastest()
                if best is not None:
                    lines.append(f"{'best kernel vs ' + self.baseline.name:<40} "
                                 f"{self.baseline.time_s / best.time_s:>9.3f}x faster")
            else:
                lines.append(f"{self.baseline.name:<40} unavailable: {_last_line(self.baseline.result)}")
        return lines

    @staticmethod
    def _row(k: KernelRecord, extra: bool, measured: bool) -> str:
        pct = lambda v: "-" if v is None else f"{v:.2f}%"  # noqa: E731
        tf = k.summary.get("tflops")
        row = f"{k.name:<40} {k.time_s:>10.6f} {'-' if tf is None else f'{tf:.1f}':>9} {k.mfu:>7.2f}%"
        if extra:
            row += f" {pct(k.mbu):>8} {pct(k.ceiling):>8}"
        if measured:
            c = k.counters
            busy, gbs, mhz = c.get("mfma_busy_percent"), c.get("hbm_gbps"), c.get("engine_clock_mhz")
            row += (f" {'-' if busy is None else f'{busy:.1f}%':>7} {'-' if gbs is None else f'{gbs:.0f}':>9}"
                    f" {'-' if mhz is None else f'{mhz:.0f}':>6}")
        return row

    def failure_lines(self) -> list[str]:
        failed = [k for k in self.records if not k.ok]
        if not failed:
            return []
        return [f"\n{len(failed)} failures:"] + [f"  {k.name}: {_last_line(k.result)}" for k in failed]

    def summary_lines(self, elapsed_s: float, cache_dir: str) -> list[str]:
        lines = ["\nSummary:", f"  Succeeded:  {len(self.ran)}/{len(self.records)}", f"  Wallclock:  {elapsed_s:.1f}s"]
        best, worst = self.fastest(), self.slowest()
        if best is not None:
            lines += [f"  Best:       {best.time_s:.6f} s ({best.name})", f"  Worst:      {worst.time_s:.6f} s"]
        if cache_dir:
            lines.append(f"  Cache:      {cache_dir}")
        return lines

    # ---- JSON view -------------------------------------------------------
    def document(self, num_kernels: int, wallclock_s: float) -> dict:
        """results.json (reference output.py:218-271 keys, plus the additions above)."""
        best, worst = self.fastest(), self.slowest()
        mfus = [k.mfu for k in self.ran]
        mbus = [k.mbu for k in self.ran if k.mbu is not None]
        counts = {key: sum(1 for k in self.records if k.failure == key) for key, _ in FAILURE_CLASSES}
        metrics = {
            "best_total_time_s": best.time_s if best else None,
            "worst_total_time_s": worst.time_s if worst else None,
            "best_kernel": best.name if best else None,
            "worst_kernel": worst.name if worst else None,
            "best_config": best.summary.get("config") if best else None,
            "best_tflops": best.summary.get("tflops") if best else None,
            "best_mfu": max(mfus, default=None),
            "worst_mfu": min(mfus, default=None),
            "best_mbu": max(mbus, default=None),
            "worst_mbu": min(mbus, default=None),
            "success": len(self.ran),
            **{key: sum(1 for k in self.records if not k.ok and mark in k.result.hardware_output)
               for key, mark in OOM_MARKS},
            **counts,
        }
        doc = {"metadata": {"num_kernels": num_kernels, "wallclock_s": wallclock_s}, "metrics": metrics,
               "kernels": [k.index_entry() for k in sorted(self.records, key=lambda k: natural_key(k.name))]}
        if self.baseline is not None:
            b = self.baseline
            doc["baseline"] = {**b.index_entry(), "library": b.summary.get("library")}
            if b.ok and best is not None:
                metrics["baseline_total_time_s"] = b.time_s
                metrics["best_speedup_vs_baseline"] = b.time_s / best.time_s
        return doc


def _last_line(r: ProfileResult) -> str:
    lines = r.hardware_output.strip().splitlines()
    return lines[-1] if lines else r.hardware_output


@dataclass
class ProfileOutput:
    """Results of one profiling run (reference output.py:52-85); ``baseline`` is an optional vendor row."""

    results: list[ProfileResult]
    compiler_logs: dict[str, str]
    elapsed_s: float
    cache_dir: str = ""
    baseline: ProfileResult | None = field(default=None)

    @property
    def model(self) -> ResultsModel:
        return ResultsModel.of(self.results, self.baseline)

    @property
    def successes(self) -> list[SuccessRow]:
        """Kernels that ran on the GPU and produced a timing summary."""
        return [k.success_row() for k in self.model.ran]

    @property
    def failures(self) -> list[ProfileResult]:
        """Kernels that failed legality, compilation, execution or the numerics check."""
        return [k.result for k in self.model.records if not k.ok]

    @property
    def best(self) -> SuccessRow | None:
        """The fastest kernel (reference examples/tune_matmul_lhsT_rhs.py:238)."""
        k = self.model.fastest()
        return k.success_row() if k else None

    def __str__(self) -> str:
        m = self.model
        return "\n".join(m.table_lines() + m.failure_lines() + m.summary_lines(self.elapsed_s, self.cache_dir))


class KernelFolder:
    """``<cache>/<stem>/``: the files of one kernel."""

    def __init__(self, cache_dir: str, kernel_name: str) -> None:
        self.stem = Path(kernel_name).stem
        self.path = os.path.join(cache_dir, self.stem)

    def write(self, file_name: str, text: str) -> None:
        os.makedirs(self.path, exist_ok=True)
        with open(os.path.join(self.path, file_name), "w") as f:
            f.write(text)


def write_kernel_sources(cache_dir: str, kernels: dict[str, KernelJob]) -> None:
    """Each kernel instance's source as ``<cache>/<stem>/<stem>.hip``."""
    for name, job in kernels.items():
        folder = KernelFolder(cache_dir, name)
        folder.write(f"{folder.stem}.hip", job.source)


def write_compiler_logs(cache_dir: str, compiler_logs: dict[str, str]) -> None:
    """Build logs as ``<cache>/<stem>/log-hipcc.txt``."""
    for name, text in compiler_logs.items():
        KernelFolder(cache_dir, name).write(COMPILE_LOG_FILE, text)


def write_results_json(cache_dir: str, num_kernels: int, results: list[ProfileResult], wallclock_s: float,
                       baseline: ProfileResult | None = None) -> None:
    """results.json (index + metrics) and each kernel's profile_summary.json / profile.json."""
    model = ResultsModel.of(results, baseline)
    for k in model.records + ([model.baseline] if model.baseline else []):
        folder = KernelFolder(cache_dir, k.name)
        if k.result.profiler_summary is not None:
            folder.write(SUMMARY_FILE, json.dumps(k.result.profiler_summary, indent=2))
        if k.result.profile_detailed is not None:
            folder.write(DETAILED_FILE, json.dumps(k.result.profile_detailed))
    with open(os.path.join(cache_dir, "results.json"), "w") as f:
        json.dump(model.document(num_kernels, wallclock_s), f, indent=2)
