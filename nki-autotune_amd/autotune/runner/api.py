"""Local profiling API (reference autotune/src/autotune/runner/api.py:24-75).

``profile(kernels, cache_dir, seed, neuron_platform_target, collect_detailed_profile)``
builds and times a set of kernel instances on this MI355X and writes the
standard cache layout (instance sources, results.json, per-kernel
profile_summary.json) under ``cache_dir``; an empty ``cache_dir`` skips all
disk output.  With ``collect_detailed_profile`` and a cache dir, each
successful instance is also re-run under rocprofv3 in child processes: a
kernel trace (``rocprof/``, ``replay.json``; the stats row goes into
``profile.json``) and one counter pass whose MFMA-busy %, HBM GB/s and
engine clock go into ``profile.json`` and results.json.  Per-kernel failures never raise: they are returned as
``ProfileResult.hardware_output`` text.  Only environment faults raise (no
GPU, wrong arch, a batch asking for more than one device).
"""

from __future__ import annotations

import logging
import os
import time

from autotune.runner.compile import canonical_name, problem_shape
from autotune.runner.driver import run_pipeline
from autotune.runner.output import ProfileOutput, write_compiler_logs, write_kernel_sources, write_results_json
from autotune.runner.types import KernelJob

logger = logging.getLogger(__name__)


# The one offload target of this build, and the reference's Neuron targets,
# which callers of the reference pass as ``neuron_platform_target`` and which
# name the same role: the device the kernels are built and run for.
TARGET = "gfx950"
NEURON_TARGETS = ("trn1", "trn2", "trn3", "inf2")


def resolve_target(neuron_platform_target: str) -> str:
    """The offload arch a ``neuron_platform_target`` value selects.

    "gfx950" selects itself; a Neuron target name (what the reference's
    callers pass) maps onto gfx950, the only device this build has kernels
    for; anything else raises ValueError.
    """
    if neuron_platform_target == TARGET:
        return TARGET
    if neuron_platform_target in NEURON_TARGETS:
        logger.info("neuron_platform_target=%r runs on this build's target %s", neuron_platform_target, TARGET)
        return TARGET
    raise ValueError(f"neuron_platform_target {neuron_platform_target!r} unsupported: the kernels are written for "
                     f"{TARGET} (Neuron names {NEURON_TARGETS} map onto it)")


def profile(
    kernels: dict[str, KernelJob],
    cache_dir: str,
    seed: int,
    neuron_platform_target: str = TARGET,
    collect_detailed_profile: bool = False,
    *,
    warmup: int = 10,
    reps: int = 50,
    flush_bytes: int = 0,
    allow_jit: bool = True,
    check_numerics: bool = True,
) -> ProfileOutput:
    """Build + benchmark kernel instances in-process on GPU 0.

    Args:
        kernels: Map of kernel file name to KernelJob.
        cache_dir: Output directory; "" skips disk output.
        seed: RNG seed of the input tensors.
        neuron_platform_target: Target the instances are built for, under the
            reference's argument name: "gfx950", or a Neuron target name
            ("trn2", ...) which maps onto gfx950 (:func:`resolve_target`).
        collect_detailed_profile: Attach per-rep timings to each result
            (``profile.json`` in the kernel's cache folder) and, with a
            cache dir, a rocprofv3 kernel trace of each successful instance.
        warmup, reps: hipEvent timing schedule (median of ``reps``).
        flush_bytes: Size of a scratch buffer written before each timed
            launch, to evict L2 / MALL (0 = off).
        allow_jit: Build configs that are not prebuilt with hipcc.
        check_numerics: Check every timed instance's output against a
            float64 evaluation of its inputs; failures become failure rows
            (the role of the reference's per-candidate simulator check).
    """
    resolve_target(neuron_platform_target)
    if cache_dir:
        os.makedirs(cache_dir, exist_ok=True)
        write_kernel_sources(cache_dir, kernels)
    t0 = time.monotonic()
    results, compiler_logs = run_pipeline(
        kernels,
        seed=seed,
        collect_compiler_logs=bool(cache_dir),
        collect_detailed_profile=collect_detailed_profile,
        warmup=warmup,
        reps=reps,
        flush_bytes=flush_bytes,
        allow_jit=allow_jit,
        check_numerics=check_numerics,
    )
    if collect_detailed_profile and cache_dir:
        _trace_successes(cache_dir, kernels, results, seed, warmup, reps, flush_bytes)
    elapsed_s = time.monotonic() - t0
    logger.info("Profile complete: %d results in %.1fs", len(results), elapsed_s)
    if cache_dir:
        write_compiler_logs(cache_dir, compiler_logs)
        write_results_json(cache_dir, len(kernels), results, elapsed_s)
        logger.info("Cache saved to %s", cache_dir)
    return ProfileOutput(results=results, compiler_logs=compiler_logs, elapsed_s=elapsed_s, cache_dir=cache_dir)


def _trace_successes(cache_dir: str, kernels: dict[str, KernelJob], results, seed: int, warmup: int, reps: int,
                     flush_bytes: int) -> None:
    """rocprofv3 kernel trace of every successful instance, into its cache folder."""
    from pathlib import Path

    from autotune.runner.trace import collect_counters, trace_kernel, write_replay_job

    for i, r in enumerate(results):
        summary = r.profiler_summary
        job = kernels.get(r.kernel_name)
        if summary is None or job is None:
            continue
        variant_dir = os.path.join(cache_dir, Path(r.kernel_name).stem)
        replay = write_replay_job(variant_dir, r.kernel_name, canonical_name(job.func_name), summary["library"],
                                  summary["config"], problem_shape(job.func_name, job.input_specs),
                                  job.input_specs, job.input_dists, seed, warmup, reps, flush_bytes)
        row = trace_kernel(variant_dir, replay)
        counters = collect_counters(variant_dir, replay)
        results[i] = r._replace(profile_detailed={**(r.profile_detailed or {}), "rocprof": row, "counters": counters},
                                ntff_b64=trace_b64(row))
        logger.info("Traced %s: %s; counters %s", r.kernel_name, row.get("avg_ns", row.get("error")),
                    {k: counters.get(k) for k in ("mfma_busy_percent", "engine_clock_mhz", "hbm_gbps", "error")})


def trace_b64(row: dict) -> str | None:
    """Base64 of the replay's rocprofv3 kernel trace (one CSV row per dispatch), the NTFF's counterpart, or None."""
    import base64

    path = os.path.join(row.get("trace_dir") or "", "run_kernel_trace.csv")
    if "error" in row or not row.get("trace_dir") or not os.path.exists(path):
        return None
    with open(path, "rb") as f:
        return base64.b64encode(f.read()).decode("ascii")
