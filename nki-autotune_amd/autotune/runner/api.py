"""Local profiling API (reference autotune/src/autotune/runner/api.py:24-75).

``profile(kernels, cache_dir, seed, platform_target, collect_detailed_profile)``
builds and times a set of kernel instances on this MI355X and writes the
standard cache layout (instance sources, results.json, per-kernel
profile_summary.json) under ``cache_dir``; an empty ``cache_dir`` skips all
disk output.  With ``collect_detailed_profile`` and a cache dir, each
successful instance is also re-run under rocprofv3 in a child process and
its kernel trace kept in its folder (``rocprof/``, ``replay.json``; the
stats row goes into ``profile.json``).  Per-kernel failures never raise: they are returned as
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


def profile(
    kernels: dict[str, KernelJob],
    cache_dir: str,
    seed: int,
    platform_target: str = "gfx950",
    collect_detailed_profile: bool = False,
    *,
    warmup: int = 10,
    reps: int = 50,
    flush_bytes: int = 0,
    allow_jit: bool = True,
) -> ProfileOutput:
    """Build + benchmark kernel instances in-process on GPU 0.

    Args:
        kernels: Map of kernel file name to KernelJob.
        cache_dir: Output directory; "" skips disk output.
        seed: RNG seed of the input tensors.
        platform_target: Offload arch the instances are built for
            (``neuron_platform_target`` in the reference); only "gfx950".
        collect_detailed_profile: Attach per-rep timings to each result
            (``profile.json`` in the kernel's cache folder) and, with a
            cache dir, a rocprofv3 kernel trace of each successful instance.
        warmup, reps: hipEvent timing schedule (median of ``reps``).
        flush_bytes: Size of a scratch buffer written before each timed
            launch, to evict L2 / MALL (0 = off).
        allow_jit: Build configs that are not prebuilt with hipcc.
    """
    if platform_target != "gfx950":
        raise ValueError(f"platform_target {platform_target!r} unsupported: the kernels are written for gfx950")
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

    from autotune.runner.trace import trace_kernel, write_replay_job

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
        results[i] = r._replace(profile_detailed={**(r.profile_detailed or {}), "rocprof": row})
        logger.info("Traced %s: %s", r.kernel_name, row.get("avg_ns", row.get("error")))
