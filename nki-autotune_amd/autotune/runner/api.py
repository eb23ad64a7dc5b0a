"""Local profiling API (reference autotune/src/autotune/runner/api.py:24-75).

``profile(kernels, cache_dir, seed, platform_target, collect_detailed_profile)``
builds and times a set of kernel instances on this MI355X and writes the
standard cache layout (instance sources, results.json, per-kernel
profile_summary.json) under ``cache_dir``; an empty ``cache_dir`` skips all
disk output.  Per-kernel failures never raise: they are returned as
``ProfileResult.hardware_output`` text.  Only environment faults raise (no
GPU, wrong arch, a batch asking for more than one device).
"""

from __future__ import annotations

import logging
import os
import time

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
            (``profile.json`` in the kernel's cache folder).
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
    elapsed_s = time.monotonic() - t0
    logger.info("Profile complete: %d results in %.1fs", len(results), elapsed_s)
    if cache_dir:
        write_compiler_logs(cache_dir, compiler_logs)
        write_results_json(cache_dir, len(kernels), results, elapsed_s)
        logger.info("Cache saved to %s", cache_dir)
    return ProfileOutput(results=results, compiler_logs=compiler_logs, elapsed_s=elapsed_s, cache_dir=cache_dir)
