"""In-process compile + benchmark pipeline on one GPU.

Control flow of reference autotune/src/autotune/runner/driver.py:126-165:
reject a batch that mixes device counts, make a scratch work dir, detect the
device, generate seeded inputs per job, submit every build to a pool, and
benchmark each job sequentially on the one device as its build completes
(``as_completed``).  Differences: builds are hipcc child processes (or a
lookup in the prebuilt library), so the pool is a thread pool; and inputs
are generated once per distinct (specs, distributions, seed) and shared by
every job that asks for them -- a sweep of 72 configs at 8192^3 then draws
its 2 x 64 Mi values once instead of 72 times (same values, since every job
of the reference draws from the same seed).
"""

from __future__ import annotations

import json
import logging
import os
import shutil
import time
from concurrent.futures import ThreadPoolExecutor, as_completed
from pathlib import Path
from typing import Any

from autotune.runner.benchmark import benchmark_one, generate_tensors, upload
from autotune.runner.compile import canonical_name, compile_one, default_work_dir, parse_source, problem_shape
from autotune.runner.detect import detect_gpus
from autotune.runner.golden import expected_output
from autotune.runner.types import CompileResult, KernelJob, OutputSpec, ProfileResult, compile_failure_result

logger = logging.getLogger(__name__)

_OUTPUT_TENSOR_NAME = "out"


def _inputs_key(job: KernelJob, seed: int) -> str:
    return json.dumps([list(map(list, [(list(s), d) for s, d in job.input_specs.values()])),
                       list(job.input_specs), repr(sorted((job.input_dists or {}).items())), seed])


def warm_clock(device, seconds: float) -> None:
    """Keep the GPU busy for ``seconds`` with bf16 GEMMs before timing.

    Under sustained load MI355X's engine clock rises over a few hundred
    milliseconds; a kernel timed right after an idle gap (start-up, a hipcc
    build) runs at the lower clock, 10-15 % slower on compute-bound shapes,
    which would bias the sweep towards whichever configs are timed later."""
    import torch

    a = torch.empty((4096, 4096), dtype=torch.bfloat16, device=device).uniform_(-1, 1)
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(20):
            torch.matmul(a, a)
        torch.cuda.synchronize(device)


def run_pipeline(
    kernels: dict[str, KernelJob],
    seed: int,
    collect_compiler_logs: bool,
    collect_detailed_profile: bool,
    warmup: int = 10,
    reps: int = 50,
    flush_bytes: int = 0,
    allow_jit: bool = True,
    work_dir: str | None = None,
    clock_warmup_s: float = 0.5,
    check_numerics: bool = True,
) -> tuple[list[ProfileResult], dict[str, str]]:
    """Build + time every job on GPU 0; return (results, compiler_logs).

    Before the first timing, and before any timing that follows more than
    0.2 s without GPU work (a just-in-time build), the GPU is kept busy for
    ``clock_warmup_s`` seconds (:func:`warm_clock`).  With
    ``check_numerics`` every timed job's output is checked against a float64
    evaluation of its inputs (:mod:`autotune.runner.golden`), computed once
    per input set; a job that fails becomes a failure row."""
    import torch

    if not kernels:
        return [], {}
    lncs = {int(job.lnc) for job in kernels.values()}
    if lncs != {1}:
        raise RuntimeError(f"lnc values {sorted(lncs)} requested; every profile run uses exactly one GPU (lnc=1)")
    first = next(iter(kernels.values()))
    work = Path(work_dir or default_work_dir(first.func_name))
    shutil.rmtree(work, ignore_errors=True)
    work.mkdir(parents=True)

    n_dev, arch, cus = detect_gpus()
    logger.info("Driver ready: %d kernels, %d CPU, %d GPU (%s, %d CUs)", len(kernels), os.cpu_count() or 1, n_dev,
                arch, cus)
    device = torch.device("cuda:0")

    dev_inputs: dict[str, dict[str, Any]] = {}
    goldens: dict[str, tuple] = {}
    meta: dict[str, tuple] = {}
    for kname, job in kernels.items():
        key = _inputs_key(job, seed)
        if key not in dev_inputs:
            dev_inputs[key] = upload(generate_tensors(job.input_specs, seed, job.input_dists), job.input_specs, device)
            if check_numerics:
                goldens[key] = expected_output(job.func_name, dev_inputs[key])
        meta[kname] = (key, problem_shape(job.func_name, job.input_specs))

    workers = min(max((os.cpu_count() or 2) - 1, 1), len(kernels), 16)
    compile_results: list[CompileResult] = []
    compile_errors: list[ProfileResult] = []
    hw_results: list[ProfileResult] = []
    last_gpu = None
    with ThreadPoolExecutor(max_workers=workers) as pool:
        futures = [
            pool.submit(compile_one, kname, job.source, job.func_name, job.input_specs, str(work), job.hipcc_args,
                        allow_jit)
            for kname, job in kernels.items()
        ]
        for f in as_completed(futures):
            cr = f.result()
            compile_results.append(cr)
            if cr.error:
                compile_errors.append(compile_failure_result(cr))
                continue
            job = kernels[cr.kernel_name]
            key, (M, N, K) = meta[cr.kernel_name]
            _fam, cfg = parse_source(job.source)
            out_dtype = next(iter(job.input_specs.values()))[1]
            out = OutputSpec(_OUTPUT_TENSOR_NAME, tuple(job.output_shape), out_dtype)
            if tuple(job.output_shape) != (M, N):
                hw_results.append(ProfileResult(cr.kernel_name, f"output_shape {tuple(job.output_shape)} does not "
                                                f"match the inputs' [M, N] = [{M}, {N}]"))
                continue
            if clock_warmup_s > 0 and (last_gpu is None or time.perf_counter() - last_gpu > 0.2):
                warm_clock(device, clock_warmup_s)
            hw_results.append(benchmark_one(cr.kernel_name, cr.library_path, canonical_name(job.func_name), cfg,
                                            dev_inputs[key], out, M, N, K, warmup, reps, flush_bytes,
                                            collect_detailed_profile, goldens.get(key)))
            last_gpu = time.perf_counter()
    logs = {}
    if collect_compiler_logs:
        for cr in compile_results:
            text = cr.compile_log
            ignored = kernels[cr.kernel_name].ignored_args
            if ignored:
                note = "ignored (Neuron compiler options with no hipcc counterpart): " + " ".join(ignored)
                text = f"{text}\n{note}" if text else note
            if text:
                logs[cr.kernel_name] = text
    return compile_errors + hw_results, logs
