"""Re-run one profiled kernel instance in a fresh process (for tracing).

``python -m autotune.runner.replay <replay.json> [--warmup W --reps R]
[--calibrate-copy-mib C]`` regenerates the job's seeded inputs, loads its
library and times ``reps`` launches after ``warmup`` (the job's schedule
unless overridden), exactly as :func:`autotune.runner.benchmark.benchmark_one`
did, then prints one JSON line with the median.  With ``--calibrate-copy-mib``
it first copies C MiB device to device: the dispatch of known traffic that
scales the byte counters of a counter pass.  :mod:`autotune.runner.trace`
runs it under rocprofv3 for the kernel trace and the counters of a detailed
profile.  The replay file is written by
:func:`autotune.runner.trace.write_replay_job`.
"""

from __future__ import annotations

import json
import statistics
import sys


def run(job: dict, warmup: int | None = None, reps: int | None = None, calibrate_copy_mib: int = 0) -> dict:
    import torch

    from autotune.runner.benchmark import Launcher, generate_tensors, time_launches, upload
    from kernel_library import _lib
    from kernel_library.config import TileConfig

    specs = {k: (tuple(s), d) for k, (s, d) in job["input_specs"].items()}
    dists = job.get("input_dists") or None
    device = torch.device("cuda:0")
    inputs = upload(generate_tensors(specs, int(job["seed"]), dists), specs, device)
    M, N, K = job["shape"]
    out_dtype = next(iter(specs.values()))[1]
    out = torch.empty((M, N), dtype=torch.float32 if out_dtype == "float32" else torch.bfloat16, device=device)
    launch = Launcher(_lib.load(job["library_path"]), job["func_name"], TileConfig(**job["config"]), inputs, out,
                      M, N, K)
    if calibrate_copy_mib > 0:
        n = calibrate_copy_mib << 18  # fp32 elements
        src = torch.ones(n, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    flush = None
    if job.get("flush_bytes"):
        scratch = torch.empty(int(job["flush_bytes"]) // 4, dtype=torch.float32, device=device)
        flush = scratch.zero_
    w = int(job["warmup"]) if warmup is None else warmup
    r = int(job["reps"]) if reps is None else reps
    times = time_launches(launch, w, r, flush)
    return {"kernel": job["kernel_name"], "median_s": statistics.median(times), "warmup": w, "reps": len(times)}


def main(argv: list[str] | None = None) -> int:
    import argparse

    ap = argparse.ArgumentParser(prog="python -m autotune.runner.replay")
    ap.add_argument("replay_json")
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--reps", type=int, default=None)
    ap.add_argument("--calibrate-copy-mib", type=int, default=0)
    args = ap.parse_args(sys.argv[1:] if argv is None else argv)
    with open(args.replay_json) as f:
        job = json.load(f)
    print(json.dumps(run(job, args.warmup, args.reps, args.calibrate_copy_mib)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
