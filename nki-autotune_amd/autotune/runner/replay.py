"""Re-run one profiled kernel instance in a fresh process (for tracing).

``python -m autotune.runner.replay <replay.json>`` regenerates the job's
seeded inputs, loads its library and times ``reps`` launches after
``warmup``, exactly as :func:`autotune.runner.benchmark.benchmark_one` did,
then prints one JSON line with the median.  :mod:`autotune.runner.trace`
runs it under rocprofv3 to capture the kernel trace of a detailed profile.
The replay file is written by :func:`autotune.runner.trace.write_replay_job`.
"""

from __future__ import annotations

import json
import statistics
import sys


def run(job: dict) -> dict:
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
    flush = None
    if job.get("flush_bytes"):
        scratch = torch.empty(int(job["flush_bytes"]) // 4, dtype=torch.float32, device=device)
        flush = scratch.zero_
    times = time_launches(launch, int(job["warmup"]), int(job["reps"]), flush)
    return {"kernel": job["kernel_name"], "median_s": statistics.median(times), "reps": len(times)}


def main(argv: list[str] | None = None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    if len(argv) != 1:
        print("usage: python -m autotune.runner.replay <replay.json>", file=sys.stderr)
        return 2
    with open(argv[0]) as f:
        job = json.load(f)
    print(json.dumps(run(job)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
