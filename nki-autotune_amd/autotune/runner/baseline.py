"""Vendor-library baseline row (reference autotune/src/autotune/runner/baseline.py:75-144).

The reference profiles the compiler's own lowering of ``lhs_T.T @ rhs``
(numpy -> nkipy -> neuronx-cc, :117) and prints it beside the tuned kernel
(examples/tune_matmul_lhsT_rhs.py:222-242).  The MI355X analogue is what
PyTorch-ROCm runs for the same expression:

* matmul_lhsT_rhs: ``torch.matmul(lhs_T.t(), rhs)`` (hipBLASLt, transposed A);
* matmul_lhs_rhs: ``torch.matmul(lhs, rhs)`` (hipBLASLt, NN);
* rmsnorm_matmul: the unfused composition
  ``((x * rsqrt(mean(x^2) + eps)) * gamma).to(bf16) @ W`` -- torch's
  elementwise kernels, then hipBLASLt.

It is timed with the same hipEvent schedule as the kernels and reported as a
``ProfileResult`` with the same summary fields, so it sits in the same
results table and results.json (``ProfileOutput.baseline``).  Its output is
checked against the same float64 golden as every kernel candidate.  It is a
comparison row only: nothing in the kernel_library path calls it.
"""

from __future__ import annotations

import statistics

from autotune.runner.benchmark import generate_tensors, time_launches, upload, utilisation, work_of
from autotune.runner.types import ProfileResult, capture_error

BASELINE_SEED = 42
LIBRARY = {"matmul_lhsT_rhs": "torch.matmul (hipBLASLt)", "matmul_lhs_rhs": "torch.matmul (hipBLASLt)",
           "rmsnorm_matmul": "torch eager rmsnorm, then torch.matmul (hipBLASLt)"}


def profile_torch_baseline(M: int, N: int, K: int, dtype: str = "bfloat16", seed: int = BASELINE_SEED,
                           warmup: int = 10, reps: int = 50, dists: dict | None = None,
                           kernel_name: str = "hipblaslt_baseline", flush_bytes: int = 0,
                           lhs_layout: str = "KM", func_name: str | None = None, out=None,
                           eps: float = 1e-6) -> ProfileResult:
    """Time the vendor path of one kernel family at (M, N, K) on seeded inputs.

    ``func_name`` picks the family (default: ``lhs_layout`` "KM" is
    matmul_lhsT_rhs, "MK" matmul_lhs_rhs).  ``flush_bytes`` > 0 overwrites a
    buffer of that size before every timed launch, as the kernel sweep does.
    ``out``, when given, receives the output (a contiguous [M, N] tensor of
    the input dtype on cuda:0).
    """
    import torch

    from autotune.runner import golden
    from autotune.runner.compile import canonical_name
    from autotune.tune import input_specs

    if lhs_layout not in ("KM", "MK"):
        raise ValueError(f"lhs_layout must be 'KM' or 'MK', got {lhs_layout!r}")
    fam = canonical_name(func_name) if func_name else ("matmul_lhsT_rhs" if lhs_layout == "KM" else "matmul_lhs_rhs")
    if fam not in LIBRARY:
        raise ValueError(f"no vendor baseline for {fam!r}")
    specs = input_specs(fam, M, N, K, dtype)
    try:
        dev = upload(generate_tensors(specs, seed, dists), specs, torch.device("cuda:0"))
        if out is None:
            out = torch.empty((M, N), dtype=next(iter(dev.values())).dtype, device="cuda:0")
        if fam == "rmsnorm_matmul":
            x, w, g = dev["lhs"], dev["rhs"], dev.get("gamma")

            def launch():
                xf = x.float()
                y = xf * torch.rsqrt(xf.pow(2).mean(dim=1, keepdim=True) + eps)
                if g is not None:
                    y = y * g.float()
                torch.matmul(y.to(x.dtype), w, out=out)
        else:
            a = dev["lhs_T"].t() if fam == "matmul_lhsT_rhs" else dev["lhs"]
            b = dev["rhs"]

            def launch():
                torch.matmul(a, b, out=out)
        flush = torch.empty(flush_bytes // 4, dtype=torch.float32, device="cuda:0").zero_ if flush_bytes else None
        times = time_launches(launch, warmup, reps, flush)
        med = statistics.median(times)
        exp, atol = golden.expected_output(fam, dev, eps)
        numerics = golden.compare(out, exp, atol, golden.rtol_for(dtype))
        del exp
        flops, nbytes = work_of(fam, M, N, K, dtype, has_gamma="gamma" in dev)
        summary = {"total_time": med, "min_time": min(times), "warmup": warmup, "reps": reps, "flops": flops,
                   "bytes": nbytes, "library": LIBRARY[fam], "flush_bytes": flush_bytes, "numerics": numerics,
                   **utilisation(flops, nbytes, med, dtype)}
        return ProfileResult(kernel_name, f"[{M}, {N}] {dtype}", summary)
    except Exception as exc:
        return ProfileResult(kernel_name, capture_error(exc))
