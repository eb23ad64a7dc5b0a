"""Hardware benchmarking of one kernel instance on the GPU.

Replaces reference autotune/src/autotune/runner/benchmark.py, which runs a
NEFF once under ``spike.run(save_trace=True)`` and reads ``neuron-profile``'s
summary JSON (:58-87, :116-153).  Here the kernel is launched through the C
ABI of the library that holds its instance, timed with HIP events on the
launch stream (warm-up launches, then ``reps`` timed launches, median
reported), and the summary carries the same utilisation fields the
reference's profiler reports (``total_time``, ``mfu_estimated_percent``,
``mbu_estimated_percent``, ``mfu_max_achievable_estimated_percent``; all
fractions, as in neuron-profile) computed from the algorithmic work:
FLOPs = 2*M*N*K, compulsory bytes = (M*K + K*N + M*N) * element size
(+ K * 2 for gamma).
"""

from __future__ import annotations

import ctypes
import statistics
from typing import Any

import numpy as np

from autotune.runner.types import OutputSpec, ProfileResult, capture_error, element_size

# MI355X published dense peaks (per GPU).
PEAK_TFLOPS = {"bfloat16": 2500.0, "float16": 2500.0, "float32": 157.3}
PEAK_HBM_GBPS = 8000.0


def generate_tensors(input_specs: dict, seed: int, dists: dict | None = None) -> dict[str, np.ndarray]:
    """Seeded host tensors in signature order (reference benchmark.py:156-169).

    One ``np.random.default_rng(seed)`` stream; each input draws in spec
    order.  Default is ``standard_normal`` (the reference's only
    distribution); ``dists`` selects "uniform" (U(-1,1)), ("normal", sigma)
    or "gamma" (1 + 0.1 N(0,1)) per input.  Returned as float32; the dtype
    cast (RNE for bfloat16) happens on upload.
    """
    rng = np.random.default_rng(seed)
    out: dict[str, np.ndarray] = {}
    for name, (shape, _dtype) in input_specs.items():
        dist = (dists or {}).get(name, "normal")
        shape = tuple(int(s) for s in shape)
        if dist == "normal":
            a = rng.standard_normal(shape).astype(np.float32)  # float64 draw, then cast (benchmark.py:168)
        elif dist == "uniform":
            a = rng.uniform(-1.0, 1.0, shape).astype(np.float32)
        elif dist == "gamma":
            a = (1.0 + 0.1 * rng.standard_normal(shape)).astype(np.float32)
        elif isinstance(dist, (tuple, list)) and dist[0] == "normal":
            a = (float(dist[1]) * rng.standard_normal(shape)).astype(np.float32)
        else:
            raise ValueError(f"unknown distribution {dist!r} for input {name!r}")
        out[name] = a
    return out


def upload(host: dict[str, np.ndarray], input_specs: dict, device) -> dict[str, Any]:
    """Host float32 tensors -> device tensors of the spec dtypes (torch casts bf16 RNE)."""
    import torch

    from autotune.runner.types import resolve_dtype

    dev = {}
    for name, (_shape, dtype) in input_specs.items():
        dev[name] = torch.from_numpy(host[name]).to(device).to(resolve_dtype(dtype)).contiguous()
    return dev


def work_of(func_name: str, M: int, N: int, K: int, dtype: str, has_gamma: bool = False) -> tuple[float, float]:
    """(algorithmic FLOPs, compulsory HBM bytes) of one launch."""
    e = element_size(dtype)
    flops = 2.0 * M * N * K
    nbytes = float((M * K + K * N + M * N) * e + (K * 2 if has_gamma else 0))
    return flops, nbytes


def utilisation(flops: float, nbytes: float, seconds: float, dtype: str) -> dict[str, float]:
    """Fractions of the MFMA and HBM peaks, and the roofline ceiling."""
    peak_f = PEAK_TFLOPS.get(dtype, PEAK_TFLOPS["bfloat16"]) * 1e12
    peak_b = PEAK_HBM_GBPS * 1e9
    ai = flops / nbytes if nbytes else float("inf")
    return {
        "tflops": flops / seconds / 1e12,
        "hbm_gbps": nbytes / seconds / 1e9,
        "mfu_estimated_percent": flops / seconds / peak_f,
        "mbu_estimated_percent": nbytes / seconds / peak_b,
        "mfu_max_achievable_estimated_percent": min(1.0, ai * peak_b / peak_f),
        "peak_tflops": peak_f / 1e12,
        "peak_hbm_gbps": PEAK_HBM_GBPS,
    }


class Launcher:
    """Bound launch of one kernel instance through a library's C ABI."""

    def __init__(self, library, func_name: str, cfg, inputs: dict[str, Any], out, M: int, N: int, K: int,
                 eps: float = 1e-6) -> None:
        import torch

        from autotune.runner.compile import canonical_name
        from kernel_library import _lib

        self._lib = _lib
        self.library = library
        self.cfg_c = cfg.to_c()
        self.fam = canonical_name(func_name)
        self.out = out
        self.M, self.N, self.K = M, N, K
        vals = list(inputs.values())
        self.stream = torch.cuda.current_stream(out.device).cuda_stream
        if self.fam == "rmsnorm_matmul":
            x, w = inputs.get("lhs", vals[0]), inputs.get("rhs", vals[-1])
            g = inputs.get("gamma")
            self.fn = library.mi_rmsnorm_matmul_bf16
            self.args = (x.data_ptr(), g.data_ptr() if g is not None else None, w.data_ptr(), out.data_ptr(), M, N,
                         K, float(eps), ctypes.byref(self.cfg_c), self.stream)
        elif self.fam == "matmul_lhs_rhs":
            a, b = vals[0], vals[1]
            self.fn = library.mi_matmul_lhs_rhs_bf16
            self.args = (a.data_ptr(), b.data_ptr(), out.data_ptr(), M, N, K, ctypes.byref(self.cfg_c), self.stream)
        else:
            a, b = vals[0], vals[1]
            fp32 = a.dtype == torch.float32
            self.fn = library.mi_matmul_lhsT_rhs_f32 if fp32 else library.mi_matmul_lhsT_rhs_bf16
            self.args = (a.data_ptr(), b.data_ptr(), out.data_ptr(), M, N, K, ctypes.byref(self.cfg_c), self.stream)

    def __call__(self) -> None:
        rc = self.fn(*self.args)
        if rc != 0:
            msg = self.library.mi_last_error()
            raise self._lib.KernelLibraryError(rc, msg.decode() if msg else self._lib.CODE_NAMES.get(rc, "HIP error"))


def time_launches(launch, warmup: int, reps: int, flush=None) -> list[float]:
    """Per-launch seconds from HIP events recorded on the current stream around each launch."""
    import torch

    for _ in range(warmup):
        launch()
    torch.cuda.synchronize()
    events = []
    for _ in range(reps):
        if flush is not None:
            flush()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        launch()
        end.record()
        events.append((start, end))
    torch.cuda.synchronize()
    return [s.elapsed_time(e) * 1e-3 for s, e in events]


def benchmark_one(kernel_name: str, library_path: str, func_name: str, cfg, inputs: dict[str, Any],
                  out_spec: OutputSpec, M: int, N: int, K: int, warmup: int = 10, reps: int = 50,
                  flush_bytes: int = 0, collect_detailed_profile: bool = False,
                  golden: tuple | None = None) -> ProfileResult:
    """Time one instance; errors become ``hardware_output`` text (reference benchmark.py:116-153).

    ``golden`` = (expected float64 output, absolute floor) from
    :mod:`autotune.runner.golden`: the output of the last timed launch must
    pass that check, or the instance is reported as a numerics failure
    instead of a success."""
    import torch

    from kernel_library import _lib

    summary = detailed = neff_b64 = None
    dtype = out_spec.dtype
    hardware_output = f"{list(out_spec.shape)} {dtype}"
    try:
        library = _lib.load(library_path)
        dev = next(iter(inputs.values())).device
        # NaN-filled, so that an output element the candidate never writes
        # fails the numerics check instead of passing on a value an earlier
        # candidate left in the same (recycled) allocation.
        out = torch.full(tuple(out_spec.shape), float("nan"), dtype=_torch_dtype(dtype), device=dev)
        launch = Launcher(library, func_name, cfg, inputs, out, M, N, K)
        flush = None
        if flush_bytes:
            scratch = torch.empty(flush_bytes // 4, dtype=torch.float32, device=dev)
            flush = scratch.zero_
        times = time_launches(launch, warmup, reps, flush)
        numerics = None
        if golden is not None:
            from autotune.runner import golden as gold

            numerics = gold.compare(out, golden[0], golden[1], gold.rtol_for(dtype))
            if not numerics["pass"]:
                return ProfileResult(kernel_name, gold.failure_text(numerics), None,
                                     {"numerics": numerics, "times_s": times} if collect_detailed_profile else None)
        med = statistics.median(times)
        flops, nbytes = work_of(func_name, M, N, K, dtype, has_gamma="gamma" in inputs)
        summary = {
            "total_time": med,
            "min_time": min(times),
            "mean_time": statistics.fmean(times),
            "warmup": warmup,
            "reps": reps,
            "flops": flops,
            "bytes": nbytes,
            "config": cfg.asdict(),
            "library": library_path,
            **utilisation(flops, nbytes, med, dtype),
        }
        if numerics is not None:
            summary["numerics"] = numerics
        if collect_detailed_profile:
            detailed = {"times_s": times, "l2_flush_bytes": flush_bytes}
            neff_b64 = code_object_b64(library_path, func_name, cfg)
    except Exception as exc:
        hardware_output = capture_error(exc)
        summary = detailed = neff_b64 = None
    return ProfileResult(kernel_name, hardware_output, summary, detailed, neff_b64)


def code_object_b64(library_path: str, func_name: str, cfg) -> str | None:
    """Base64 of the gfx950 code object holding the instance (the NEFF's counterpart), or None."""
    import base64

    from autotune.runner.codeobj import code_object_of
    from autotune.runner.compile import canonical_name

    co = code_object_of(library_path, canonical_name(func_name), cfg)
    return None if co is None else base64.b64encode(co).decode("ascii")


def _torch_dtype(name: str):
    from autotune.runner.types import resolve_dtype

    return resolve_dtype(name)
