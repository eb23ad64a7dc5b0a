"""Shared types of the MI355X autotune runner.

Mirrors reference autotune/src/autotune/runner/types.py: the same
``KernelJob`` / ``CompileResult`` / ``ProfileResult`` / ``OutputSpec``
records and helpers, with the Neuron-specific fields re-read for HIP:

* ``KernelJob.source`` is the HIP source text of one kernel instance
  (``autotune.runner.compile.render_source``): a translation unit that
  instantiates the kernel template for one tile config.  The config is
  also carried in a machine-readable header line of that text, so a job is
  fully described by its source, as in the reference (types.py:32-58).
* ``hipcc_args`` replaces ``neuronx_cc_args``; ``lnc`` (logical device
  count) must be 1 -- every run uses one GPU.
* ``ProfileResult.profiler_summary`` is the hipEvent timing summary written
  by ``benchmark.benchmark_one`` (``total_time`` in seconds plus the
  utilisation fractions), in place of the ``neuron-profile`` summary JSON.
"""

from __future__ import annotations

import traceback
from typing import Any, NamedTuple

_TORCH_DTYPES = {
    "bfloat16": "bfloat16",
    "bf16": "bfloat16",
    "float32": "float32",
    "fp32": "float32",
    "float16": "float16",
    "fp16": "float16",
}


def resolve_dtype(name: str):
    """torch dtype of a dtype string ("bfloat16", "float32", "float16").

    The reference resolves bfloat16 through ml_dtypes
    (reference autotune/src/autotune/runner/types.py:17-30); here device
    tensors are torch tensors, so the name maps to a torch dtype.
    """
    import torch

    try:
        return getattr(torch, _TORCH_DTYPES[name])
    except KeyError as exc:
        raise ValueError(f"unsupported dtype {name!r}; known: {sorted(_TORCH_DTYPES)}") from exc


def element_size(name: str) -> int:
    """Bytes per element of a dtype string."""
    return 4 if _TORCH_DTYPES.get(name) == "float32" else 2


class KernelJob(NamedTuple):
    """Per-kernel configuration for profiling (reference types.py:32-58).

    Attributes:
        source: HIP source text of the kernel instance (one tile config).
        func_name: Kernel family: ``matmul_lhsT_rhs``, ``matmul_lhsT_rhs_f32``
            or ``rmsnorm_matmul`` (reference names ``matmul_lhsT_rhs_nkigym``
            and ``rmsnorm_matmul_online`` are accepted as aliases).
        output_shape: Shape of the kernel's output tensor.
        input_specs: Map of param name to (shape, dtype_str), in signature order.
        hipcc_args: Extra hipcc flags for a just-in-time build of ``source``.
        lnc: Logical device count; only 1 is supported (one GPU).
        input_dists: Optional per-input distribution ("normal", "uniform",
            ("normal", sigma), "gamma"); default standard normal, as in the
            reference's ``generate_tensors`` (benchmark.py:156-169).
    """

    source: str
    func_name: str
    output_shape: tuple[int, ...]
    input_specs: dict[str, tuple[tuple[int, ...], str]]
    hipcc_args: tuple[str, ...] = ()
    lnc: int = 1
    input_dists: dict[str, Any] | None = None


class CompileResult(NamedTuple):
    """Result of "compiling" one kernel instance (reference types.py:61-67).

    ``library_path`` is the shared library holding the instance: the
    prebuilt ``libmi_kernels.so`` when the config is one of its compiled
    instances, or a per-config library built from ``source`` by hipcc.
    ``error`` is empty on success, else the full message / traceback.
    """

    kernel_name: str
    source_path: str
    library_path: str
    error: str
    compile_log: str = ""


class ProfileResult(NamedTuple):
    """Benchmark result for a single kernel (reference types.py:70-98).

    ``hardware_output`` is ``"[M, N] bfloat16"`` on success (so success is
    ``hardware_output.startswith("[")``, as in the reference) or the error
    text.  ``profiler_summary`` holds the hipEvent timing summary;
    ``profile_detailed`` the optional per-rep timings and rocprofv3 kernel-trace row.
    """

    kernel_name: str
    hardware_output: str
    profiler_summary: dict | None = None
    profile_detailed: dict | None = None


class OutputSpec(NamedTuple):
    """Output tensor specification (reference types.py:101-106)."""

    name: str
    shape: tuple[int, ...]
    dtype: str


def capture_error(exc: BaseException) -> str:
    """Full traceback of ``exc`` as a string (reference types.py:109-111)."""
    return "".join(traceback.format_exception(type(exc), exc, exc.__traceback__))


def make_failure(kernel_name: str, hardware_output: str) -> ProfileResult:
    """A failed ProfileResult with no profiler summary."""
    return ProfileResult(kernel_name=kernel_name, hardware_output=hardware_output)


def compile_failure_result(cr: CompileResult) -> ProfileResult:
    """Convert a failed CompileResult into a ProfileResult."""
    return make_failure(cr.kernel_name, cr.error)


def profiler_percent(summary: dict | None, field: str) -> float | None:
    """Fractional utilisation field of a summary, scaled to percent.

    Same contract as the reference (types.py:129-143): fields are fractions
    in [0, 1]; a missing field or a negative sentinel gives ``None``.
    """
    result: float | None = None
    if summary is not None:
        value = summary.get(field)
        if value is not None:
            scaled = float(value) * 100.0
            if scaled >= 0:
                result = scaled
    return result
