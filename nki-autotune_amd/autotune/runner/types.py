"""Shared types of the MI355X autotune runner.

Mirrors reference autotune/src/autotune/runner/types.py: the same
``KernelJob`` / ``CompileResult`` / ``ProfileResult`` / ``OutputSpec``
records and helpers, with the Neuron-specific fields re-read for HIP:

* ``KernelJob.source`` is the HIP source text of one kernel instance
  (``autotune.runner.compile.render_source``): a translation unit that
  instantiates the kernel template for one tile config.  The config is
  also carried in a machine-readable header line of that text, so a job is
  fully described by its source, as in the reference (types.py:32-58).
* ``neuronx_cc_args`` keeps its name; its command-line flags go to hipcc
  (``KernelJob.hipcc_args``); ``lnc`` (logical device count) must be 1 --
  every run uses one GPU.
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
        func_name: Kernel family: ``matmul_lhsT_rhs``, ``matmul_lhsT_rhs_f32``,
            ``matmul_lhs_rhs`` or ``rmsnorm_matmul`` (the reference names
            ``matmul_lhsT_rhs_nkigym``, ``matmul_lhs_rhs_nkigym`` and
            ``rmsnorm_matmul_online`` are accepted as aliases).
        output_shape: Shape of the kernel's output tensor.
        input_specs: Map of param name to (shape, dtype_str), in signature order.
        neuronx_cc_args: Extra compiler arguments, under the reference's field
            name.  Entries that are command-line flags (they start with
            ``-``) go to hipcc for a just-in-time build of ``source``; the
            Neuron pipeline options the reference's hand kernels pass (such
            as ``enable-instruction-scheduling=false``) have no hipcc
            counterpart and are listed as ignored in the compile log.
        lnc: Logical device count; only 1 is supported (one GPU).
        input_dists: Optional per-input distribution ("normal", "uniform",
            ("normal", sigma), "gamma"); default standard normal, as in the
            reference's ``generate_tensors`` (benchmark.py:156-169).
    """

    source: str
    func_name: str
    output_shape: tuple[int, ...]
    input_specs: dict[str, tuple[tuple[int, ...], str]]
    neuronx_cc_args: tuple[str, ...] = ()
    lnc: int = 1
    input_dists: dict[str, Any] | None = None

    @property
    def hipcc_args(self) -> tuple[str, ...]:
        """The entries of ``neuronx_cc_args`` that hipcc takes (command-line flags)."""
        return tuple(a for a in self.neuronx_cc_args if a.startswith("-"))

    @property
    def ignored_args(self) -> tuple[str, ...]:
        """Neuron compiler pipeline options with no hipcc counterpart."""
        return tuple(a for a in self.neuronx_cc_args if not a.startswith("-"))


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

    Filled only when the caller asks for a detailed profile, else None (as
    in the reference):

    * ``neff_b64``: the compiled artifact, base64 -- the gfx950 code object
      (ELF) of the translation unit that defines the instance, read from
      the library that holds it (:mod:`autotune.runner.codeobj`; the NEFF's
      counterpart);
    * ``ntff_b64``: the trace, base64 -- the rocprofv3 kernel trace
      (``run_kernel_trace.csv``, one row per dispatch) of the instance's
      replay, taken when the run has a cache dir (the NTFF's counterpart).
    """

    kernel_name: str
    hardware_output: str
    profiler_summary: dict | None = None
    profile_detailed: dict | None = None
    neff_b64: str | None = None
    ntff_b64: str | None = None


class OutputSpec(NamedTuple):
    """Output tensor specification (reference types.py:101-106)."""

    name: str
    shape: tuple[int, ...]
    dtype: str


def capture_error(exc: BaseException) -> str:
    """The formatted traceback of ``exc``: how a per-kernel failure is reported."""
    return "".join(traceback.TracebackException.from_exception(exc).format())


def compile_failure_result(cr: CompileResult) -> ProfileResult:
    """The ProfileResult of a job that never reached the GPU: its build error, no summary."""
    return ProfileResult(kernel_name=cr.kernel_name, hardware_output=cr.error)


def profiler_percent(summary: dict | None, field: str) -> float | None:
    """A utilisation field of a profiler summary (a fraction) in percent.

    None when there is no summary, no such field, or the field holds a
    negative value (the "not measured" sentinel), as callers of the
    reference's helper expect (types.py:129-143).
    """
    value = (summary or {}).get(field)
    if value is None:
        return None
    pct = 100.0 * float(value)
    return pct if pct >= 0.0 else None
