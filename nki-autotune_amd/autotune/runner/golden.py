"""Numerics gate of every autotune candidate.

The reference checks every candidate kernel before it is profiled: it runs
the kernel source in its fp32 CPU simulator and compares the result with
``lhs_T.T @ rhs`` (examples/tune_matmul_lhsT_rhs.py:156-172, 189-218;
examples/profile_hand_90mfu.py:45-56), so only correct kernels can be
selected.  Here candidates are tile configs of hand-written HIP kernels, so
the check is made on the GPU output itself: after a candidate is timed, its
output on the profiling inputs is compared with a float64 evaluation of the
same function on the same (bf16-rounded) inputs, computed once per input
set.  A candidate that fails becomes a failure row ("numerics check
failed: ..."), never a selectable success.

Pass criterion: the reference's ``np.allclose`` form (kernel_transforms.py:
592-596) with the benchmark's rtol = 1e-2.  The absolute floor is the
reference's 5e-3 for the matmuls (fp32 inputs: 5e-3 relative too, as in
test/codegen/test_render.py:49); for rmsnorm_matmul it is 1e-2 * RMS(out),
since rounding the normalised rows to bf16 -- which the reference kernel
does as well (kernel_hand_online.py:139-149) -- leaves ~1.5e-3 * RMS(out)
of absolute error on every output.  ``max_rel = max |a - e| / (|e| + atol)``
is reported beside it, as the reference prints it.
"""

from __future__ import annotations

from typing import Any

RTOL = 1e-2
ATOL = 5e-3
F32_RTOL = 5e-3
RMS_ATOL_FRAC = 1e-2
EPS = 1e-6


def expected_output(func_name: str, inputs: dict[str, Any], eps: float = EPS):
    """float64 torch evaluation of the kernel family on the device inputs, and its absolute floor."""
    from autotune.runner.compile import canonical_name

    fam = canonical_name(func_name)
    vals = list(inputs.values())
    if fam == "rmsnorm_matmul":
        x = inputs.get("lhs", vals[0]).double()
        w = inputs.get("rhs", vals[-1]).double()
        y = x * (x * x).mean(dim=1, keepdim=True).add(eps).rsqrt()
        g = inputs.get("gamma")
        if g is not None:
            y = y * g.double()[None, :]
        exp = y @ w
        return exp, RMS_ATOL_FRAC * float(exp.square().mean().sqrt())
    a, b = vals[0].double(), vals[1].double()
    exp = a @ b if fam == "matmul_lhs_rhs" else a.t() @ b
    return exp, ATOL


def compare(out, expected, atol: float, rtol: float = RTOL) -> dict:
    """The gate's report: allclose(atol, rtol), no non-finite values, max_abs and max_rel."""
    import torch

    o = out.double()
    diff = (o - expected).abs()
    finite = torch.isfinite(o)
    rep = {
        "max_abs": float(diff.max()) if diff.numel() else 0.0,
        "max_rel": float((diff / (expected.abs() + atol)).max()) if diff.numel() else 0.0,
        "atol": atol,
        "rtol": rtol,
        "nonfinite": int((~finite).sum()),
        "allclose": bool((diff <= atol + rtol * expected.abs()).all()),
    }
    rep["pass"] = rep["allclose"] and rep["nonfinite"] == 0
    return rep


def rtol_for(dtype: str) -> float:
    return F32_RTOL if dtype == "float32" else RTOL


def failure_text(rep: dict) -> str:
    return (f"numerics check failed: max_abs {rep['max_abs']:.4g}, max_rel {rep['max_rel']:.4g} "
            f"(atol {rep['atol']:.3g}, rtol {rep['rtol']:.3g}), {rep['nonfinite']} non-finite values")
