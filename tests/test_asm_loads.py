"""The asynchronous register loads of the fused kernels stay untouched until
their wait (see tests/asm_loads.py), in the gfx950 code hipcc emits for the
shipped instance files; and the pipelined kernels compile to straight-line
kernel code (no outlined calls, no scratch spills).  Needs hipcc, not a GPU."""

from __future__ import annotations

import shutil
import subprocess
import sys
from pathlib import Path

import pytest

from asm_loads import check_kernel, kernels

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "nki-autotune_amd" / "csrc"
sys.path.insert(0, str(ROOT / "nki-autotune_amd"))


def _hipcc():
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    pytest.skip("hipcc not available")


@pytest.fixture(scope="module")
def asm_of(tmp_path_factory):
    """unit -> gfx950 assembly text, compiled once per module."""
    import build_lib

    cache: dict[str, str] = {}
    tmp = tmp_path_factory.mktemp("asm")

    def get(unit: str) -> str:
        if unit not in cache:
            out = tmp / (unit + ".s")
            flags = [f for f in build_lib.HIPCC_FLAGS if f != "-fPIC"]
            subprocess.run([_hipcc(), *flags, f"-I{build_lib.INCLUDE}", "--cuda-device-only", "-S",
                            str(CSRC / unit), "-o", str(out)], check=True, capture_output=True)
            cache[unit] = out.read_text()
        return cache[unit]

    return get


@pytest.mark.parametrize("unit", ["rms_bf16_xreg.hip"])
def test_async_register_loads_untouched_until_waited(unit, asm_of):
    ks = kernels(asm_of(unit))
    assert ks
    total = 0
    for name, lines in ks.items():
        n, bad = check_kernel(lines)
        total += n
        assert not bad, (name, bad[:3])
    assert total > 0


@pytest.mark.parametrize("unit", ["mm_bf16_pipe.hip", "mm_bf16_kw.hip", "mm_bf16_lhs.hip", "mm_bf16_reg.hip",
                                  "rms_bf16_xreg.hip", "rms_bf16_2pass.hip"])
def test_kernels_straight_line(unit, asm_of):
    """The unrolled tile lambdas are inlined: a device-function call would
    pass buffer descriptors in VGPRs and read captures through flat loads."""
    ks = kernels(asm_of(unit))
    assert ks
    for name, lines in ks.items():
        bad = [ln for ln in lines if ln.strip().startswith(("s_swappc", "s_setpc", "flat_load", "scratch_"))]
        assert not bad, (name, bad[:3])
