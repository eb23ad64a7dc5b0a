"""The asynchronous register loads of the fused kernels stay untouched until
their wait (see tests/asm_loads.py), in the gfx950 code hipcc emits for the
shipped instance files; and the pipelined kernels compile to straight-line
kernel code (no outlined calls, no scratch spills).  Needs hipcc, not a GPU."""

from __future__ import annotations

import os
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


UNITS = ("mm_bf16_pipe.hip", "mm_bf16_kw.hip", "mm_bf16_lhs.hip", "mm_bf16_reg.hip", "rms_bf16_xreg.hip",
         "rms_bf16_2pass.hip", "rms_bf16_sq.hip")


@pytest.fixture(scope="module")
def asm_of(tmp_path_factory):
    """unit -> gfx950 assembly text, compiled once per module.

    In a run without xdist workers every unit's compile starts at the first
    request, all at once, so the module waits for the slowest unit rather
    than for the sum of them; under xdist each worker compiles only what its
    own tests ask for."""
    import build_lib

    cache: dict[str, str] = {}
    running: dict[str, tuple[subprocess.Popen, object]] = {}
    tmp = tmp_path_factory.mktemp("asm")
    flags = [f for f in build_lib.HIPCC_FLAGS if f != "-fPIC"]

    def start(unit: str) -> None:
        if unit in cache or unit in running:
            return
        out = tmp / (unit + ".s")
        proc = subprocess.Popen([_hipcc(), *flags, f"-I{build_lib.INCLUDE}", "--cuda-device-only", "-S",
                                 str(CSRC / unit), "-o", str(out)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
        running[unit] = (proc, out)

    def get(unit: str) -> str:
        if unit not in cache:
            if not running and not os.environ.get("PYTEST_XDIST_WORKER"):
                for u in UNITS:
                    start(u)
            start(unit)
            proc, out = running.pop(unit)
            log, _ = proc.communicate()
            if proc.returncode != 0:
                raise subprocess.CalledProcessError(proc.returncode, proc.args, log)
            cache[unit] = out.read_text()
        return cache[unit]

    yield get
    for proc, _ in running.values():
        proc.kill()
        proc.wait()


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


@pytest.mark.parametrize("unit", UNITS)
def test_kernels_straight_line(unit, asm_of):
    """The unrolled tile lambdas are inlined: a device-function call would
    pass buffer descriptors in VGPRs and read captures through flat loads."""
    ks = kernels(asm_of(unit))
    assert ks
    for name, lines in ks.items():
        bad = [ln for ln in lines if ln.strip().startswith(("s_swappc", "s_setpc", "flat_load", "scratch_"))]
        assert not bad, (name, bad[:3])


def test_row_square_sums_read_every_pair_of_the_fragment(asm_of):
    """The fused kernels without gamma (rmsnorm_matmul variants 14 and 16)
    sum the squares of each A fragment's four bf16 pairs with four dependent
    v_dot2c_f32_bf16 into one accumulator.  Each such chain must read four
    different registers (the fragment's dwords): a bit-cast of the
    fragment's dword d to bf16x2 was compiled as dword 0 for every d."""
    import re

    ks = kernels(asm_of("rms_bf16_sq.hip"))
    assert ks
    dot2 = re.compile(r"^\s*v_dot2c_f32_bf16(?:_e32)?\s+v(\d+),\s*v(\d+),\s*v(\d+)")
    ks = {name: lines for name, lines in ks.items()
          if "rmsnorm_mm_bf16_sq_kernel" in name or "rmsnorm_mm_bf16_sq_pair_kernel" in name}
    assert any("sq_pair_kernel" in n for n in ks) and any("sq_kernel" in n and "pair" not in n for n in ks)
    for name, lines in ks.items():
        per_acc: dict[int, list[int]] = {}
        for ln in lines:
            m = dot2.match(ln)
            if m:
                assert m.group(2) == m.group(3), (name, ln)   # a square: the pair with itself
                per_acc.setdefault(int(m.group(1)), []).append(int(m.group(2)))
        assert per_acc, name
        for acc, srcs in per_acc.items():
            assert len(srcs) % 4 == 0, (name, acc, len(srcs))
            for i in range(0, len(srcs), 4):
                assert len(set(srcs[i:i + 4])) == 4, (name, acc, srcs[i:i + 4])
