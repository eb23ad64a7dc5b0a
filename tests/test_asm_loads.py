"""The asynchronous register loads of the fused kernels stay untouched until
their wait (see tests/asm_loads.py), in the gfx950 code hipcc emits for the
shipped instance files.  Needs hipcc, not a GPU."""

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


@pytest.mark.parametrize("unit", ["rms_bf16_xreg.hip", "rms_bf16_direct.hip", "rms_bf16_xpair.hip"])
def test_async_register_loads_untouched_until_waited(unit, tmp_path):
    import build_lib

    out = tmp_path / "k.s"
    flags = [f for f in build_lib.HIPCC_FLAGS if f != "-fPIC"]
    subprocess.run([_hipcc(), *flags, f"-I{build_lib.INCLUDE}", "--cuda-device-only", "-S", str(CSRC / unit),
                    "-o", str(out)], check=True, capture_output=True)
    ks = kernels(out.read_text())
    assert ks
    total = 0
    for name, lines in ks.items():
        n, bad = check_kernel(lines)
        total += n
        assert not bad, (name, bad[:3])
    assert total > 0
