"""Build libmi_kernels.so (gfx950) from nki-autotune_amd/csrc.

Every ``*.hip`` translation unit under ``csrc/`` is compiled ahead of time
with ``hipcc --offload-arch=gfx950`` (in parallel, one process per unit) and
linked into ``kernel_library/libmi_kernels.so``, which the ctypes loader in
``kernel_library/_lib.py`` opens.  The tile-config search space lives in the
instance tables of those units, so building the library is the "compile"
step of every autotune candidate at once.  The units under ``csrc/probe/``
(measurement probes for bench.py, outside the kernel_library ABI) are linked
into ``kernel_library/libmi_probe.so``.

Usage: ``python nki-autotune_amd/build_lib.py [--jobs N] [--force]``.
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD = PKG_DIR / "_build"
LIB = PKG_DIR / "kernel_library" / "libmi_kernels.so"
PROBE_LIB = PKG_DIR / "kernel_library" / "libmi_probe.so"
INCLUDE = PKG_DIR.parent / "include"

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed-FP32 VALU forms stay off: some of them have produced silently
    # wrong results on MI355X.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    """Path of hipcc (ROCm install), raising if absent."""
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the MI355X kernels cannot be built")


def _sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _headers() -> list[Path]:
    return sorted(CSRC.glob("*.hpp")) + sorted(INCLUDE.glob("*.h"))


def _compile(src: Path, force: bool) -> tuple[Path, str]:
    obj = BUILD / (("probe_" if src.parent.name == "probe" else "") + src.stem + ".o")
    newest_dep = max(p.stat().st_mtime for p in [src, *_headers()])
    if not force and obj.exists() and obj.stat().st_mtime >= newest_dep:
        return obj, ""
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    log = "\n".join(line for line in (proc.stdout + proc.stderr).splitlines() if "packed-fp32-ops" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{log}")
    return obj, log


def _link(objs: list[Path], lib: Path) -> None:
    tmp = lib.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link of {lib.name} failed:\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, lib)


def build(jobs: int | None = None, force: bool = False, verbose: bool = False) -> Path:
    """Compile every csrc/*.hip unit and link libmi_kernels.so (and csrc/probe/ into libmi_probe.so)."""
    BUILD.mkdir(parents=True, exist_ok=True)
    srcs = _sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    probes = sorted((CSRC / "probe").glob("*.hip"))
    jobs = jobs or max(1, min(len(srcs) + len(probes), (os.cpu_count() or 2)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        results = list(pool.map(lambda s: _compile(s, force), srcs + probes))
    if verbose:
        for obj, log in results:
            if log.strip():
                print(f"[build] {obj.name}: {log.strip()}")
    objs = [obj for obj, _ in results]
    _link(objs[:len(srcs)], LIB)
    if probes:
        _link(objs[len(srcs):], PROBE_LIB)
    return LIB


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--force", action="store_true")
    ap.add_argument("-v", "--verbose", action="store_true")
    args = ap.parse_args()
    path = build(args.jobs, args.force, args.verbose)
    print(f"[build] {path}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
