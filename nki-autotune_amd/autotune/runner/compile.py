"""The "compile" step of the autotune pipeline: kernel instance -> shared library.

Replaces reference autotune/src/autotune/runner/compile.py (NKI source ->
NEFF through neuronx-cc, :154-244).  Here a candidate is one tile config of
a templated HIP kernel, and its ``KernelJob.source`` is the HIP translation
unit that instantiates that config (:func:`render_source`).  Compiling it
means:

1. parse the config back from the source header and check its static
   legality at the job's shape (LDS budget, wave tiling, alignment, 32-bit
   buffer offsets) through ``mi_cfg_check``;
2. if ``libmi_kernels.so`` already holds the instance (the whole 72-point
   grid is prebuilt), use it -- no hipcc run;
3. otherwise build the source with hipcc for gfx950 into a per-config
   library that exports the same C ABI (``include/mi_kernels.h``).

Same worker contract as the reference (compile_one :197-244): failures are
returned as strings in ``CompileResult.error`` and never raised, and every
build has a timeout (600 s in the reference, :230-231).  Builds run hipcc as
a child process, so a thread pool gives the parallelism the reference gets
from its process pool.
"""

from __future__ import annotations

import json
import os
import re
import subprocess
import threading
from pathlib import Path

from autotune.runner.types import CompileResult, capture_error
from kernel_library.config import REFERENCE_NAMES

HEADER_TAG = "// mi-autotune-instance: "
COMPILE_TIMEOUT_S = 600

# func_name aliases: the reference's kernel names map onto the MI355X families.
ALIASES = REFERENCE_NAMES

# Kernel families a single-config library can be generated for (fp32: no).
_JIT_FAMILIES = ("matmul_lhsT_rhs", "matmul_lhs_rhs", "rmsnorm_matmul")


def _instance(fam: str, cfg) -> tuple[str, str, str] | None:
    """(instantiation macro, table-row macro, macro arguments) of ``cfg``.

    Mirrors the instance files under csrc/: each variant of a family is a
    different kernel template (mi_registry.hpp).  None for a variant with no
    template.
    """
    bm, bn, bk, w, s, v = cfg.block_m, cfg.block_n, cfg.block_k, cfg.waves, cfg.lds_stages, int(cfg.variant)
    base = f"{bm}, {bn}, {bk}, {w}"
    if fam == "matmul_lhsT_rhs":
        macro = {0: "MI_MM", 1: "MI_MMP", 2: "MI_MMR", 3: "MI_MMPN", 4: "MI_MMW", 5: "MI_MMS", 6: "MI_MMSN"}.get(v)
        return (f"{macro}_INST", f"{macro}_ROW", f"{base}, {s}") if macro else None
    if fam == "matmul_lhs_rhs":
        macro = {0: "MI_MMK", 1: "MI_MMKP", 2: "MI_MMKN"}.get(v)
        return (f"{macro}_INST", f"{macro}_ROW", f"{base}, {s}") if macro else None
    if fam == "rmsnorm_matmul":
        if v in (0, 1):
            return "MI_RMS_INST", "MI_RMS_ROW", f"{base}, {s}, {v}"
        if v in (4, 5):
            return "MI_RMSX_INST", "MI_RMSX_ROW", f"{base}, {s}, {v - 2}"
        if v in (11, 12):
            return "MI_RMSXN_INST", "MI_RMSXN_ROW", f"{base}, {s}, {v - 9}"
        if v == 13:
            return "MI_RMS2_INST", "MI_RMS2_ROW", f"{base}, {s}"
        if v == 15:
            return "MI_RMS2P_INST", "MI_RMS2P_ROW", f"{base}, {s}"
        if v == 14:
            return "MI_RMSQ_INST", "MI_RMSQ_ROW", f"{base}, {s}"
        if v == 16:
            return "MI_RMSQP_INST", "MI_RMSQP_ROW", f"{base}, {s}"
    return None


def canonical_name(func_name: str) -> str:
    """Kernel family of a (possibly reference-named) function."""
    return ALIASES.get(func_name, func_name)


def render_source(func_name: str, cfg) -> str:
    """HIP translation unit instantiating ``func_name`` at tile config ``cfg``.

    The first line carries the config as JSON (the job's machine-readable
    description); the rest is a self-contained unit that, linked with
    ``mi_capi.hip``, yields a library exporting the full C ABI with exactly
    this one instance.
    """
    fam = canonical_name(func_name)
    head = HEADER_TAG + json.dumps({"func_name": fam, "config": cfg.asdict()}, sort_keys=True)
    spec = _instance(fam, cfg) if fam in _JIT_FAMILIES else None
    if spec is None:
        # fp32 path, or a variant without a template: prebuilt instances only.
        return head + "\n// prebuilt-only kernel family or variant: no generated unit\n"
    inst, row, args = spec
    return "\n".join(
        [
            head,
            f"// {fam} instance {cfg.name}, generated for a just-in-time autotune build (gfx950).",
            '#include "mi_registry.hpp"',
            "",
            "namespace mi {",
            f"{inst}({args})",
            "",
            "static const MiEntry* table_jit(int* n) {",
            f"  static const MiEntry t[] = {{{row}({args})}};",
            "  *n = 1;",
            "  return t;",
            "}",
            "",
            "const TableFn* table_list(int* n) {",
            "  static const TableFn tables[] = {table_jit};",
            "  *n = 1;",
            "  return tables;",
            "}",
            "}  // namespace mi",
            "",
        ]
    )


def parse_source(source: str):
    """``(func_name, TileConfig)`` from the header line of a rendered source."""
    from kernel_library.config import TileConfig

    first = source.splitlines()[0] if source else ""
    if not first.startswith(HEADER_TAG):
        raise ValueError("kernel source has no mi-autotune-instance header; build it with render_source()")
    meta = json.loads(first[len(HEADER_TAG):])
    return meta["func_name"], TileConfig(**meta["config"])


_CAPI_LOCK = threading.Lock()


# The C ABI units every per-config library links: the entry points and the
# library default config.
CAPI_UNITS = ("mi_capi.hip", "mi_defaults.hip")


def _capi_objects(work_dir: Path, hipcc_args: tuple[str, ...]) -> list[Path]:
    """Objects of the C ABI units, built once per work dir."""
    import build_lib

    objs = []
    with _CAPI_LOCK:
        for unit in CAPI_UNITS:
            obj = work_dir / unit.replace(".hip", ".o")
            if not obj.exists():
                cmd = [build_lib.hipcc(), *build_lib.HIPCC_FLAGS, *hipcc_args, "-c", str(build_lib.CSRC / unit),
                       "-o", str(obj)]
                proc = subprocess.run(cmd, capture_output=True, text=True, timeout=COMPILE_TIMEOUT_S)
                if proc.returncode != 0:
                    raise RuntimeError(f"hipcc failed for {unit}:\n{proc.stderr}")
            objs.append(obj)
    return objs


def build_instance(source: str, out_dir: Path, stem: str, hipcc_args: tuple[str, ...] = (),
                   timeout_s: int = COMPILE_TIMEOUT_S) -> tuple[Path, str]:
    """hipcc ``source`` (one instance) + the C ABI into ``out_dir/lib<stem>.so``; return (path, log)."""
    import build_lib

    out_dir.mkdir(parents=True, exist_ok=True)
    src = out_dir / f"{stem}.hip"
    src.write_text(source)
    obj = out_dir / f"{stem}.o"
    lib = out_dir / f"lib{stem}.so"
    capi = _capi_objects(out_dir.parent, hipcc_args)
    cmd = [build_lib.hipcc(), *build_lib.HIPCC_FLAGS, *hipcc_args, f"-I{build_lib.CSRC}", "-c", str(src), "-o",
           str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout_s)
    log = "\n".join(ln for ln in (proc.stdout + proc.stderr).splitlines() if "packed-fp32-ops" not in ln)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{log}")
    cmd = [build_lib.hipcc(), f"--offload-arch={build_lib.ARCH}", "-shared", "-fPIC", str(obj), *map(str, capi), "-o",
           str(lib)]
    proc = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout_s)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed for {lib.name}:\n{proc.stdout}{proc.stderr}")
    return lib, log


def problem_shape(func_name: str, input_specs: dict) -> tuple[int, int, int]:
    """(M, N, K) of a job from its input specs (signature order)."""
    shapes = [tuple(s) for s, _ in input_specs.values()]
    fam = canonical_name(func_name)
    if fam in ("matmul_lhsT_rhs", "matmul_lhsT_rhs_f32"):
        (K, M), (K2, N) = shapes[0], shapes[1]
    elif fam == "matmul_lhs_rhs":
        (M, K), (K2, N) = shapes[0], shapes[1]
    elif fam == "rmsnorm_matmul":
        (M, K), (K2, N) = shapes[0], shapes[-1]
    else:
        raise ValueError(f"unknown kernel family {func_name!r}")
    if K != K2:
        raise ValueError(f"contraction mismatch in input specs: {shapes}")
    return M, N, K


def _stem(kernel_name: str) -> str:
    return re.sub(r"[^A-Za-z0-9_.-]", "_", Path(kernel_name).stem)


def compile_one(kernel_name: str, source: str, func_name: str, input_specs: dict, work_dir: str,
                hipcc_args: tuple[str, ...] = (), allow_jit: bool = True,
                timeout_s: int = COMPILE_TIMEOUT_S) -> CompileResult:
    """Resolve one job to a library holding its instance; never raises."""
    from kernel_library import _lib
    from kernel_library.config import check

    src_path = ""
    try:
        fam, cfg = parse_source(source)
        if canonical_name(func_name) != fam:
            raise ValueError(f"job func_name {func_name!r} does not match its source ({fam!r})")
        M, N, K = problem_shape(func_name, input_specs)
        rc, msg = check(fam, cfg, M, N, K)
        if rc == 0:
            return CompileResult(kernel_name, src_path, str(_lib.LIB_PATH), "", "prebuilt instance")
        if rc != _lib.MI_E_NO_INSTANCE:
            return CompileResult(kernel_name, src_path, "", f"illegal config {cfg.name} at M={M} N={N} K={K}: "
                                 f"[{_lib.CODE_NAMES.get(rc, rc)}] {msg}")
        if not allow_jit:
            return CompileResult(kernel_name, src_path, "", f"config {cfg.name} is not prebuilt and JIT is off: {msg}")
        if fam not in _JIT_FAMILIES or _instance(fam, cfg) is None:
            return CompileResult(kernel_name, src_path, "", f"config {cfg.name} is not prebuilt and has no template "
                                 f"to build it from: {msg}")
        out_dir = Path(work_dir) / _stem(kernel_name)
        lib, log = build_instance(source, out_dir, "mi_" + _stem(kernel_name).replace(".", "_"), hipcc_args,
                                  timeout_s)
        return CompileResult(kernel_name, str(out_dir / (lib.stem[3:] + ".hip")), str(lib), "", log)
    except subprocess.TimeoutExpired as exc:
        return CompileResult(kernel_name, src_path, "", f"Compilation timed out after {exc.timeout} s")
    except Exception as exc:  # the worker contract: errors are strings
        return CompileResult(kernel_name, src_path, "", capture_error(exc))


def default_work_dir(func_name: str) -> str:
    """Scratch directory of a profile run (reference driver.py:143-150 uses /tmp/autotune-<func>)."""
    return os.path.join(os.environ.get("TMPDIR", "/tmp"), f"autotune-{canonical_name(func_name)}")
