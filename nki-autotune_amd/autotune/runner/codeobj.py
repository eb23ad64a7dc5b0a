"""The gfx950 code object that holds a kernel instance, read from its library.

The reference attaches the compiled artifact of each kernel to its result
when a detailed profile is asked for: ``ProfileResult.neff_b64``, the
base64 of the NEFF (reference autotune/src/autotune/runner/types.py:70-98,
filled at benchmark.py:133-143).  Here an instance is compiled into a HIP
shared library (the prebuilt ``libmi_kernels.so`` or a per-config library
built just in time).  hipcc places each translation unit's device code in
the library's ``.hip_fatbin`` section as one clang offload bundle, whose
``hipv4-amdgcn-amd-amdhsa--gfx950`` entry is an AMDGPU code object (an ELF
that ``hipModuleLoad`` and ``llvm-objdump`` take).  :func:`code_object_of`
returns the code object of the translation unit that defines the
instance's kernel: its Itanium-mangled name (template name and tile
parameters) appears in that code object's symbol strings only.  The code
object also holds the other instances of the same unit.

Only libraries built from this repository's sources are read.
"""

from __future__ import annotations

import struct

BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
ARCH = "gfx950"

# Kernel template of each (family, variant) and how many leading int
# template parameters (the tile config) it takes.
_TEMPLATES = {
    ("matmul_lhsT_rhs", 0): ("mm_lhsT_rhs_bf16_kernel", 5),
    ("matmul_lhsT_rhs", 1): ("mm_lhsT_rhs_bf16_pipe_kernel", 5),
    ("matmul_lhsT_rhs", 2): ("mm_lhsT_rhs_bf16_reg_kernel", 5),
    ("matmul_lhsT_rhs", 3): ("mm_lhsT_rhs_bf16_pipe_kernel", 5),
    ("matmul_lhsT_rhs", 4): ("mm_lhsT_rhs_bf16_kw_kernel", 5),
    ("matmul_lhsT_rhs", 5): ("mm_lhsT_rhs_bf16_sk_kernel", 5),
    ("matmul_lhsT_rhs", 6): ("mm_lhsT_rhs_bf16_sk_kernel", 5),
    ("matmul_lhs_rhs", 0): ("mm_lhs_rhs_bf16_pipe_kernel", 5),
    ("matmul_lhs_rhs", 1): ("mm_lhs_rhs_bf16_pair_kernel", 5),
    ("matmul_lhs_rhs", 2): ("mm_lhs_rhs_bf16_pipe_kernel", 5),
    ("rmsnorm_matmul", 0): ("rmsnorm_mm_bf16_kernel", 5),
    ("rmsnorm_matmul", 1): ("rmsnorm_mm_bf16_kernel", 5),
    ("rmsnorm_matmul", 4): ("rmsnorm_mm_bf16_xreg_kernel", 5),
    ("rmsnorm_matmul", 5): ("rmsnorm_mm_bf16_xreg_kernel", 5),
    ("rmsnorm_matmul", 11): ("rmsnorm_mm_bf16_xreg_kernel", 5),
    ("rmsnorm_matmul", 12): ("rmsnorm_mm_bf16_xreg_kernel", 5),
    ("rmsnorm_matmul", 13): ("rmsnorm_mm_bf16_2pass_kernel", 5),
    ("rmsnorm_matmul", 14): ("rmsnorm_mm_bf16_sq_kernel", 5),
    ("rmsnorm_matmul", 15): ("rmsnorm_mm_bf16_2pass_pair_kernel", 5),
    ("rmsnorm_matmul", 16): ("rmsnorm_mm_bf16_sq_pair_kernel", 5),
    ("matmul_lhsT_rhs_f32", 0): ("mm_f32_kernel", 3),
    ("matmul_lhsT_rhs_f32", 1): ("mm_f32_mfma_kernel", 2),
}


def mangled_stem(family: str, cfg) -> bytes | None:
    """The mangled-name fragment ``<len><template>ILi<bm>E...`` of the instance's main kernel, or None."""
    entry = _TEMPLATES.get((family, int(cfg.variant)))
    if entry is None:
        return None
    name, nargs = entry
    args = (cfg.block_m, cfg.block_n, cfg.block_k, cfg.waves, cfg.lds_stages)[:nargs]
    return (f"{len(name)}{name}I" + "".join(f"Li{int(a)}E" for a in args)).encode()


def _fatbin_section(data: bytes) -> bytes:
    """The ``.hip_fatbin`` section of an ELF64 shared library (the whole file if it has none)."""
    if data[:4] != b"\x7fELF" or data[4] != 2:
        return data
    shoff, = struct.unpack_from("<Q", data, 0x28)
    shentsize, shnum, shstrndx = struct.unpack_from("<HHH", data, 0x3A)
    if shoff == 0 or shnum == 0 or shstrndx >= shnum:
        return data

    def header(i: int):
        return struct.unpack_from("<IIQQQQIIQQ", data, shoff + i * shentsize)

    names_off = header(shstrndx)[4]
    for i in range(shnum):
        sh_name, _type, _flags, _addr, off, size = header(i)[:6]
        end = data.index(b"\0", names_off + sh_name)
        if data[names_off + sh_name:end] == b".hip_fatbin":
            return data[off:off + size]
    return data


def bundle_code_objects(data: bytes, arch: str = ARCH) -> list[bytes]:
    """Every ``arch`` code object in the clang offload bundles of ``data``, in order.

    Bundle layout: the magic string, a u64 entry count, then per entry a u64
    offset (from the bundle's start), u64 size, u64 triple length and the
    triple; the entries' bytes follow."""
    out = []
    pos = data.find(BUNDLE_MAGIC)
    while pos >= 0:
        try:
            n, = struct.unpack_from("<Q", data, pos + len(BUNDLE_MAGIC))
            p = pos + len(BUNDLE_MAGIC) + 8
            for _ in range(min(int(n), 64)):
                off, size, tlen = struct.unpack_from("<QQQ", data, p)
                triple = data[p + 24:p + 24 + tlen].decode("ascii", "replace")
                p += 24 + tlen
                if triple.startswith("hip") and triple.endswith(arch) and size > 0:
                    co = data[pos + off:pos + off + size]
                    if co[:4] == b"\x7fELF":
                        out.append(co)
        except struct.error:
            pass
        pos = data.find(BUNDLE_MAGIC, pos + len(BUNDLE_MAGIC))
    return out


def code_object_of(library_path: str, family: str, cfg) -> bytes | None:
    """The gfx950 code object of ``library_path`` that defines ``family``'s instance ``cfg``, or None."""
    stem = mangled_stem(family, cfg)
    if stem is None:
        return None
    with open(library_path, "rb") as f:
        data = f.read()
    for co in bundle_code_objects(_fatbin_section(data)):
        if stem in co:
            return co
    return None
