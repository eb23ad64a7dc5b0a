"""Write the golden fixtures of the parity tests (tests/golden/*.npz).

The reference ships no stored vectors for this path: its pins are
procedures (seed-0 N(0,1) inputs against ``lhs_T.T @ rhs``,
test/ops/test_direct_numpy_call.py:32-38, test/codegen/test_render.py:35-49).
Its own implementation (nki.simulate) is not installed here and cannot be
imported, so the fixtures are made by this repository's oracle on
seeded inputs: inputs are stored as drawn (bf16 as uint16 bit patterns),
expected outputs in float64 from the oracle's closed forms, which
tests/test_oracle.py pins against independent implementations.

Usage: ``python tests/golden/make_golden.py`` (rewrites the .npz files).
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import bf16, inputs, matmul, rmsnorm  # noqa: E402

FIXTURES = {
    # name: (kind, shape, seed, dists)
    "mm_f32_128cube_seed0": ("mm", (128, 128, 128), 0, None, "float32"),        # reference 128^3 procedure
    "mm_bf16_k160_m96_n128": ("mm", (160, 96, 128), 11, "uniform", "bfloat16"),  # ragged vs every block size
    "mm_bf16_k1040_m40_n136": ("mm", (1040, 40, 136), 12, ("normal", 0.02), "bfloat16"),
    "lhs_bf16_m72_k296_n160": ("lhs", (72, 296, 160), 15, "uniform", "bfloat16"),   # K tail past a 32 tile
    "rms_bf16_m64_k256_n96": ("rms", (64, 256, 96), 13, None, "bfloat16"),
    "rms_bf16_m40_k520_n72_nogamma": ("rms", (40, 520, 72), 14, None, "bfloat16"),
}


def make(name: str) -> dict[str, np.ndarray]:
    kind, (a, b, c), seed, dist, dtype = FIXTURES[name]
    if kind == "mm":
        K, M, N = a, b, c
        d = inputs.generate({"lhs_T": ((K, M), dtype), "rhs": ((K, N), dtype)}, seed,
                            None if dist is None else {"lhs_T": dist, "rhs": dist})
        out = {"expected": matmul.closed_form(d["lhs_T"], d["rhs"])}
        if dtype == "bfloat16":
            out.update(lhs_T_bits=bf16.to_bf16_bits(d["lhs_T"]), rhs_bits=bf16.to_bf16_bits(d["rhs"]))
        else:
            out.update(lhs_T=d["lhs_T"], rhs=d["rhs"])
    elif kind == "lhs":
        M, K, N = a, b, c
        d = inputs.generate({"lhs": ((M, K), dtype), "rhs": ((K, N), dtype)}, seed, {"lhs": dist, "rhs": dist})
        out = {"expected": matmul.closed_form_lhs(d["lhs"], d["rhs"]),
               "lhs_bits": bf16.to_bf16_bits(d["lhs"]), "rhs_bits": bf16.to_bf16_bits(d["rhs"])}
    else:
        M, K, N = a, b, c
        gamma = not name.endswith("nogamma")
        specs = {"lhs": ((M, K), dtype)}
        if gamma:
            specs["gamma"] = ((K,), dtype)
        specs["rhs"] = ((K, N), dtype)
        d = inputs.generate(specs, seed, {"gamma": "gamma", "rhs": ("normal", 1 / np.sqrt(K))})
        out = {"expected": rmsnorm.closed_form(d["lhs"], d["rhs"], d.get("gamma")),
               "lhs_bits": bf16.to_bf16_bits(d["lhs"]), "rhs_bits": bf16.to_bf16_bits(d["rhs"])}
        if gamma:
            out["gamma_bits"] = bf16.to_bf16_bits(d["gamma"])
    out["seed"] = np.array(seed)
    return out


def load(name: str) -> dict[str, np.ndarray]:
    """Fixture arrays, bf16 bit patterns decoded to float32 under the plain names."""
    with np.load(HERE / f"{name}.npz", allow_pickle=False) as z:
        d = {k: z[k] for k in z.files}
    for k in list(d):
        if k.endswith("_bits"):
            d[k[:-5]] = bf16.from_bf16_bits(d[k])
    return d


def main() -> int:
    for name in FIXTURES:
        np.savez_compressed(HERE / f"{name}.npz", **make(name))
        print(f"wrote {name}.npz ({os.path.getsize(HERE / f'{name}.npz')} bytes)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
