"""The tile-config MDP and the frontier-expansion sampler (CPU only).

Pins the sampler's contract (reference docs/superpowers/specs/
2026-05-05-unified-tune-stage-design.md:27-54): every pooled config is
legal, same seed gives the same sample, each (config, atom) edge is tried
once, and at exhaustion the pool is the whole reachable set whatever the
seed -- checked against a plain breadth-first closure of the same moves.
"""

from __future__ import annotations

from collections import deque

import pytest

import kernel_library as kl
from autotune.search import Atom, IllegalMove, TileMDP, atoms_for, frontier_pool, frontier_sample
from kernel_library.config import TileConfig


def _closure(mdp: TileMDP) -> set[str]:
    root = mdp.reset()
    seen = {root.name: root}
    q = deque([root])
    while q:
        s = q.popleft()
        for a in mdp.atoms:
            try:
                n = mdp.step(s, a)
            except IllegalMove:
                continue
            if n.name not in seen:
                seen[n.name] = n
                q.append(n)
    return set(seen)


def test_mdp_moves_and_legality():
    mdp = TileMDP("matmul_lhsT_rhs", 4096, 4096, 4096, prebuilt_only=True)
    s = mdp.reset()
    assert mdp.is_legal(s)
    acts = mdp.legal_actions(s)
    assert acts and all(isinstance(a, Atom) for a in acts)
    for a in acts:
        n = mdp.step(s, a)
        assert n != s and kl.check("matmul_lhsT_rhs", n, 4096, 4096, 4096)[0] == 0
    with pytest.raises(IllegalMove):
        mdp.step(TileConfig(512, 512, 32, 8, 2, variant=1), Atom("block_m", "x2"))   # 1024 out of range
    with pytest.raises(IllegalMove):
        mdp.step(s, Atom("variant", f"={s.variant}"))                                 # no-op move
    assert Atom("variant", "=13") in atoms_for("rmsnorm_matmul")
    assert Atom("split_k", "x2") in atoms_for("matmul_lhsT_rhs")
    assert Atom("split_k", "x2") in atoms_for("rmsnorm_matmul")
    assert Atom("split_k", "x2") not in atoms_for("matmul_lhsT_rhs_f32")
    assert not mdp.is_terminal(s)
    # Variant moves reach every variant of the family, 0 and those above 8 included.
    assert mdp.step(TileConfig(256, 256, 32, 4, 2, variant=1), Atom("variant", "=0")).variant == 0
    rms = TileMDP("rmsnorm_matmul", 4096, 4096, 4096, prebuilt_only=True)
    assert rms.step(TileConfig(256, 256, 32, 4, 2, variant=0), Atom("variant", "=13")).variant == 13


@pytest.mark.parametrize("fam", ["matmul_lhsT_rhs", "matmul_lhs_rhs", "rmsnorm_matmul"])
def test_exhaustion_is_the_reachable_set_for_any_seed(fam):
    mdp = TileMDP(fam, 2048, 2048, 2048, prebuilt_only=True)
    want = _closure(mdp)
    assert len(want) > 10
    for seed in (0, 1, 7):
        got = {c.name for c in frontier_pool(TileMDP(fam, 2048, 2048, 2048, prebuilt_only=True), 10**6, seed)}
        assert got == want, seed


def test_sample_is_deterministic_legal_and_capped():
    mk = lambda: TileMDP("matmul_lhsT_rhs", 8192, 8192, 8192)   # noqa: E731
    a = frontier_sample(mk(), 12, seed=3)
    b = frontier_sample(mk(), 12, seed=3)
    c = frontier_sample(mk(), 12, seed=4)
    assert [x.name for x in a] == [x.name for x in b]
    assert [x.name for x in a] != [x.name for x in c]
    assert len({x.name for x in a}) == 12
    mdp = mk()
    assert all(mdp.is_legal(x) for x in a)
    pool = frontier_pool(mk(), 30, seed=0)
    assert len(pool) == 30          # capped before exhaustion: the JIT-reachable space is larger
    with pytest.raises(ValueError):
        frontier_sample(mk(), 0)


def test_prebuilt_only_stays_in_the_library():
    prebuilt = {c.name for c in kl.compiled_configs("matmul_lhsT_rhs")}
    for c in frontier_pool(TileMDP("matmul_lhsT_rhs", 4096, 4096, 4096, prebuilt_only=True), 10**6, 0):
        # split_k is a launch parameter of a prebuilt instance, not an instance of its own
        base = TileConfig(c.block_m, c.block_n, c.block_k, c.waves, c.lds_stages, 1, 8, c.variant)
        assert base.name in prebuilt, c
        assert c.split_k == 1 or c.variant in (1, 3, 4), c
    assert Atom("split_k", "x2") in atoms_for("matmul_lhs_rhs")


@pytest.mark.parametrize("fam,shape", [("matmul_lhsT_rhs", (4096, 4096, 4096)),
                                       ("matmul_lhsT_rhs", (128, 28672, 8192)),
                                       ("matmul_lhs_rhs", (2048, 2048, 2048)),
                                       ("rmsnorm_matmul", (4096, 4096, 4096)),
                                       ("rmsnorm_matmul", (64, 28672, 8192))])
def test_sampled_jit_configs_instantiate(fam, shape, tmp_path):
    """Every config the sampler takes as legal but not prebuilt is one its
    template instantiates: a sample of them, instantiated together in one
    unit, passes hipcc's device-side semantic checks (the templates'
    static_asserts) -- the sampler never proposes a compile error."""
    import random
    import shutil
    import subprocess
    from pathlib import Path

    import build_lib
    from autotune.runner.compile import _instance
    from kernel_library import _lib

    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    mdp = TileMDP(fam, *shape, prebuilt_only=False)
    pool = frontier_pool(mdp, 600, seed=0)
    jit = [c for c in pool if kl.check(fam, c, *shape)[0] == _lib.MI_E_NO_INSTANCE]
    assert jit, "the sampler reached no config outside the prebuilt set"
    sample = random.Random(0).sample(jit, min(16, len(jit)))
    lines = ['#include "mi_registry.hpp"', "namespace mi {"]
    seen = set()
    for c in sample:
        inst, _row, args = _instance(fam, c)
        if (inst, args) not in seen:
            seen.add((inst, args))
            lines.append(f"{inst}({args})")
    lines.append("}  // namespace mi")
    unit = tmp_path / "sampled.hip"
    unit.write_text("\n".join(lines) + "\n")
    flags = [f for f in build_lib.HIPCC_FLAGS if f != "-fPIC"]
    proc = subprocess.run([hipcc, *flags, f"-I{build_lib.CSRC}", f"-I{build_lib.INCLUDE}", "--cuda-device-only",
                           "-fsyntax-only", "-ferror-limit=0", str(unit)], capture_output=True, text=True)
    assert proc.returncode == 0, ([c.name for c in sample], proc.stderr[-3000:])
