"""Search front end over tile configs: an MDP and a frontier-expansion sampler.

The reference explores its kernel space as an MDP whose actions are the
legal transforms of a state (``KernelMDP``, nkigym/src/nkigym/environment/
mdp.py:19-72) and samples it with a seeded, dedup'd frontier expansion
(docs/superpowers/specs/2026-05-05-unified-tune-stage-design.md:8-60).  Here
a state is a :class:`~kernel_library.config.TileConfig` and an action (an
"atom") changes one knob:

* ``block_m`` / ``block_n`` / ``block_k`` doubled or halved,
* ``waves`` 4 <-> 8,
* ``lds_stages`` +1 / -1,
* ``group_m`` (the L2 raster height) doubled or halved,
* ``variant`` set to another pipeline of the same kernel family,
* ``split_k`` (K split over several workgroups per output tile) doubled or
  halved, for the two matmuls and the fused kernel.

An atom is legal at a state when its result passes the library's static
legality check at the problem shape (``mi_cfg_check``: LDS budget, wave
tiling, alignment, 32-bit offsets, gamma capacity) and is either prebuilt
or, unless ``prebuilt_only``, buildable from its variant's template.

:func:`frontier_sample` keeps one pool of distinct configs (keyed by name)
and a frontier of pool members with untried atoms; each step picks a
frontier member and one of its untried atoms uniformly at random
(``random.Random(seed)``), applies it, and adds the result when it is new.
It stops when the pool holds ``pool_factor * num_kernels`` configs or the
frontier is empty (the whole reachable space), then draws ``num_kernels``
configs uniformly from the pool.  So every (config, atom) edge is tried at
most once, the pool at exhaustion is the reachable set whatever the seed,
and the same seed gives the same configs.
"""

from __future__ import annotations

import random
from dataclasses import replace
from typing import NamedTuple

import kernel_library as kl
from autotune.runner.compile import _JIT_FAMILIES, _instance, canonical_name
from kernel_library import _lib
from kernel_library.config import TileConfig


class Atom(NamedTuple):
    """One single-knob move: ``knob`` changed by ``op`` (``x2``, ``/2``, ``+1``, ``-1``, ``swap``, ``=<v>``)."""

    knob: str
    op: str


# Variants of each family that compute the same function (include/mi_kernels.h);
# rmsnorm_matmul 14 and 16 are left out: they compute the product without gamma only.
FAMILY_VARIANTS = {
    "matmul_lhsT_rhs": (0, 1, 2, 3, 4, 5, 6),
    "matmul_lhs_rhs": (0, 1, 2),
    "rmsnorm_matmul": (0, 1, 4, 5, 11, 12, 13, 15),
    "matmul_lhsT_rhs_f32": (0, 1),
}

_POW2_KNOBS = {"block_m": (32, 512), "block_n": (32, 512), "block_k": (16, 128), "group_m": (1, 64),
               "split_k": (1, 16)}


def atoms_for(func_name: str) -> list[Atom]:
    fam = canonical_name(func_name)
    out = [Atom(k, op) for k in ("block_m", "block_n", "block_k") for op in ("x2", "/2")]
    out += [Atom("waves", "swap"), Atom("lds_stages", "+1"), Atom("lds_stages", "-1"),
            Atom("group_m", "x2"), Atom("group_m", "/2")]
    out += [Atom("variant", f"={v}") for v in FAMILY_VARIANTS.get(fam, (0,))]
    if fam in ("matmul_lhsT_rhs", "matmul_lhs_rhs", "rmsnorm_matmul"):
        out += [Atom("split_k", "x2"), Atom("split_k", "/2")]
    return out


class IllegalMove(ValueError):
    """The atom does not apply at this state (out of range or illegal at the shape)."""


class TileMDP:
    """Pure-functional MDP over tile configs of one kernel family at one problem shape."""

    def __init__(self, func_name: str, M: int, N: int, K: int, prebuilt_only: bool = False) -> None:
        self.fam = canonical_name(func_name)
        self.M, self.N, self.K = M, N, K
        self.prebuilt_only = prebuilt_only
        self.atoms = atoms_for(self.fam)
        self._legal: dict[str, bool] = {}

    def reset(self) -> TileConfig:
        """The library's default (tuned) config at the shape, with an explicit raster height."""
        cfg = kl.default_config(self.fam, self.M, self.N, self.K)
        return cfg if cfg.group_m > 0 else replace(cfg, group_m=8)

    def is_legal(self, cfg: TileConfig) -> bool:
        if cfg.name not in self._legal:
            rc, _ = kl.check(self.fam, cfg, self.M, self.N, self.K)
            ok = rc == _lib.MI_OK
            if rc == _lib.MI_E_NO_INSTANCE and not self.prebuilt_only:
                ok = self.fam in _JIT_FAMILIES and _instance(self.fam, cfg) is not None
            self._legal[cfg.name] = ok
        return self._legal[cfg.name]

    def apply(self, state: TileConfig, atom: Atom) -> TileConfig:
        """The config ``atom`` leads to (not yet checked for legality)."""
        k, op = atom
        v = getattr(state, k)
        if op == "x2":
            nv = v * 2
        elif op == "/2":
            nv = v // 2
        elif op == "+1":
            nv = v + 1
        elif op == "-1":
            nv = v - 1
        elif op == "swap":
            nv = 8 if v == 4 else 4
        elif op.startswith("="):
            nv = int(op[1:])
        else:
            raise IllegalMove(f"unknown atom {atom}")
        if nv == v:
            raise IllegalMove(f"{atom} leaves {state.name} unchanged")
        # The variant moves name their family's variants (FAMILY_VARIANTS), so
        # only the numeric knobs have a range.
        lo, hi = _POW2_KNOBS.get(k, (1, 8))
        if k != "variant" and not lo <= nv <= hi:
            raise IllegalMove(f"{k}={nv} outside [{lo}, {hi}]")
        return replace(state, **{k: nv})

    def step(self, state: TileConfig, atom: Atom) -> TileConfig:
        nxt = self.apply(state, atom)
        if not self.is_legal(nxt):
            raise IllegalMove(f"{nxt.name} is illegal at {self.M}x{self.N}x{self.K}")
        return nxt

    def legal_actions(self, state: TileConfig) -> list[Atom]:
        out = []
        for a in self.atoms:
            try:
                self.step(state, a)
            except IllegalMove:
                continue
            out.append(a)
        return out

    def is_terminal(self, state: TileConfig) -> bool:
        return not self.legal_actions(state)


def frontier_pool(mdp: TileMDP, limit: int, seed: int = 0) -> list[TileConfig]:
    """Frontier expansion from ``mdp.reset()`` until ``limit`` configs or exhaustion (pool in discovery order)."""
    rng = random.Random(seed)
    root = mdp.reset()
    if not mdp.is_legal(root):
        raise IllegalMove(f"start config {root.name} is illegal at {mdp.M}x{mdp.N}x{mdp.K}")
    pool: dict[str, TileConfig] = {root.name: root}
    untried: dict[str, list[Atom]] = {root.name: list(mdp.atoms)}
    frontier: list[str] = [root.name]
    while frontier and len(pool) < limit:
        i = rng.randrange(len(frontier))
        name = frontier[i]
        atoms = untried[name]
        atom = atoms.pop(rng.randrange(len(atoms)))
        if not atoms:
            frontier[i] = frontier[-1]
            frontier.pop()
        try:
            nxt = mdp.step(pool[name], atom)
        except IllegalMove:
            continue
        if nxt.name not in pool:
            pool[nxt.name] = nxt
            untried[nxt.name] = list(mdp.atoms)
            frontier.append(nxt.name)
    return list(pool.values())


def frontier_sample(mdp: TileMDP, num_kernels: int, seed: int = 0, pool_factor: int = 100) -> list[TileConfig]:
    """``num_kernels`` configs drawn uniformly from a frontier-expanded pool of at most ``pool_factor`` x that."""
    if num_kernels <= 0:
        raise ValueError("num_kernels must be positive")
    pool = frontier_pool(mdp, pool_factor * num_kernels, seed)
    rng = random.Random(seed + 1)
    names = sorted(c.name for c in pool)
    by = {c.name: c for c in pool}
    return [by[n] for n in rng.sample(names, min(num_kernels, len(names)))]


__all__ = ["Atom", "IllegalMove", "TileMDP", "atoms_for", "frontier_pool", "frontier_sample"]
