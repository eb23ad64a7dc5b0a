"""bench.py's host-side pieces, on the CPU: the seeded shape sets of the default-config study."""

from __future__ import annotations

import importlib.util
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_random_default_shapes_are_seeded_and_in_bounds():
    """Each seed gives the same 30 shapes every time: 14 lhsT.rhs, 6 lhs.rhs and 10 rmsnorm_matmul, every size
    a multiple of 8 that the C ABI accepts, at most 5e11 FLOP each; different seeds give different shapes."""
    b = _bench()
    a1, a2, c = b.random_default_shapes(2028), b.random_default_shapes(2028), b.random_default_shapes(2026)
    assert a1 == a2 and a1 != c and len(a1) == 30
    fams = [f for f, _ in a1]
    assert (fams.count("matmul_lhsT_rhs"), fams.count("matmul_lhs_rhs"), fams.count("rmsnorm_matmul")) == (14, 6, 10)
    for _, (m, n, k) in a1 + c:
        assert m % 8 == 0 and n % 8 == 0 and k % 8 == 0
        assert 8 <= m <= 8192 and 512 <= n <= 14336 and 512 <= k <= 16384
        assert 2.0 * m * n * k <= 5e11
    skinny = sum(1 for _, (m, _, _) in a1 if m <= 128)
    assert 2 <= skinny <= 24  # 1/4 of the draws, more after the FLOP cap's redraws
