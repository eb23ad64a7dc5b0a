"""CPU pins of the oracle (oracle/), so that it can be trusted as the checker.

Every oracle function is checked against something other than its own
formula: known answers worked by hand, numpy's published seeded streams,
torch's independent bf16 conversion, a brute-force loop, textbook
identities, and the reference's own test procedures (seed-0 128^3 at
atol=rtol=1e-4, test/ops/test_direct_numpy_call.py:32-38; the 256x256x512
fixture, test/transforms/_fixtures.py:36-59; fp32 atol=rtol=5e-3 end to end,
test/codegen/test_render.py:35-49).
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import bf16, inputs, matmul, metrics, rmsnorm

# --------------------------------------------------------------------- bf16


@pytest.mark.parametrize(
    "value,bits",
    [
        (1.0, 0x3F80),
        (-2.0, 0xC000),
        (1.0 + 2.0**-8, 0x3F80),          # tie -> even (mantissa 0)
        (1.0 + 3 * 2.0**-8, 0x3F82),      # tie -> even (rounds up)
        (1.0 + 2.0**-8 + 2.0**-20, 0x3F81),  # just above the tie -> up
        (float("inf"), 0x7F80),
        (-float("inf"), 0xFF80),
        (3.3895313892515355e38, 0x7F7F),  # largest bf16 is exact
        (3.4028234663852886e38, 0x7F80),  # fp32 max rounds to inf
        (0.0, 0x0000),
        (-0.0, 0x8000),
        (2.0**-133, 0x0001),              # smallest bf16 subnormal
    ],
)
def test_bf16_known_answers(value, bits):
    assert int(bf16.to_bf16_bits(np.array([value], dtype=np.float32))[0]) == bits


def test_bf16_nan_is_canonical_quiet_nan():
    out = bf16.to_bf16_bits(np.array([np.nan, -np.nan], dtype=np.float32))
    assert list(out) == [0x7FC0, 0x7FC0]


def test_bf16_matches_torch_rounding():
    """torch's float32 -> bfloat16 cast is an independent RNE implementation."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(5)
    x = np.concatenate([
        rng.standard_normal(200_000).astype(np.float32) * np.float32(1e3),
        rng.uniform(-1, 1, 100_000).astype(np.float32) * np.float32(1e-38),   # subnormals
        (np.arange(1 << 16, dtype=np.uint32) << 16 | 0x8000).view(np.float32),  # every tie pattern
    ])
    x = x[np.isfinite(x)]
    ours = bf16.to_bf16_bits(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    assert np.array_equal(bf16.round_bf16(x), torch.from_numpy(x).to(torch.bfloat16).float().numpy())


# ------------------------------------------------------------------- inputs


def test_inputs_follow_numpy_published_stream():
    """default_rng(0).standard_normal starts 0.12573022, -0.13210486, 0.64042265, 0.10490012;
    tensors draw in signature order (reference benchmark.py:163-168)."""
    d = inputs.generate({"lhs_T": ((2,), "float32"), "rhs": ((2,), "float32")}, 0)
    np.testing.assert_allclose(d["lhs_T"], [0.12573022, -0.13210486], rtol=1e-7)
    np.testing.assert_allclose(d["rhs"], [0.64042265, 0.10490012], rtol=1e-7)
    s42 = inputs.generate({"a": ((2,), "float32")}, 42)["a"]
    np.testing.assert_allclose(s42, [0.30471708, -1.03998411], rtol=1e-7)


def test_inputs_uniform_gamma_sigma_and_bf16():
    d = inputs.generate({"u": ((2,), "float32")}, 0, {"u": "uniform"})
    np.testing.assert_allclose(d["u"], [0.27392337, -0.46042657], rtol=1e-7)
    g = inputs.generate({"g": ((2,), "float32")}, 0, {"g": "gamma"})["g"]
    np.testing.assert_allclose(g, 1 + 0.1 * np.array([0.12573022, -0.13210486]), rtol=1e-6)
    s = inputs.generate({"s": ((2,), "float32")}, 0, {"s": ("normal", 0.02)})["s"]
    np.testing.assert_allclose(s, 0.02 * np.array([0.12573022, -0.13210486]), rtol=1e-6)
    b = inputs.generate({"b": ((1000,), "bfloat16")}, 3)["b"]
    assert np.array_equal(b, bf16.round_bf16(b))          # representable in bf16
    f = inputs.generate({"b": ((1000,), "float32")}, 3)["b"]
    assert np.max(np.abs(b - f) / np.abs(f)) <= 2.0**-8     # RNE bound: 8 significant bits


def test_product_generator_draws_the_same_stream():
    """The profiler's generate_tensors and the oracle's generator agree value for value."""
    from autotune.runner.benchmark import generate_tensors

    specs = {"lhs_T": ((64, 32), "bfloat16"), "gamma": ((64,), "bfloat16"), "rhs": ((64, 48), "bfloat16")}
    dists = {"lhs_T": "uniform", "gamma": "gamma", "rhs": ("normal", 0.125)}
    prod = generate_tensors(specs, 7, dists)
    ora = inputs.generate({k: (s, "float32") for k, (s, _d) in specs.items()}, 7, dists)
    for k in specs:
        assert np.array_equal(prod[k], ora[k]), k


# ------------------------------------------------------------------- matmul


def test_matmul_hand_example():
    """out[m, n] = sum_k lhs_T[k, m] rhs[k, n], worked by hand."""
    lhs_T = np.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]])   # K=2, M=3
    rhs = np.array([[1.0, -1.0], [0.5, 2.0]])              # K=2, N=2
    expected = np.array([[1 + 2.0, -1 + 8.0], [2 + 2.5, -2 + 10.0], [3 + 3.0, -3 + 12.0]])
    assert np.array_equal(matmul.closed_form(lhs_T, rhs), expected)
    assert np.array_equal(matmul.brute_force(lhs_T, rhs), expected)
    assert np.array_equal(matmul.tiled(lhs_T, rhs, "float32"), expected)


@pytest.mark.parametrize("K,M,N", [(7, 5, 3), (16, 8, 12), (33, 17, 9)])
def test_matmul_closed_form_vs_brute_force(K, M, N):
    d = inputs.generate({"lhs_T": ((K, M), "float32"), "rhs": ((K, N), "float32")}, K)
    np.testing.assert_allclose(matmul.closed_form(d["lhs_T"], d["rhs"]), matmul.brute_force(d["lhs_T"], d["rhs"]),
                               rtol=1e-12, atol=1e-12)


def test_matmul_identities():
    rng = np.random.default_rng(1)
    K, M, N = 96, 40, 56
    a = rng.standard_normal((K, M))
    b = rng.standard_normal((K, N))
    c = rng.standard_normal((K, N))
    # lhs_T = I gives rhs
    assert np.array_equal(matmul.closed_form(np.eye(K), b), b)
    # linearity in rhs
    np.testing.assert_allclose(matmul.closed_form(a, 2 * b + c),
                               2 * matmul.closed_form(a, b) + matmul.closed_form(a, c), atol=1e-11)
    # K-split associativity (the reference's 2-stage K reduction in exact arithmetic)
    np.testing.assert_allclose(matmul.closed_form(a, b),
                               matmul.closed_form(a[:40], b[:40]) + matmul.closed_form(a[40:], b[40:]), atol=1e-11)
    # permuting K rows of both operands together changes nothing
    p = rng.permutation(K)
    np.testing.assert_allclose(matmul.closed_form(a[p], b[p]), matmul.closed_form(a, b), atol=1e-11)
    # transposition: (lhs_T^T rhs)^T = rhs^T lhs_T
    np.testing.assert_allclose(matmul.closed_form(a, b).T, matmul.closed_form(b, a), atol=1e-11)


def test_matmul_reference_128cube_procedure():
    """test/ops/test_direct_numpy_call.py:32-38: seed 0, 128^3 fp32, atol=rtol=1e-4."""
    rng = np.random.default_rng(0)
    lhs_T = rng.standard_normal((128, 128)).astype(np.float32)
    rhs = rng.standard_normal((128, 128)).astype(np.float32)
    np.testing.assert_allclose(matmul.tiled(lhs_T, rhs, "float32"), matmul.closed_form(lhs_T, rhs),
                               atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("K,M,N", [(512, 256, 256),   # reference small fixture (test/transforms/_fixtures.py:36-59)
                                   (512, 256, 512),   # benchmark config C1
                                   (2304, 640, 1100)])  # several K blocks, ragged M/N edge tiles
def test_matmul_tiled_fp32_matches_closed_form(K, M, N):
    """The loop-nest emulation at fp32 is the simulate_fp32 path: allclose 5e-3 (test_render.py:49)."""
    d = inputs.generate({"lhs_T": ((K, M), "float32"), "rhs": ((K, N), "float32")}, 0)
    np.testing.assert_allclose(matmul.tiled(d["lhs_T"], d["rhs"], "float32"),
                               matmul.closed_form(d["lhs_T"], d["rhs"]), atol=5e-3, rtol=5e-3)


def test_matmul_tiled_bf16_two_stage_k():
    """bf16 tiled output: each 1024-row K block is drained to bf16 and added in bf16
    (kernel_hand_90.92mfu.py:92-98).  With the second K block zero, the result is one
    drain of the first block; with both blocks equal it is round(2 * round(p)) = 2 * round(p)."""
    rng = np.random.default_rng(2)
    M, N = 128, 512
    # small integers: every fp32 partial sum is exact, so the summation order cannot matter
    a1 = rng.integers(-2, 3, (1024, M)).astype(np.float32)
    b1 = rng.integers(-2, 3, (1024, N)).astype(np.float32)
    p = (a1.T @ b1).astype(np.float32)
    assert np.any(bf16.round_bf16(p) != p)   # some sums need rounding to bf16
    zeros_a = np.zeros_like(a1)
    one_block = matmul.tiled(np.vstack([a1, zeros_a]), np.vstack([b1, b1]), "bfloat16")
    np.testing.assert_array_equal(one_block, bf16.round_bf16(p))
    two_equal = matmul.tiled(np.vstack([a1, a1]), np.vstack([b1, b1]), "bfloat16")
    np.testing.assert_array_equal(two_equal, 2 * bf16.round_bf16(p))


def test_matmul_lhs_hand_example():
    """matmul_lhs_rhs: out[m, n] = sum_k lhs[m, k] rhs[k, n], worked by hand (lhs row-major, K contiguous)."""
    lhs = np.array([[1.0, 4.0], [2.0, 5.0], [3.0, 6.0]])   # M=3, K=2
    rhs = np.array([[1.0, -1.0], [0.5, 2.0]])              # K=2, N=2
    expected = np.array([[1 + 2.0, -1 + 8.0], [2 + 2.5, -2 + 10.0], [3 + 3.0, -3 + 12.0]])
    assert np.array_equal(matmul.closed_form_lhs(lhs, rhs), expected)
    assert np.array_equal(matmul.tiled_lhs(lhs, rhs, "float32"), expected)
    with pytest.raises(ValueError):
        matmul.closed_form_lhs(lhs.T, rhs[:1])


@pytest.mark.parametrize("M,K,N", [(5, 7, 3), (17, 33, 9)])
def test_matmul_lhs_vs_brute_force(M, K, N):
    """lhs . rhs against the BLAS-free triple loop of the transposed operand."""
    d = inputs.generate({"lhs": ((M, K), "float32"), "rhs": ((K, N), "float32")}, M)
    np.testing.assert_allclose(matmul.closed_form_lhs(d["lhs"], d["rhs"]),
                               matmul.brute_force(np.ascontiguousarray(d["lhs"].T), d["rhs"]), rtol=1e-12, atol=1e-12)


def test_matmul_lhs_tiled_two_stage_k():
    """The lhs.rhs kernel drains each 1024-row K block to bf16 and adds in bf16
    (kernel_handtuned_89.26mfu.py:120-166): integer operands make every fp32
    partial exact, so only the drains round."""
    rng = np.random.default_rng(3)
    M, N = 128, 512
    a1 = rng.integers(-2, 3, (M, 1024)).astype(np.float32)
    b1 = rng.integers(-2, 3, (1024, N)).astype(np.float32)
    p = (a1 @ b1).astype(np.float32)
    assert np.any(bf16.round_bf16(p) != p)
    two_equal = matmul.tiled_lhs(np.hstack([a1, a1]), np.vstack([b1, b1]), "bfloat16")
    np.testing.assert_array_equal(two_equal, 2 * bf16.round_bf16(p))
    d = inputs.generate({"lhs": ((640, 2304 + 100), "float32"), "rhs": ((2304 + 100, 300), "float32")}, 0)
    np.testing.assert_allclose(matmul.tiled_lhs(d["lhs"], d["rhs"], "float32"),
                               matmul.closed_form_lhs(d["lhs"], d["rhs"]), atol=5e-3, rtol=5e-3)


# ------------------------------------------------------------------ rmsnorm


def _rmsnorm_loops(x, w, gamma, eps):
    """Pure-Python loops with math.sqrt: an implementation independent of numpy broadcasting."""
    M, K = len(x), len(x[0])
    N = len(w[0])
    out = [[0.0] * N for _ in range(M)]
    for m in range(M):
        ms = sum(float(v) * float(v) for v in x[m]) / K
        r = 1.0 / math.sqrt(ms + eps)
        y = [float(x[m][k]) * r * (1.0 if gamma is None else float(gamma[k])) for k in range(K)]
        for n in range(N):
            out[m][n] = sum(y[k] * float(w[k][n]) for k in range(K))
    return np.array(out)


def test_rmsnorm_hand_example():
    """x = [3, 4]: mean(x^2) = 12.5, so y = x / sqrt(12.5 + eps); W = I returns y."""
    x = np.array([[3.0, 4.0]])
    y = rmsnorm.closed_form(x, np.eye(2), None, eps=0.0)
    np.testing.assert_allclose(y, [[3 / math.sqrt(12.5), 4 / math.sqrt(12.5)]], rtol=1e-15)
    np.testing.assert_allclose(rmsnorm.inv_rms(x, eps=1e-6), [1 / math.sqrt(12.5 + 1e-6)], rtol=1e-15)


@pytest.mark.parametrize("gamma", [False, True])
def test_rmsnorm_closed_form_vs_loops(gamma):
    d = inputs.generate({"lhs": ((5, 24), "float32"), "gamma": ((24,), "float32"), "rhs": ((24, 7), "float32")}, 4,
                        {"gamma": "gamma"})
    g = d["gamma"] if gamma else None
    np.testing.assert_allclose(rmsnorm.closed_form(d["lhs"], d["rhs"], g),
                               _rmsnorm_loops(d["lhs"].tolist(), d["rhs"].tolist(), g, 1e-6), rtol=1e-12, atol=1e-12)


def test_rmsnorm_special_cases():
    rng = np.random.default_rng(3)
    K, N = 64, 16
    w = rng.standard_normal((K, N))
    g = 1 + 0.1 * rng.standard_normal(K)
    x = rng.standard_normal((6, K))
    x[1] = 0.0                     # zero row -> 0 (0 * finite rsqrt(eps))
    x[2] = -0.25                   # constant row -> -1 (eps negligible) then gamma @ W
    out = rmsnorm.closed_form(x, w, g)
    assert np.all(out[1] == 0.0)
    np.testing.assert_allclose(out[2], -(g @ w), rtol=1e-4)
    # scale invariance f(c x) = f(x), c > 0, up to eps
    np.testing.assert_allclose(rmsnorm.closed_form(8 * x, w, g), out, rtol=1e-5, atol=1e-6)
    # W = I is plain RMSNorm * gamma; gamma = None is gamma = 1
    np.testing.assert_allclose(rmsnorm.closed_form(x, np.eye(K), g), x * rmsnorm.inv_rms(x)[:, None] * g[None, :],
                               rtol=1e-12)
    np.testing.assert_allclose(rmsnorm.closed_form(x, w, None), rmsnorm.closed_form(x, w, np.ones(K)), rtol=1e-12)


@pytest.mark.parametrize("M,K,N", [(64, 512, 128), (1100, 1600, 600)])
def test_rmsnorm_online_equals_two_pass(M, K, N):
    """The online recurrence (kernel_hand_online.py:10-17) equals the two-pass form, in fp32."""
    d = inputs.generate({"lhs": ((M, K), "float32"), "gamma": ((K,), "float32"),
                         "rhs": ((K, N), "float32")}, 0, {"gamma": "gamma", "rhs": ("normal", 1 / math.sqrt(K))})
    for g in (None, d["gamma"]):
        np.testing.assert_allclose(rmsnorm.online(d["lhs"], d["rhs"], g), rmsnorm.closed_form(d["lhs"], d["rhs"], g),
                                   atol=5e-4, rtol=5e-4)


def test_rmsnorm_online_bf16_error_is_bounded():
    """The bf16-tile recurrence (rounded scaled tiles and O) stays within the rmsnorm gate of the closed form."""
    M, K, N = 256, 2048, 256
    d = inputs.generate({"lhs": ((M, K), "bfloat16"), "rhs": ((K, N), "bfloat16")}, 1,
                        {"rhs": ("normal", 1 / math.sqrt(K))})
    exp = rmsnorm.closed_form(d["lhs"], d["rhs"])
    got = rmsnorm.online(d["lhs"], d["rhs"], tile_dtype="bfloat16")
    floor = 0.05 * float(np.sqrt(np.mean(exp**2)))
    assert metrics.within(got, exp, atol=floor, rtol=5e-2)


# ------------------------------------------------------------------ metrics


def test_metrics_known_answers():
    a = np.array([1.0, 2.0, 0.0, -4.0])
    e = np.array([1.0, 2.5, 0.01, -4.0])
    rep = metrics.report(a, e, atol=5e-3, rtol=1e-2)
    assert rep["max_abs"] == pytest.approx(0.5)
    assert rep["max_rel"] == pytest.approx(max(0.5 / 2.505, 0.01 / 0.015))
    assert rep["normwise"] == pytest.approx(0.5 / 4.0)
    assert rep["nonfinite"] == 0 and rep["allclose"] is False
    # |a - e| <= atol + rtol * |e| with e = 1: the bound is 0.015
    assert metrics.within(np.array([1.0149]), np.array([1.0]), 5e-3, 1e-2)
    assert not metrics.within(np.array([1.0151]), np.array([1.0]), 5e-3, 1e-2)
    assert not metrics.within(np.array([np.nan]), np.array([0.0]), 1.0, 1.0)
    assert metrics.report(np.array([np.inf, 1.0]), np.array([1.0, 1.0]))["nonfinite"] == 1
