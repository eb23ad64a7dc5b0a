"""Planted mistakes in the oracle (CPU only): each pin of tests/test_oracle.py must catch one.

A mistake is planted by swapping one oracle function for a plausible wrong
variant (a dropped term, a wrong axis or index, a transposed operand, the
wrong rounding) and re-running the pin, which must then fail.
"""

from __future__ import annotations

import numpy as np
import pytest

import test_oracle as pins
from oracle import bf16, matmul, rmsnorm


def _fails(fn, *args):
    with pytest.raises((AssertionError, ValueError)):
        fn(*args)


def test_transposed_operand_is_caught(monkeypatch):
    monkeypatch.setattr(matmul, "closed_form", lambda a, b: np.asarray(a, np.float64) @ np.asarray(b, np.float64))
    _fails(pins.test_matmul_hand_example)


def test_lhs_used_as_lhs_T_is_caught(monkeypatch):
    monkeypatch.setattr(matmul, "closed_form_lhs", lambda a, b: np.asarray(a, np.float64).T @ np.asarray(b, np.float64))
    _fails(pins.test_matmul_lhs_hand_example)


def test_lhs_tiled_without_transpose_is_caught(monkeypatch):
    monkeypatch.setattr(matmul, "tiled_lhs", lambda a, b, out_dtype="bfloat16": matmul.tiled(a, b, out_dtype))
    _fails(pins.test_matmul_lhs_hand_example)


def test_dropped_k_tail_is_caught(monkeypatch):
    real = matmul.tiled

    def tail_dropped(lhs_T, rhs, out_dtype="bfloat16"):
        K = lhs_T.shape[0] // matmul.TILE_K * matmul.TILE_K
        return real(lhs_T[:K], rhs[:K], out_dtype)

    monkeypatch.setattr(matmul, "tiled", tail_dropped)
    _fails(pins.test_matmul_tiled_fp32_matches_closed_form, 2304 + 100, 640, 1100)


def test_fp32_drain_instead_of_bf16_is_caught(monkeypatch):
    monkeypatch.setattr(matmul, "round_bf16", lambda x: np.asarray(x, np.float32))
    _fails(pins.test_matmul_tiled_bf16_two_stage_k)


def test_truncating_bf16_is_caught(monkeypatch):
    def truncate(x):
        return (np.ascontiguousarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)

    monkeypatch.setattr(bf16, "to_bf16_bits", truncate)
    _fails(pins.test_bf16_known_answers, 1.0 + 3 * 2.0**-8, 0x3F82)


def test_sum_instead_of_mean_is_caught(monkeypatch):
    def bad(lhs, eps=rmsnorm.EPS):
        x = np.asarray(lhs, np.float64)
        return 1.0 / np.sqrt((x * x).sum(axis=1) + eps)

    monkeypatch.setattr(rmsnorm, "inv_rms", bad)
    _fails(pins.test_rmsnorm_hand_example)


def test_eps_outside_sqrt_is_caught(monkeypatch):
    def bad(lhs, eps=rmsnorm.EPS):
        x = np.asarray(lhs, np.float64)
        return 1.0 / np.sqrt((x * x).mean(axis=1)) + eps

    monkeypatch.setattr(rmsnorm, "inv_rms", bad)
    _fails(pins.test_rmsnorm_hand_example)


def test_gamma_on_wrong_axis_is_caught(monkeypatch):
    real = rmsnorm.closed_form

    def bad(lhs, rhs, gamma=None, eps=rmsnorm.EPS):
        if gamma is None:
            return real(lhs, rhs, None, eps)
        y = real(lhs, np.eye(lhs.shape[1]), None, eps)
        return (y * np.resize(np.asarray(gamma, np.float64), lhs.shape[0])[:, None]) @ rhs

    monkeypatch.setattr(rmsnorm, "closed_form", bad)
    _fails(pins.test_rmsnorm_closed_form_vs_loops, True)


def test_online_without_rescale_is_caught(monkeypatch):
    real = rmsnorm.online

    def no_rescale(lhs, rhs, gamma=None, eps=rmsnorm.EPS, tile_dtype="float32"):
        # sum of per-block products each scaled by its own running rms (s_k = 1 dropped)
        x = np.asarray(lhs, np.float32)
        out = np.zeros((x.shape[0], rhs.shape[1]), np.float32)
        m = np.zeros(x.shape[0], np.float32)
        for k0 in range(0, x.shape[1], rmsnorm.BLOCK_K):
            t = x[:, k0:k0 + rmsnorm.BLOCK_K]
            m += (t * t).sum(axis=1)
            r = 1.0 / np.sqrt(m / x.shape[1] + eps)
            y = t * r[:, None]
            if gamma is not None:
                y = y * np.asarray(gamma, np.float32)[None, k0:k0 + rmsnorm.BLOCK_K]
            out += y @ np.asarray(rhs, np.float32)[k0:k0 + rmsnorm.BLOCK_K]
        return out

    assert real is not no_rescale
    monkeypatch.setattr(rmsnorm, "online", no_rescale)
    _fails(pins.test_rmsnorm_online_equals_two_pass, 64, 512 * 3, 128)
