"""The oracle's qk_rope and output gate (oracle/attention.py), pinned on the CPU: the norm against float64 within its
roundings, rope's closed cases (no rotation, a quarter turn, the norm of each rotated pair kept), the gate's."""

import numpy as np
import pytest

from oracle import attention as OA
from oracle import route as OR

U = {"float16": 2.0 ** -11, "bfloat16": 2.0 ** -8}


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_the_norm_without_rope_is_rms_norm_within_two_roundings(dtype):
    rng = np.random.default_rng(1)
    S, H, D = 3, 4, 128
    x = OR.round_to(rng.standard_normal((S, H * D)) * 3, dtype)
    w = OR.round_to(1 + 0.1 * rng.standard_normal(D), dtype)
    got = OA.qk_rope(x, w, np.zeros((S, 0)), np.zeros((S, 0)), H, D, D, 1e-6, dtype).astype(np.float64)
    xs = x.reshape(S, H, D).astype(np.float64)
    want = (xs / np.sqrt((xs ** 2).mean(axis=-1, keepdims=True) + 1e-6) * w).transpose(1, 0, 2)
    assert (np.abs(got - want) <= 2.01 * U[dtype] * np.abs(want) + 1e-30).all()
    # a head of constant values c: normed to 1 times the weight
    xc = np.full((1, D), 2.5, np.float32)
    got = OA.qk_rope(xc, w, np.zeros((1, 0)), np.zeros((1, 0)), 1, D, D, 0.0, dtype)
    np.testing.assert_array_equal(got[0, 0], w)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_rope_closed_cases(dtype):
    rng = np.random.default_rng(2)
    S, H, D, rot = 2, 2, 64, 32
    x = OR.round_to(rng.standard_normal((S, H * 2 * D)), dtype)  # stride 2D: the second half is not read
    w = np.ones(D, np.float32)
    plain = OA.qk_rope(x, w, np.zeros((S, 0)), np.zeros((S, 0)), H, D, 2 * D, 1e-6, dtype)
    same = OA.qk_rope(x, w, np.ones((S, rot)), np.zeros((S, rot)), H, D, 2 * D, 1e-6, dtype)
    np.testing.assert_array_equal(same, plain)  # cos 1, sin 0: no rotation
    quarter = OA.qk_rope(x, w, np.zeros((S, rot)), np.ones((S, rot)), H, D, 2 * D, 1e-6, dtype)
    np.testing.assert_array_equal(quarter[..., :rot // 2], -plain[..., rot // 2:rot])  # (a, b) -> (-b, a)
    np.testing.assert_array_equal(quarter[..., rot // 2:rot], plain[..., :rot // 2])
    np.testing.assert_array_equal(quarter[..., rot:], plain[..., rot:])  # dims past rot untouched
    th = rng.uniform(0, 6.3, (S, rot // 2))
    cos = OR.round_to(np.cos(np.concatenate([th, th], axis=1)), dtype)
    sin = OR.round_to(np.sin(np.concatenate([th, th], axis=1)), dtype)
    turned = OA.qk_rope(x, w, cos, sin, H, D, 2 * D, 1e-6, dtype).astype(np.float64)
    p = plain.astype(np.float64)
    n0 = p[..., :rot // 2] ** 2 + p[..., rot // 2:rot] ** 2
    n1 = turned[..., :rot // 2] ** 2 + turned[..., rot // 2:rot] ** 2
    assert np.allclose(n1, n0, rtol=8 * U[dtype], atol=1e-6)  # a rotation keeps each pair's length


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_gate_closed_cases(dtype):
    out = np.array([1.5, -2.0, 0.75], np.float32)
    np.testing.assert_array_equal(OA.gate_out(out, np.zeros(3), dtype), out * 0.5)  # sigmoid(0) = 1/2
    np.testing.assert_array_equal(OA.gate_out(out, np.full(3, 30.0), dtype), out)  # rounds to 1
    assert (OA.gate_out(out, np.full(3, -30.0), dtype) == 0).all() or dtype == "bfloat16"
