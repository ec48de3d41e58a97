"""The hyper-connection oracle (oracle/hc.py, strata_mlx/fused.py:46-131, 281-323) pinned on the CPU: float64
evaluation of the reference kernels' formulas, and closed cases a dropped term, factor or sign would break."""

import numpy as np
import pytest

from oracle import hc as OH
from oracle.route import round_to


def layer(rng, T, hc, D, R, inject=True, dtype="float32"):
    HD = hc * D
    before = round_to(rng.standard_normal((T, HD)), dtype)
    out = round_to(rng.standard_normal((T, D)), dtype)
    inject_in = round_to(2 * rng.random((T, hc)), dtype)
    norm = round_to(1 + 0.2 * rng.standard_normal(HD), dtype)
    down = round_to(rng.standard_normal((R, HD)) / np.sqrt(HD), dtype)
    up = round_to(rng.standard_normal((HD, R)) / np.sqrt(R), dtype)
    inject_w = round_to(rng.standard_normal((hc, HD)) / np.sqrt(HD), dtype) if inject else None
    return before, out, inject_in, norm, down, up, inject_w


def float64(before, out, inject_in, norm, down, up, inject_w, hc, eps):
    """The reference kernels' arithmetic, all in float64."""
    T, HD = before.shape
    D = HD // hc
    b = before.astype(np.float64).reshape(T, hc, D)
    h = b + out.astype(np.float64)[:, None, :] * inject_in.astype(np.float64)[:, :, None]
    rms = 1.0 / np.sqrt(np.mean(h * h, axis=2) + eps)
    normed = (h * rms[:, :, None] * norm.astype(np.float64).reshape(1, hc, D)).reshape(T, HD)
    sig = lambda v: 1.0 / (1.0 + np.exp(-v))
    z = normed @ down.astype(np.float64).T / hc
    low = z * sig(z)
    g = low @ up.astype(np.float64).T
    mixed = np.sum((normed * sig(g)).reshape(T, hc, D), axis=1) / hc
    inject = 2 * sig(normed @ inject_w.astype(np.float64).T / hc) if inject_w is not None else inject_in
    return mixed, h.reshape(T, HD), inject


@pytest.mark.parametrize("T, hc, D, R, inject", [(1, 4, 96, 24, True), (5, 4, 96, 24, False), (3, 2, 128, 16, True),
                                                  (8, 4, 256, 32, True)])
def test_the_oracle_is_the_formulas_in_float64(T, hc, D, R, inject):
    rng = np.random.default_rng(T * 100 + D)
    args = layer(rng, T, hc, D, R, inject)
    got = OH.fused_residual(*args, hc, 1e-6, "float32")
    want = float64(*args, hc, 1e-6)
    for g, w in zip(got, want):
        np.testing.assert_allclose(g, w, rtol=2e-5, atol=2e-6)


def test_nothing_before_is_a_plain_read():
    """out = 0 and inject_in = 0 (fused.py's own test): the residual is `before`, bit for bit."""
    rng = np.random.default_rng(1)
    before, _, _, norm, down, up, inject_w = layer(rng, 2, 4, 96, 24, True, "float16")
    out, inject_in = np.zeros((2, 96), np.float32), np.zeros((2, 4), np.float32)
    mixed, residual, inject = OH.fused_residual(before, out, inject_in, norm, down, up, inject_w, 4, 1e-6,
                                                "float16")
    assert np.array_equal(residual, before)


def test_zero_weights_leave_half_the_streams_mean():
    """down, inject and up all zero: z = 0, so low = 0 and inject = 2 sigmoid(0) = 1 exactly; every gate is
    sigmoid(0) = 1/2, so mixed = the streams' mean of normed, halved."""
    rng = np.random.default_rng(2)
    before, out, inject_in, norm, down, up, inject_w = layer(rng, 3, 4, 64, 16)
    zero = (np.zeros_like(down), np.zeros_like(up), np.zeros_like(inject_w))
    low, inject = OH.hc_down(OH.hc_norm(before, out, inject_in, norm, 4, 1e-6, "float32")[1], zero[0], zero[2], 4,
                             "float32")
    assert np.array_equal(low, np.zeros_like(low)) and np.array_equal(inject, np.ones_like(inject))
    mixed, residual, _ = OH.fused_residual(before, out, inject_in, norm, *zero, 4, 1e-6, "float32")
    _, normed = OH.hc_norm(before, out, inject_in, norm, 4, 1e-6, "float32")
    np.testing.assert_allclose(mixed, 0.5 * normed.reshape(3, 4, 64).mean(axis=1), rtol=1e-6, atol=1e-7)


def test_a_constant_stream_normalizes_to_its_sign():
    """h constant c_s over a stream: mean(h^2) = c_s^2, so with eps = 0 normed = sign(c_s) * norm."""
    hc, D = 4, 128
    c = np.array([3.0, -0.25, 7.5, -2.0], np.float32)
    before = np.repeat(c, D)[None, :].astype(np.float32)
    norm = np.linspace(0.5, 1.5, hc * D).astype(np.float32)
    residual, normed = OH.hc_norm(before, np.zeros((1, D), np.float32), np.zeros((1, hc), np.float32), norm, hc,
                                  0.0, "float32")
    np.testing.assert_allclose(normed[0], np.repeat(np.sign(c), D) * norm, rtol=2e-7)
    # eps enters under the root, beside the mean: c = 1, eps = 3 gives a scale of exactly 1/2
    _, half = OH.hc_norm(np.ones((1, hc * D), np.float32), np.zeros((1, D), np.float32),
                         np.zeros((1, hc), np.float32), np.ones(hc * D, np.float32), hc, 3.0, "float32")
    assert np.array_equal(half, np.full((1, hc * D), 0.5, np.float32))


def test_one_hot_rows_pick_single_products():
    """A down row that is a times the unit vector at k gives z = a normed_k / HC and low = z sigmoid(z); an inject
    row the same through 2 sigmoid; an up row b e_r gives the gate b low_r, so that column of a stream mixes in
    normed * sigmoid(b low_r) / HC."""
    rng = np.random.default_rng(3)
    T, hc, D, R = 2, 4, 64, 8
    before, out, inject_in, norm, _, _, _ = layer(rng, T, hc, D, R)
    _, normed = OH.hc_norm(before, out, inject_in, norm, hc, 1e-6, "float32")
    down = np.zeros((R, hc * D), np.float32)
    down[3, 77] = 2.5
    inject_w = np.zeros((hc, hc * D), np.float32)
    inject_w[1, 200] = -1.5
    low, inject = OH.hc_down(normed, down, inject_w, hc, "float32")
    z = 2.5 * normed[:, 77].astype(np.float64) / hc
    np.testing.assert_allclose(low[:, 3], z / (1 + np.exp(-z)), rtol=1e-6)
    assert np.array_equal(low[:, [0, 1, 2, 4, 5, 6, 7]], np.zeros((T, 7), np.float32))
    zi = -1.5 * normed[:, 200].astype(np.float64) / hc
    np.testing.assert_allclose(inject[:, 1], 2 / (1 + np.exp(-zi)), rtol=1e-6)
    up = np.zeros((hc * D, R), np.float32)
    up[2 * D + 5, 3] = 4.0  # stream 2, column 5
    mixed = OH.hc_up(normed, up, low, hc, "float32")
    gates = np.full((T, hc), 0.5)
    gates[:, 2] = 1 / (1 + np.exp(-4.0 * low[:, 3].astype(np.float64)))
    want = np.sum(normed.reshape(T, hc, D)[:, :, 5] * gates, axis=1) / hc
    np.testing.assert_allclose(mixed[:, 5], want, rtol=1e-6)


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
def test_a_token_gets_the_same_bits_alone_and_in_a_window(dtype):
    rng = np.random.default_rng(4)
    args = layer(rng, 6, 4, 96, 24, True, dtype)
    window = OH.fused_residual(*args, 4, 1e-6, dtype)
    for t in range(6):
        alone = OH.fused_residual(args[0][t:t + 1], args[1][t:t + 1], args[2][t:t + 1], *args[3:], 4, 1e-6, dtype)
        for a, w in zip(alone, window):
            assert np.array_equal(a, w[t:t + 1])
