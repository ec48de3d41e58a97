"""The oracle's Q6_K split (oracle/dense.py) and the library's host copy of it (strata_hip.dense.q6k_parts), pinned
against ggml's scalar dequantizer restated in tests/independent.py. CPU only."""

import numpy as np

import independent
from oracle import dense as OD
from strata_hip import dense as SD


def random_q6k(rng, rows, cols):
    b = rng.integers(0, 256, (rows * cols // 256, 210), dtype=np.uint8)
    b[:, 208:210] = rng.uniform(-0.05, 0.05, (len(b), 1)).astype("<f2").view(np.uint8)
    return b


def test_q6k_parts_are_ggmls_weights():
    rng = np.random.default_rng(1)
    rows, cols = 4, 512
    b = random_q6k(rng, rows, cols)
    parts = OD.q6k_parts(b, rows, cols)
    got = OD.scaled_weights(*parts).reshape(-1)
    want = independent.dequantize(b, "Q6_K", 210, None)
    np.testing.assert_array_equal(got, want)
    for mine, theirs in zip(SD.q6k_parts(b, rows, cols), parts):  # the library's host split is the same
        np.testing.assert_array_equal(mine, theirs)
    codes = parts[0]
    assert codes.min() >= -32 and codes.max() <= 31


def test_q6k_hand_made_block():
    """ql byte 0 = 0x21, qh byte 0 = 0b11100100: weight 0 = (1 | 0 << 4) - 32, weight 32 = (ql[32] & 15 | 1 << 4) - 32,
    weight 64 = (2 | 2 << 4) - 32, weight 96 = (ql[32] >> 4 | 3 << 4) - 32; scales 1, 2, 3, ...; d = 0.5."""
    b = np.zeros((1, 210), np.uint8)
    b[0, 0], b[0, 32], b[0, 128] = 0x21, 0x7A, 0b11100100
    b[0, 192:208] = np.arange(1, 17, dtype=np.int8).view(np.uint8)
    b[0, 208:210] = np.array([0.5], "<f2").view(np.uint8)
    w = OD.scaled_weights(*OD.q6k_parts(b, 1, 256))[0]
    assert w[0] == 0.5 * 1 * (1 - 32)
    assert w[32] == 0.5 * 3 * ((0xA | 1 << 4) - 32)  # run 1 of the half: scale index 2
    assert w[64] == 0.5 * 5 * ((2 | 2 << 4) - 32)
    assert w[96] == 0.5 * 7 * ((0x7 | 3 << 4) - 32)
    assert w[16] == 0.5 * 2 * (0 - 32)  # weights 16..31 take the second scale
    np.testing.assert_array_equal(w, independent.dequantize(b, "Q6_K", 210, None))


def test_scaled_floats_round_once_from_float32():
    rng = np.random.default_rng(2)
    parts = OD.q6k_parts(random_q6k(rng, 4, 256), 4, 256)
    exact = OD.scaled_weights(*parts)
    f32 = OD.scaled_floats(*parts, "float32").astype(np.float64)
    assert (np.abs(f32 - exact) <= 2.0 ** -24 * np.abs(exact)).all()
    bf = OD.scaled_floats(*parts, "bfloat16").astype(np.float64)
    assert (np.abs(bf - exact) <= 2.0 ** -8 * np.abs(exact) * 1.001).all()
