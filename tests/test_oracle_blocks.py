"""The oracle's block decoding, pinned: closed forms, hand-made blocks with known weights, and second restatements
from other texts (tests/independent.py). CPU only."""

import numpy as np
import pytest

import independent
from oracle import blocks as OB
from strata_hip import synth
from strata_hip.blocks import BLOCK

KINDS = sorted(BLOCK)


@pytest.mark.parametrize("kind", KINDS)
def test_oracle_matches_a_second_restatement(kind, tables):
    rng = np.random.default_rng(11)
    per_block, block_bytes = BLOCK[kind]
    raw = synth.random_blocks(kind, 3, 512, rng, dist="uniform")
    got = OB.dequantize(raw, kind, (3, 512), tables).reshape(-1)
    want = independent.dequantize(raw, kind, block_bytes, tables)
    assert got.dtype == np.float32
    np.testing.assert_array_equal(got.astype(np.float64), want)  # exact: no weight rounds in float32


@pytest.mark.parametrize("kind", KINDS)
def test_weights_are_exact_in_float32(kind, tables):
    """Every weight is an fp16 scale times factors of few bits: float32 holds it exactly, so the oracle's value
    equals the same computation in float64."""
    rng = np.random.default_rng(12)
    raw = synth.random_blocks(kind, 4, 256, rng, dist="uniform")
    w32 = OB.dequantize(raw, kind, (4, 256), tables).astype(np.float64).reshape(-1)
    w64 = independent.dequantize(raw, kind, BLOCK[kind][1], tables)
    assert np.array_equal(w32, w64)
    assert np.isfinite(w32).all() and np.abs(w32).max() > 0


def test_q2_0_closed_form(tables):
    """tests/test_gguf.py:34-38: weight 4i+j of a block is (((q[i] >> 2j) & 3) - 1) * d."""
    rng = np.random.default_rng(1)
    raw = synth.random_blocks("Q2_0", 5, 128, rng).reshape(-1, 18)
    d = raw[:, :2].copy().view("<f2").astype(np.float64)
    code = np.stack([(raw[:, 2:] >> s) & 3 for s in (0, 2, 4, 6)], axis=2).reshape(-1, 64)
    want = (code - 1.0) * d
    got = OB.dequantize(raw, "Q2_0", (5, 128), tables).reshape(-1, 64)
    np.testing.assert_array_equal(got, want)


def test_hand_made_blocks(tables):
    # Q2_0: d = 1, first byte codes 0, 1, 2, 3 -> -1, 0, 1, 2; the rest code 1 -> 0
    b = np.zeros(18, np.uint8)
    b[0:2] = np.array([1.0], "<f2").view(np.uint8)
    b[2] = 0b11100100
    b[3:] = 0b01010101
    w = OB.dequantize(b, "Q2_0", (1, 64), tables)[0]
    assert list(w[:4]) == [-1, 0, 1, 2] and (w[4:] == 0).all()
    # IQ4_NL: d = 0.5, byte i = i | (15 - i) << 4 -> 0.5 * kv[i], 0.5 * kv[15 - i]
    b = np.zeros(18, np.uint8)
    b[0:2] = np.array([0.5], "<f2").view(np.uint8)
    b[2:] = [i | ((15 - i) << 4) for i in range(16)]
    w = OB.dequantize(b, "IQ4_NL", (1, 32), tables)[0]
    kv = OB.KVALUES_IQ4NL
    assert list(w[:16]) == [0.5 * kv[i] for i in range(16)] and list(w[16:]) == [0.5 * kv[15 - i] for i in range(16)]
    # IQ3_S: d = 2, sub-block 0 scale nibble 3 -> db = 2 * 7 = 14; entry 0 index 5 with qh bit -> 261; signs 0b0101
    b = np.zeros(110, np.uint8)
    b[0:2] = np.array([2.0], "<f2").view(np.uint8)
    b[2] = 5
    b[66] = 1  # qh bit 0 -> index 256 + 5
    b[74] = 0b0101
    b[106] = 3
    g = tables["iq3s_grid"].reshape(512, 4).astype(int)
    w = OB.dequantize(b, "IQ3_S", (1, 256), tables)[0]
    assert list(w[:4]) == [-14 * g[261][0], 14 * g[261][1], -14 * g[261][2], 14 * g[261][3]]
    # Q3_K: all scale bits 0 except the first scale = 33 (-> +1); hmask bit 0 set for weight 0 (no -4); d = 1
    b = np.zeros(110, np.uint8)
    b[108:110] = np.array([1.0], "<f2").view(np.uint8)
    b[96] = 1       # low four bits of scale 0
    b[104] = 2      # high two bits of scale 0 (byte 8 + 0, bits 0-1) -> 1 | 2 << 4 = 33
    b[0] = 1        # weight 0: hmask bit r=0 set
    b[32] = 3       # weight 0: two bits = 3
    w = OB.dequantize(b, "Q3_K", (1, 256), tables)[0]
    assert w[0] == 3 * (33 - 32)
    assert w[1] == (0 - 4) * (33 - 32)  # no high bit: value 0 - 4, scale 1
    # scales 1..15 have raw value 0 -> -32; weight 16 (scale 1): value -4 -> 128
    assert w[16] == -4 * -32


def test_matvec_is_the_float64_product(tables):
    rng = np.random.default_rng(3)
    raw = synth.random_blocks("Q2_0", 3 * 8, 256, rng)
    w = OB.dequantize(raw, "Q2_0", (3, 8, 256), tables)
    x = rng.standard_normal((5, 256)).astype(np.float32)
    idx = np.array([2, 0, 1, 1, 2])
    got = OB.matvec(w, idx, x, 1)
    for p in range(5):
        np.testing.assert_allclose(got[p], w[idx[p]].astype(np.float64) @ x[p].astype(np.float64), rtol=1e-12)
    got2 = OB.matvec(w, idx[:4], x[:2], 2)  # share 2: pairs 0,1 read row 0, pairs 2,3 read row 1
    np.testing.assert_allclose(got2[3], w[idx[3]].astype(np.float64) @ x[1].astype(np.float64), rtol=1e-12)


def test_share_rule():
    assert OB.share_of((5, 2), (5, 2)) == 1
    assert OB.share_of((5, 1), (5, 2)) == 2
    assert OB.share_of((3,), (5, 2)) == -1


def test_row_bytes_rejects_partial_blocks():
    assert OB.row_bytes("IQ3_S", 2048) == 880 and OB.row_bytes("Q2_0", 2048) == 576
    with pytest.raises(ValueError):
        OB.row_bytes("IQ3_S", 640)


def test_ksigns_is_ggmls_published_table():
    """The sign table the IQ2_XS / IQ2_XXS / IQ3_XXS kinds read: the first 32 of the 128 entries of ggml's
    ksigns_iq2xs (ggml-common.h) as published, and every entry seven stored sign bits with an eighth making the
    count of set bits even (the property the decoders rely on: a group's signs are 7 bits in the block)."""
    from strata_hip import tables as T

    k = T.even_parity_signs()
    published = [0, 129, 130, 3, 132, 5, 6, 135, 136, 9, 10, 139, 12, 141, 142, 15,
                 144, 17, 18, 147, 20, 149, 150, 23, 24, 153, 154, 27, 156, 29, 30, 159]
    assert k.dtype == np.uint8 and k.shape == (128,)
    assert list(k[:32]) == published
    assert all((int(v) & 127) == i and bin(int(v)).count("1") % 2 == 0 for i, v in enumerate(k))
