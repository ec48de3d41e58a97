"""The oracle's Q2_0 table of sums (oracle/lookup.py), pinned on the CPU: entries against the exact sums within one
rounding, hand-built entries (exact ones and a tie), and the products against the float64 product of the dequantized
weights within the table's rounding — a swapped code order or a dropped half of a byte fails it."""

import numpy as np
import pytest

from oracle import blocks as OB
from oracle import lookup as OL
from oracle import route as OR
from strata_hip import synth

U16 = 2.0 ** -11


def test_table_entries_are_the_sums_rounded_once():
    rng = np.random.default_rng(1)
    x = OR.round_to(rng.standard_normal((3, 256)), "float16")
    t = OL.lookup_table(x, "float16").astype(np.float64)
    a, b = x[:, 0::2].astype(np.float64), x[:, 1::2].astype(np.float64)
    c = np.arange(16)
    exact = ((c & 3) - 1)[None, None] * a[..., None] + ((c >> 2) - 1)[None, None] * b[..., None]
    assert (np.abs(t - exact) <= U16 * np.abs(exact) + 2.0 ** -25).all()
    np.testing.assert_array_equal(t[..., 5], 0)  # codes (1, 1): both weights zero
    np.testing.assert_array_equal(t[..., 6], a)  # (2, 1): a alone, exact
    np.testing.assert_array_equal(t[..., 9], b)  # (1, 2): b alone
    np.testing.assert_array_equal(t[..., 7], 2 * a)  # (3, 1): 2a, exact
    np.testing.assert_array_equal(t[..., 0], OR.round_to(-(a + b), "float16"))  # (0, 0): -(a + b), one rounding


def test_table_rounds_in_the_activations_type():
    # a = 1, b = 2^-12: a + b lies below half a float16 step of 1 (2^-11): entry (2, 2) rounds to 1; entry (3, 3),
    # 2 + 2^-11, to 2 as well; bf16 keeps neither
    x = np.array([[1.0, 2.0 ** -12]], np.float32)
    t = OL.lookup_table(x, "float16")[0, 0]
    assert t[10] == 1.0 and t[15] == 2.0 and t[9] == 2.0 ** -12
    x = np.array([[1.0, 1.0 + 2.0 ** -10]], np.float32)  # a + b = 2 + 2^-10: a float16 tie between 2 and 2 + 2^-9
    assert OL.lookup_table(x, "float16")[0, 0, 10] == 2.0  # to even


@pytest.mark.parametrize("share", [1, 2])
def test_lookup_product_is_the_weights_product_within_the_tables_rounding(share, tables):
    rng = np.random.default_rng(3)
    E, R, C = 3, 16, 512
    raw = synth.random_blocks("Q2_0", E * R, C, rng, dist="uniform")
    w = OB.dequantize(raw, "Q2_0", (E, R, C), tables).astype(np.float64)
    idx = np.array([2, 0, 1, 1])
    x = OR.round_to(rng.standard_normal((4 // share, C)), "float16")
    table = OL.lookup_table(x, "float16")
    got = OL.lookup_matvec(raw, (E, R, C), idx, table, share)
    want = OB.matvec(w, idx, x, share)
    # each lookup is off by at most half a float16 step of its entry; a row's error is at most sum |d| u |entry|
    d = np.abs(np.ascontiguousarray(raw.reshape(E, R, C // 64, 18)[..., :2]).view("<f2")[..., 0].astype(np.float64))
    xa = np.abs(x.astype(np.float64))
    pair_mag = 3 * (xa[:, 0::2] + xa[:, 1::2])  # |entry| <= 2|a| + 2|b| <= 3(|a| + |b|)
    bound = np.stack([(d[e][:, :, None] * pair_mag[p // share].reshape(C // 64, 32)[None]).sum(axis=(1, 2))
                      for p, e in enumerate(idx)]) * U16
    assert (np.abs(got - want) <= bound + 1e-9).all()
    # the table's rounding is visible: with float32 entries the product is the exact one
    exact = OL.lookup_matvec(raw, (E, R, C), idx, OL.lookup_table(x, "float32"), share)
    np.testing.assert_allclose(exact, want, rtol=1e-12, atol=1e-9 * np.abs(want).max())
    assert np.abs(got - want).max() > 0


def test_lookup_detects_a_swapped_code_order(tables):
    """Entries indexed with the two codes of a byte's half swapped would give another product."""
    rng = np.random.default_rng(4)
    raw = synth.random_blocks("Q2_0", 8, 256, rng, dist="uniform")
    w = OB.dequantize(raw, "Q2_0", (1, 8, 256), tables).astype(np.float64)
    x = rng.standard_normal((1, 256)).astype(np.float32)
    t = OL.lookup_table(x, "float32")
    swapped = t.reshape(1, 128, 4, 4).transpose(0, 1, 3, 2).reshape(1, 128, 16)
    want = OB.matvec(w, [0], x, 1)
    assert np.allclose(OL.lookup_matvec(raw, (1, 8, 256), [0], t, 1), want, rtol=1e-6, atol=1e-7)
    assert not np.allclose(OL.lookup_matvec(raw, (1, 8, 256), [0], swapped, 1), want, rtol=1e-3, atol=1e-3)


def test_glu_table_is_the_table_of_silu_times_up(tables):
    rng = np.random.default_rng(5)
    g = OR.round_to(2 * rng.standard_normal((2, 128)), "float16")
    u = OR.round_to(rng.standard_normal((2, 128)), "float16")
    t = OL.lookup_table_glu(g, u, "float16").astype(np.float64)
    h = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u.astype(np.float64)
    a, b = h[:, 0::2], h[:, 1::2]
    c = np.arange(16)
    exact = ((c & 3) - 1)[None, None] * a[..., None] + ((c >> 2) - 1)[None, None] * b[..., None]
    # float32 silu products (a few float32 roundings) then one float16 rounding
    assert (np.abs(t - exact) <= U16 * np.abs(exact) + 1e-6 * (np.abs(a) + np.abs(b))[..., None] + 2.0 ** -25).all()
    # the silu products enter unrounded: entry (2, 1) is h rounded once to float16, not swiglu's three roundings
    np.testing.assert_array_equal(t[..., 6], OR.round_to(OR.sigmoid32(g[:, 0::2]) * g[:, 0::2] * u[:, 0::2],
                                                          "float16"))
