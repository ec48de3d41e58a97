"""The oracle's router choice, SwiGLU, combine, MoE composition and tiles, pinned on the CPU against what the
mathematics fixes: brute-force selection, the full softmax, float64 products within the documented roundings,
hand-built cases whose bits change under a plausible mistake (a left fold in place of the reference's order, a
fused multiply-add, a dropped term), a composition worked by hand, and the invariants of the reference's own tiles
test (tests/test_blocks.py:177-195). Nothing here compares the oracle with vectors it wrote itself."""

import math

import numpy as np
import pytest

from oracle import moe as OM
from oracle import route as OR
from oracle import tiles as OT

U = {"bfloat16": 2.0 ** -8, "float16": 2.0 ** -11}  # unit roundoff of the activation types


def brute_top_k(row, k):
    return sorted(range(len(row)), key=lambda j: (-float(row[j]), j))[:k]


# ---- top_k (strata_mlx/fused.py:400-418; order of argpartition, tests/test_fused.py:111-120)

@pytest.mark.parametrize("ties", [False, True])
@pytest.mark.parametrize("n, k", [(512, 10), (64, 8), (32, 1), (96, 32)])
def test_top_k_is_the_brute_force_order(n, k, ties):
    rng = np.random.default_rng(n + k + ties)
    logits = rng.standard_normal((12, n)).astype(np.float32)
    if ties:
        logits = np.round(logits * 4) / 4  # many equal values, ties at the k-th place included
    got = OR.top_k(logits, k)
    for r in range(len(logits)):
        assert got[r].tolist() == brute_top_k(logits[r], k)


def test_top_k_special_rows():
    eq = np.full((1, 64), 0.5, np.float32)
    assert OR.top_k(eq, 5)[0].tolist() == [0, 1, 2, 3, 4]  # all equal: the lowest indices, in order
    row = np.zeros((1, 8), np.float32)
    row[0, 6], row[0, 2], row[0, 5] = 3.0, 3.0, -1.0
    assert OR.top_k(row, 4)[0].tolist() == [2, 6, 0, 1]  # the tied maxima by index, then the tied zeros
    neg = -np.arange(16, dtype=np.float32)[None] - 1.0
    assert OR.top_k(neg, 3)[0].tolist() == [0, 1, 2]
    inf = np.array([[1.0, np.inf, -np.inf, 2.0]], np.float32)
    assert OR.top_k(inf, 4)[0].tolist() == [1, 3, 0, 2]
    zeros = np.array([[-0.0, 1.0, 0.0, -0.0, -1.0, 0.0]], np.float32)
    assert OR.top_k(zeros, 4)[0].tolist() == [1, 0, 2, 3]  # -0 and +0 equal (float comparisons): by index


# ---- routing weights (fused.py:491: softmax of the chosen float32 logits)

def test_routing_weights_are_the_full_softmax_renormalised():
    rng = np.random.default_rng(5)
    logits = (3 * rng.standard_normal((20, 512))).astype(np.float32)
    idx = OR.top_k(logits, 10)
    got = OR.routing_weights(logits, idx).astype(np.float64)
    full = np.exp(logits.astype(np.float64) - logits.max(axis=-1, keepdims=True))
    full /= full.sum(axis=-1, keepdims=True)
    chosen = np.take_along_axis(full, idx, axis=-1)
    want = chosen / chosen.sum(axis=-1, keepdims=True)
    np.testing.assert_allclose(got, want, rtol=2e-7, atol=1e-9)
    np.testing.assert_allclose(got.sum(axis=-1), 1.0, atol=1e-6)
    assert (np.diff(got, axis=-1) <= 0).all()  # the chosen are in descending order, so are their weights


def test_routing_weights_closed_forms():
    logits = np.array([[0.0, math.log(3.0), -50.0, 1.0]], np.float32)
    idx = np.array([[1, 0]])
    w = OR.routing_weights(logits, idx)[0]
    np.testing.assert_allclose(w, [0.75, 0.25], rtol=1e-6)  # e^ln3 : e^0
    assert OR.routing_weights(np.zeros((1, 8), np.float32), np.array([[3, 1, 7, 0]]))[0].tolist() == [0.25] * 4
    assert OR.routing_weights(logits, np.array([[2]]))[0].tolist() == [1.0]


# ---- swiglu (blocks.py:222-237: sigmoid rounded to the type, then g * sigma and * u, each rounded)

def test_sigmoid32_is_within_float32_rounding():
    x = np.linspace(-30, 30, 20001).astype(np.float32)
    want = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    got = OR.sigmoid32(x).astype(np.float64)
    assert (np.abs(got - want) <= 4 * 2.0 ** -24 * np.maximum(want, 2.0 ** -126) + 1e-30).all()
    assert OR.sigmoid32(np.float32([0.0]))[0] == 0.5


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_swiglu_is_silu_times_up_within_three_roundings(dtype):
    rng = np.random.default_rng(7)
    g = OR.round_to(4 * rng.standard_normal(4096), dtype)
    u = OR.round_to(rng.standard_normal(4096), dtype)
    got = OR.swiglu(g, u, dtype).astype(np.float64)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    want = g64 / (1 + np.exp(-g64)) * u64
    # sigma, g * sigma and the product each rounded once: relative u each, or half the type's smallest step where
    # a value is subnormal (sigma's absolute error carried by |g u|)
    half_step = 2.0 ** -134 if dtype == "bfloat16" else 2.0 ** -25
    bound = 3.01 * U[dtype] * np.abs(want) + half_step * (np.abs(g64 * u64) + np.abs(u64) + 1)
    assert (np.abs(got - want) <= bound).all()
    assert np.isin(got, OR.round_to(got, dtype)).all()  # results are values of the type


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_swiglu_closed_cases(dtype):
    u = OR.round_to(np.array([1.5, -3.0, 0.25], np.float32), dtype)
    assert (OR.swiglu(np.zeros(3, np.float32), u, dtype) == 0).all()  # silu(0) = 0
    big = np.full(3, 20.0, np.float32)  # sigma(20) rounds to 1 in both types: 20 * u exactly
    np.testing.assert_array_equal(OR.swiglu(big, u, dtype), OR.round_to(20.0 * u, dtype))
    small = np.full(3, -20.0, np.float32)  # |silu(-20)| = 20 e^-20 ~ 4e-8
    assert (np.abs(OR.swiglu(small, u, dtype)) <= 1e-7 * np.abs(u) + (6e-8 if dtype == "float16" else 0)).all()
    # sigma(1) = 0.7310586: bf16 0.73046875, fp16 0.73095703; g * sigma exact; then * 2 exact
    want = {"bfloat16": 0.73046875, "float16": 0.730957031}[dtype] * 2
    np.testing.assert_allclose(OR.swiglu(np.float32([1.0]), np.float32([2.0]), dtype), [want], rtol=1e-9)


# ---- moe_combine (fused.py:448-462: experts j, j + 8, ... a row, rows in order, each product rounded)

@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_combine_is_the_float64_sum_within_its_roundings(dtype):
    rng = np.random.default_rng(9)
    T, K, D = 6, 10, 512
    y = OR.round_to(0.5 * rng.standard_normal((T, K, D)), dtype)
    logits = rng.standard_normal((T, K)).astype(np.float32)
    w = np.exp(logits) / np.exp(logits).sum(axis=-1, keepdims=True)
    w = w.astype(np.float32)
    g = OR.round_to(2 * rng.standard_normal(T), dtype)
    s = OR.round_to(0.5 * rng.standard_normal((T, D)), dtype)
    got = OR.moe_combine(y, w, g, s, dtype).astype(np.float64)
    routed = np.einsum("tkd,tk->td", y.astype(np.float64), w.astype(np.float64))
    shared = 1 / (1 + np.exp(-g.astype(np.float64)))[:, None] * s.astype(np.float64)
    want = routed + shared
    u = U[dtype]
    bound = u * (np.abs(routed) + 2.01 * np.abs(shared) + np.abs(want)) + 1e-6 * np.abs(y).sum(axis=1).max()
    assert (np.abs(got - want) <= bound).all()
    # every term matters: leaving out expert 9 or the shared expert moves many outputs past the bound
    short = OR.moe_combine(y[:, :9], w[:, :9], g, s, dtype).astype(np.float64)
    assert (np.abs(short - want) > bound).mean() > 0.3


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_combine_adds_in_the_references_order(dtype):
    """K = 10, y all ones, w = [1, e x 7, -1, 0] with e = 2^-25: row 0 adds experts 0 and 8 first (1 - 1 = 0), then
    rows 1..7 add e each, so the sum is 7e. A left fold over k would add e to 1 seven times (each lost to rounding)
    before the -1 and give 0."""
    e = 2.0 ** -25
    y = np.ones((1, 10, 2), np.float32)
    w = np.array([[1.0] + [e] * 7 + [-1.0, 0.0]], np.float32)
    g = np.array([-30.0], np.float32)  # sigmoid(-30) ~ 1e-13: the shared term rounds to 0 times s = 0
    s = np.zeros((1, 2), np.float32)
    got = OR.moe_combine(y, w, g, s, dtype)
    want = OR.round_to(np.float32(7 * e), dtype)
    assert want != 0 and (got == want).all()
    fold = np.float32(0)
    for k in range(10):
        fold = np.float32(fold + np.float32(y[0, k, 0] * w[0, k]))
    assert fold == 0  # the order that must not be the one taken


def test_combine_rounds_each_product_before_it_adds():
    """Experts 0 and 8 meet first: y0 w0 = -(1 + 2^-7 + 2^-23) exactly, y8 w8 = (1 + 2^-7)(1 + 2^-23) = 1 + 2^-7 +
    2^-23 + 2^-30, whose float32 rounding drops the 2^-30. Rounded products cancel to 0; a fused multiply-add would
    keep 2^-30."""
    y = np.zeros((1, 10, 1), np.float32)
    w = np.zeros((1, 10), np.float32)
    y[0, 0, 0], w[0, 0] = -1.0, 1 + 2.0 ** -7 + 2.0 ** -23
    y[0, 8, 0], w[0, 8] = 1 + 2.0 ** -7, 1 + 2.0 ** -23
    got = OR.moe_combine(y, w, np.array([-30.0], np.float32), np.zeros((1, 1), np.float32), "bfloat16")
    assert got[0, 0] == 0.0
    assert np.float64(y[0, 8, 0]) * np.float64(w[0, 8]) + np.float64(y[0, 0, 0]) * np.float64(w[0, 0]) == 2.0 ** -30


def test_combine_rounds_the_routed_sum_and_the_shared_term_separately():
    """routed = 1 + 2^-9 (a bf16 tie: rounds to 1), shared = sigmoid(0) * 2^-8 = 2^-9 -> 1 + 2^-9 -> tie -> 1. Without
    the routed rounding the sum 1 + 2^-8 would be exact in bf16."""
    y = np.zeros((1, 1, 1), np.float32)
    y[0, 0, 0] = 1.0
    w = np.array([[1 + 2.0 ** -9]], np.float32)
    got = OR.moe_combine(y, w, np.zeros(1, np.float32), np.full((1, 1), 2.0 ** -8, np.float32), "bfloat16")
    assert got[0, 0] == 1.0


# ---- the MoE block's composition (fused.py:484-497 over switch_glu's bf16 branch), worked by hand

def _toy():
    """Two experts, d 2, ffn 1. x = [1, 2]. Expert 0: gate [0, 0] (g = 0, h = 0). Expert 1: gate [16, 0] (g = 16,
    sigma rounds to 1 in bf16, silu = 16), up [0.5, 0] (u = 0.5), h = 8, down [[0.25], [1]] -> y1 = [2, 8]. Shared:
    gate [1, 0] (g = 1, bf16 sigma(1) = 0.73046875 = silu), up [0, 1] (u = 2), h = 1.4609375, down [[1], [0]] ->
    s = [1.4609375, 0]; its gate weight [0, 0] -> sigmoid(0) = 0.5 -> 0.73046875 * [1, 0]."""
    gate = np.array([[[0.0, 0.0]], [[16.0, 0.0]]], np.float32)
    up = np.array([[[0.0, 0.0]], [[0.5, 0.0]]], np.float32)
    down = np.array([[[0.0], [0.0]], [[0.25], [1.0]]], np.float32)
    shared = (np.array([[[1.0, 0.0]]], np.float32), np.array([[[0.0, 1.0]]], np.float32),
              np.array([[[1.0], [0.0]]], np.float32))
    return (gate, up, down), shared, np.zeros(2, np.float32), np.array([[1.0, 2.0]], np.float32)


def test_moe_composition_by_hand_top1():
    stacks, shared, sgw, x = _toy()
    # logits favour expert 1: k = 1 -> weight 1; out = [2 + 0.73046875, 8] -> bf16 [2.734375, 8] (2.73046875 is
    # 174.75 steps of 2^-6 -> 175)
    out, idx, w = OM.moe_decode(np.array([[0.5, 1.0]], np.float32), x, 1, stacks, shared, sgw)
    assert idx.tolist() == [[1]] and w.tolist() == [[1.0]]
    assert out.tolist() == [[2.734375, 8.0]]


def test_moe_composition_by_hand_top2_tie():
    stacks, shared, sgw, x = _toy()
    # equal logits: experts [0, 1] by index, weights 0.5 each; routed = [1, 4]; out = [1.73046875, 4] -> bf16 tie
    # (221.5 steps of 2^-7) to even -> 1.734375
    out, idx, w = OM.moe_decode(np.array([[1.0, 1.0]], np.float32), x, 2, stacks, shared, sgw)
    assert idx.tolist() == [[0, 1]] and w.tolist() == [[0.5, 0.5]]
    assert out.tolist() == [[1.734375, 4.0]]


# ---- tiles_of: the invariants of the reference's test (tests/test_blocks.py:177-195)

@pytest.mark.parametrize("tokens, k, experts", [(211, 3, 7), (5, 2, 40), (64, 10, 512), (1, 1, 3), (2048, 10, 512)])
def test_tiles_hold_every_pair_with_its_expert(tokens, k, experts):
    rng = np.random.default_rng(tokens)
    idx = rng.integers(0, experts, (1, tokens, k))
    idx[0, : tokens // 3] = 1
    if tokens >= 33 and experts > 4:
        idx[0, -33:, 0] = np.repeat([3, 4], [16, 17])
    tile_expert, token, where = OT.tiles_of(idx, experts)
    flat = idx.reshape(-1)
    T = OT.TOKENS_TILE
    assert len(tile_expert) * T == len(token) and len(where) == len(flat)
    assert len(tile_expert) == len(flat) // T + min(experts, len(flat))
    assert len(set(where.tolist())) == len(flat)
    np.testing.assert_array_equal(tile_expert[where // T], flat)
    np.testing.assert_array_equal(token[where], np.arange(len(flat)) // k)
    used = np.zeros(len(tile_expert), dtype=bool)
    used[where // T] = True
    assert (tile_expert[~used] == experts).all() and (tile_expert[used] < experts).all()
    assert used.sum() == sum(-(-c // T) for c in np.bincount(flat))
    # the layout blocks.py:549-557 fixes: experts ascending, each expert's pairs in their order, tiles packed
    assert (np.diff(tile_expert) >= 0).all()
    for e in np.unique(flat):
        slots = where[flat == e]
        assert (np.diff(slots) == 1).all() and slots[0] % T == 0
