"""numpy restatement of the Q2_0 table of sums (strata_mlx/blocks.py:579-771) — TEST INFRASTRUCTURE ONLY.

Two Q2_0 weights of a row are each (code - 1) times the block's scale, code 0..3: of two inputs a and b they make
one of 16 sums (c0 - 1) a + (c1 - 1) b, c = c0 | c1 << 2. The reference keeps those 16 sums of every input pair in
a table in the activations' type and multiplies a row by two lookups a code byte.

  * lookup_table — blocks.py:595-603 (`_TABLE`): entry c = OutT(float32((c & 3) - 1) a + ((c >> 2) - 1) b). The
    coefficients are -1, 0, 1, 2, so both products are exact and one float32 rounding of their sum precedes the
    rounding to OutT, as here.
  * lookup_table_glu — blocks.py:606-616 (`_TABLE_GLU`): the same table of silu(gate) * up computed in float32
    (not rounded to OutT before the table).
  * lookup_matvec — blocks.py:618-643 (`_LOOKUP`): out[pair, r] = sum over runs of d * sum of the run's lookups;
    float64 here over the table's rounded entries (the reference's float32 sums differ by their order only).
  * lookup_down_glu — blocks.py:702-760 (`_DOWN_GLU`): lookup_matvec over lookup_table_glu, one pair a row.

Pinned in tests/test_oracle_lookup.py: table entries against the exact sums within one rounding and on
hand-built ties, the products against the float64 product of the dequantized weights within the table's
rounding, and the code-to-entry order (a swapped order fails the product check).
"""

import numpy as np

from .route import round_to, sigmoid32

f32 = np.float32
_CA = (np.arange(16) & 3).astype(f32) - f32(1)  # coefficient of the first input of a pair
_CB = (np.arange(16) >> 2).astype(f32) - f32(1)  # of the second


def _table_of(a: np.ndarray, b: np.ndarray, dtype: str) -> np.ndarray:
    s = (_CA * a[..., None]).astype(f32) + (_CB * b[..., None]).astype(f32)
    return round_to(s.astype(f32), dtype)


def lookup_table(x: np.ndarray, dtype: str) -> np.ndarray:
    """x (n, cols) values of `dtype` -> (n, cols / 2, 16) float32 values of `dtype`."""
    x = np.asarray(x, f32)
    return _table_of(x[:, 0::2], x[:, 1::2], dtype)


def lookup_table_glu(gate: np.ndarray, up: np.ndarray, dtype: str) -> np.ndarray:
    """The table of silu(gate) * up, each input pair's silu products in float32."""
    g, u = np.asarray(gate, f32), np.asarray(up, f32)
    h = (g * sigmoid32(g)).astype(f32) * u
    h = h.astype(f32)
    return _table_of(h[:, 0::2], h[:, 1::2], dtype)


def lookup_matvec(blocks: np.ndarray, shape: tuple, idx: np.ndarray, table: np.ndarray, share: int) -> np.ndarray:
    """blocks: a Q2_0 stack of `shape` (experts, rows, cols) as bytes; table (n, cols / 2, 16); out (pairs, rows)
    float64: sum over blocks of d * sum of the table entries its codes name, for table row pair // share."""
    experts, rows, cols = shape
    b = np.asarray(blocks, np.uint8).reshape(experts, rows, cols // 64, 18)
    d = np.ascontiguousarray(b[..., :2]).view("<f2")[..., 0].astype(np.float64)  # (E, R, cols / 64)
    q = b[..., 2:].astype(np.int64)  # byte i of a block: codes of weights 4i .. 4i + 3
    lo, hi = q & 15, q >> 4  # the entries of pairs 2i and 2i + 1 of the block
    idx = np.asarray(idx).reshape(-1)
    t = np.asarray(table, np.float64)
    out = np.empty((len(idx), rows))
    for p, e in enumerate(idx):
        tp = t[p // share].reshape(cols // 64, 32, 16)  # 32 pairs a block
        pair_lo = np.arange(16) * 2
        ent = (np.take_along_axis(tp[None, :, pair_lo, :], lo[e][..., None], axis=-1)[..., 0]
               + np.take_along_axis(tp[None, :, pair_lo + 1, :], hi[e][..., None], axis=-1)[..., 0])
        out[p] = (d[e] * ent.sum(axis=-1)).sum(axis=-1)
    return out


def lookup_down_glu(blocks: np.ndarray, shape: tuple, idx: np.ndarray, gate: np.ndarray, up: np.ndarray,
                    dtype: str) -> np.ndarray:
    return lookup_matvec(blocks, shape, idx, lookup_table_glu(gate, up, dtype), 1)
