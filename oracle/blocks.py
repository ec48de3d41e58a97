"""numpy restatement of strata-mlx's block formats and expert products (strata_mlx/blocks.py).

Dequantization follows the per-type `unpack32` bodies of `_UNPACK` (strata_mlx/blocks.py:57-194) with the
helpers of `_COMMON` (blocks.py:40-54). Every weight is an fp16 scale times small integer or dyadic factors
(at most 23 significant bits), so the float32 results here are exact and order-independent: the GPU's
dequantized weights must equal them bit for bit.

Parity:
  * Q2_0 — pinned by the closed form of tests/test_gguf.py:34-38 (also gguf.py:191-194).
  * Q3_K, IQ4_NL, IQ4_XS, IQ3_S (structure) — pinned against the second restatement in
    strata_mlx/gguf.py:182-276 (`to_affine`), re-expressed independently in tests/independent.py.
  * IQ3_XXS, IQ2_S, IQ2_XS, IQ2_XXS, IQ1_M (structure) — pinned against ggml's published scalar
    dequantizers (gguf-py 0.19.0 / ggml-quants), restated independently in tests/independent.py.
  * Codebook *content* for the six grid types — parity unpinned: the grids come from gguf-py, which is
    absent; every function takes the tables as data.
"""

import numpy as np

# type -> (weights per block, bytes per block): strata_mlx/blocks.py:36-38
BLOCK = {"IQ4_NL": (32, 18), "IQ4_XS": (256, 136), "IQ3_S": (256, 110), "IQ3_XXS": (256, 98),
         "IQ2_S": (256, 82), "IQ2_XS": (256, 74), "IQ2_XXS": (256, 66), "IQ1_M": (256, 56), "Q2_0": (64, 18),
         "Q3_K": (256, 110)}

# strata_mlx/gguf.py:34
KVALUES_IQ4NL = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], dtype=np.int16)

f32 = np.float32


def _f16(b: np.ndarray, at: int) -> np.ndarray:
    """The little-endian fp16 at byte `at` of every block, as float32 (blocks.py:41-43 `half_at`)."""
    return np.ascontiguousarray(b[:, at:at + 2]).view("<f2").astype(f32)[:, 0]


def _u16(b: np.ndarray, at: int) -> np.ndarray:
    return b[:, at].astype(np.uint32) | (b[:, at + 1].astype(np.uint32) << 8)


def _u32(b: np.ndarray, at: int) -> np.ndarray:
    return _u16(b, at) | (_u16(b, at + 2) << 16)


def _signed(values: np.ndarray, sign_bits: np.ndarray) -> np.ndarray:
    """values (..., m) times -1 where bit j of sign_bits (...) is set, j along the last axis."""
    j = np.arange(values.shape[-1], dtype=np.uint32)
    neg = (sign_bits[..., None].astype(np.uint32) >> j) & 1
    return np.where(neg == 1, -values, values)


# byte value -> its four codes less one, weight 4i + j from bits 2j..2j+1 of byte i
_Q2_CODES = (((np.arange(256, dtype=np.uint32)[:, None] >> (2 * np.arange(4, dtype=np.uint32))) & 3).astype(f32)
             - f32(1))


def _q2_0(b, t):  # blocks.py:58-68
    d = _f16(b, 0)
    codes = _Q2_CODES[b[:, 2:18]].reshape(len(b), 64)  # 16 bytes, byte i holds weights 4i..4i+3
    return d[:, None] * codes


def _iq4_nl(b, t):  # blocks.py:69-77
    d = _f16(b, 0)
    q = b[:, 2:18]
    kv = t["kvalues"].astype(f32)
    return d[:, None] * np.concatenate([kv[q & 15], kv[q >> 4]], axis=1)


def _iq4_xs(b, t):  # blocks.py:78-88
    n = len(b)
    d = _f16(b, 0)
    high = _u16(b, 2)
    kv = t["kvalues"].astype(f32)
    out = np.empty((n, 256), f32)
    for ib in range(8):
        ls = ((b[:, 4 + ib // 2].astype(np.uint32) >> (4 * (ib % 2))) & 15) | (((high >> (2 * ib)) & 3) << 4)
        dl = d * (ls.astype(f32) - f32(32))
        q = b[:, 8 + 16 * ib: 24 + 16 * ib]
        out[:, 32 * ib: 32 * ib + 32] = dl[:, None] * np.concatenate([kv[q & 15], kv[q >> 4]], axis=1)
    return out


def _iq3_s(b, t):  # blocks.py:89-102
    n = len(b)
    d = _f16(b, 0)
    grid = t["iq3s_grid"].reshape(512, 4).astype(f32)
    out = np.empty((n, 256), f32)
    for ib in range(8):
        db = d * (1 + 2 * ((b[:, 106 + ib // 2].astype(np.uint32) >> (4 * (ib % 2))) & 15)).astype(f32)
        high = b[:, 66 + ib].astype(np.uint32)
        for l in range(8):
            idx = b[:, 2 + 8 * ib + l].astype(np.uint32) | (((high >> l) & 1) << 8)
            sign = b[:, 74 + 4 * ib + l // 2].astype(np.uint32) >> (4 * (l % 2))
            v = db[:, None] * grid[idx]
            out[:, 32 * ib + 4 * l: 32 * ib + 4 * l + 4] = _signed(v, sign & 15)
    return out


def _iq3_xxs(b, t):  # blocks.py:103-116
    n = len(b)
    d = _f16(b, 0)
    grid = t["iq3xxs_grid"].reshape(256, 4).astype(f32)
    ksigns = t["ksigns"].astype(np.uint32)
    out = np.empty((n, 256), f32)
    for ib in range(8):
        aux = _u32(b, 66 + 4 * ib)
        db = d * (f32(0.5) + (aux >> 28).astype(f32)) * f32(0.5)
        for l in range(8):
            g = grid[b[:, 2 + 8 * ib + l]]
            sign = ksigns[(aux >> (7 * (l // 2))) & 127] >> (4 * (l % 2))
            out[:, 32 * ib + 4 * l: 32 * ib + 4 * l + 4] = _signed(db[:, None] * g, sign & 15)
    return out


def _iq2_s(b, t):  # blocks.py:117-131
    n = len(b)
    d = _f16(b, 0) * f32(0.25)
    grid = t["iq2s_grid"].reshape(1024, 8).astype(f32)
    out = np.empty((n, 256), f32)
    for ib in range(8):
        high = b[:, 66 + ib].astype(np.uint32)
        scales = b[:, 74 + ib].astype(np.uint32)
        for l in range(4):
            idx = b[:, 2 + 4 * ib + l].astype(np.uint32) | (((high >> (2 * l)) & 3) << 8)
            sign = b[:, 34 + 4 * ib + l].astype(np.uint32)
            dl = d * (f32(0.5) + (scales & 15 if l < 2 else scales >> 4).astype(f32))
            out[:, 32 * ib + 8 * l: 32 * ib + 8 * l + 8] = _signed(dl[:, None] * grid[idx], sign)
    return out


def _iq2_xs(b, t):  # blocks.py:132-147
    n = len(b)
    d = _f16(b, 0) * f32(0.25)
    grid = t["iq2xs_grid"].reshape(512, 8).astype(f32)
    ksigns = t["ksigns"].astype(np.uint32)
    out = np.empty((n, 256), f32)
    for ib in range(8):
        scales = b[:, 66 + ib].astype(np.uint32)
        for l in range(4):
            q = _u16(b, 2 + 2 * (4 * ib + l))
            dl = d * (f32(0.5) + (scales & 15 if l < 2 else scales >> 4).astype(f32))
            out[:, 32 * ib + 8 * l: 32 * ib + 8 * l + 8] = _signed(dl[:, None] * grid[q & 511], ksigns[q >> 9])
    return out


def _iq2_xxs(b, t):  # blocks.py:148-161
    n = len(b)
    d = _f16(b, 0)
    grid = t["iq2xxs_grid"].reshape(256, 8).astype(f32)
    ksigns = t["ksigns"].astype(np.uint32)
    out = np.empty((n, 256), f32)
    for ib in range(8):
        base = 2 + 8 * ib
        aux = _u32(b, base + 4)
        db = d * (f32(0.5) + (aux >> 28).astype(f32)) * f32(0.25)
        for l in range(4):
            g = grid[b[:, base + l]]
            out[:, 32 * ib + 8 * l: 32 * ib + 8 * l + 8] = _signed(db[:, None] * g, ksigns[(aux >> (7 * l)) & 127])
    return out


def _q3k_scales(s: np.ndarray) -> np.ndarray:
    """The sixteen 6-bit scales of Q3_K blocks less 32, (n, 16) (blocks.py:49-53 `q3k_scale`)."""
    out = np.empty((len(s), 16), f32)
    for k in range(16):
        p, word = k % 4, k // 4
        low = (s[:, 4 * word + p] & 15) if word < 2 else (s[:, 4 * (word - 2) + p] >> 4)
        high = (s[:, 8 + p].astype(np.uint32) >> (2 * word)) & 3
        out[:, k] = (low.astype(np.int32) | (high.astype(np.int32) << 4)) - 32
    return out


def _q3_k(b, t):  # blocks.py:164-175
    n = len(b)
    d = _f16(b, 108)
    sc = _q3k_scales(b[:, 96:108])
    out = np.empty((n, 256), f32)
    hmask = b[:, 0:32].astype(np.int32)
    for r in range(8):
        q = b[:, 32 + 32 * (r // 4): 64 + 32 * (r // 4)].astype(np.int32)
        v = ((q >> (2 * (r % 4))) & 3) - np.where((hmask >> r) & 1 == 1, 0, 4)
        s0, s1 = d * sc[:, 2 * r], d * sc[:, 2 * r + 1]
        scale = np.concatenate([np.repeat(s0[:, None], 16, 1), np.repeat(s1[:, None], 16, 1)], axis=1)
        out[:, 32 * r: 32 * r + 32] = scale * v.astype(f32)
    return out


def _iq1_m(b, t):  # blocks.py:177-193 (the table holds the grid's -1, 0, 1 as 0, 1, 2: blocks.py:286)
    n = len(b)
    w = [_u16(b, 48 + 2 * i) for i in range(4)]
    packed = (w[0] >> 12) | ((w[1] >> 8) & 0x00F0) | ((w[2] >> 4) & 0x0F00) | (w[3] & 0xF000)
    d = packed.astype(np.uint16).view("<f2").astype(f32)
    grid = t["iq1_grid"].reshape(2048, 8).astype(f32)
    out = np.empty((n, 256), f32)
    for ib in range(8):
        scales = w[ib // 2] >> (6 * (ib % 2))
        for l in range(4):
            high = (b[:, 32 + 2 * ib + l // 2].astype(np.uint32) >> (4 * (l % 2))) & 15
            idx = b[:, 4 * ib + l].astype(np.uint32) | ((high & 7) << 8)
            dl = d * (2 * ((scales >> (3 * (l // 2))) & 7) + 1).astype(f32)
            delta = np.where(high & 8, f32(-1.125), f32(-0.875)).astype(f32)
            out[:, 32 * ib + 8 * l: 32 * ib + 8 * l + 8] = dl[:, None] * (grid[idx] + delta[:, None])
    return out


_DECODE = {"Q2_0": _q2_0, "IQ4_NL": _iq4_nl, "IQ4_XS": _iq4_xs, "IQ3_S": _iq3_s, "IQ3_XXS": _iq3_xxs,
           "IQ2_S": _iq2_s, "IQ2_XS": _iq2_xs, "IQ2_XXS": _iq2_xxs, "Q3_K": _q3_k, "IQ1_M": _iq1_m}


def row_bytes(kind: str, cols: int) -> int:
    per_block, block_bytes = BLOCK[kind]
    if cols % per_block:
        raise ValueError(f"{kind}: rows of {cols} weights do not end on a block of {per_block}")
    return cols // per_block * block_bytes


def dequantize(blocks: np.ndarray, kind: str, shape: tuple, tables: dict) -> np.ndarray:
    """Every weight of `blocks` (uint8 bytes of a tensor of `shape`, rows along the last axis) as float32.

    strata_mlx/blocks.py:397-404 (`dequantize`, kernel `_DEQUANT` 261-270)."""
    per_block, block_bytes = BLOCK[kind]
    n = int(np.prod(shape)) // per_block
    b = np.asarray(blocks, dtype=np.uint8).reshape(-1)[: n * block_bytes].reshape(n, block_bytes)
    return _DECODE[kind](b, tables).astype(f32).reshape(shape)


def matvec(w: np.ndarray, idx: np.ndarray, x: np.ndarray, share: int) -> np.ndarray:
    """out[pair, r] = sum_c W[idx[pair], r, c] * x[pair // share, c], in float64 over exact weights.

    strata_mlx/blocks.py:196-220 (`_MATVEC`) and 407-436 (`BlockSwitchLinear.__call__`): the reference sums
    in float32; float64 here is the tolerance reference (tests/test_blocks.py:35-39)."""
    idx = np.asarray(idx).reshape(-1)
    xs = np.asarray(x, dtype=np.float64).reshape(-1, w.shape[-1])
    rows = xs[np.arange(len(idx)) // share]
    return np.einsum("prc,pc->pr", w[idx].astype(np.float64), rows)


def share_of(x_batch: tuple, indices_shape: tuple) -> int:
    """The reference's rule for how many pairs read one row of x (blocks.py:420-428); -1 = broadcast."""
    k = indices_shape[-1] if len(indices_shape) else 1
    if tuple(x_batch) == tuple(indices_shape):
        return 1
    if tuple(x_batch) == (*indices_shape[:-1], 1):
        return k
    return -1


def threads_per_row(runs: int) -> int:
    """blocks.py:303-308 — kept for the reference's launch rule; it fixes bits, not semantics."""
    p = 1
    while p < 32 and runs % (2 * p) == 0 and runs // (2 * p) >= 4:
        p *= 2
    return p
