"""numpy restatement of the dense layers (strata_mlx/dense.py) — TEST INFRASTRUCTURE ONLY.

  * q6k_parts — strata_mlx/gguf.py:150-164: a Q6_K block (210 bytes: ql 128, qh 64, scales 16 int8, d fp16) as
    codes (six bits less 32), scales of 16 weights and d of 256. Pinned in tests/test_oracle_dense.py against
    ggml's published scalar dequantizer (dequantize_row_q6_K), restated independently in tests/independent.py.
  * scaled_weights — the weight code * scale * d in float64 (exact: at most 25 significant bits), and
    scaled_floats — as the reference's `_FLOATS` kernel rounds it (dense.py:72-82): s = d * scale in float32
    (exact), s * code rounded to float32, then to the output type.
  * scaled_matvec / block_matvec — float64 products over those weights (the reference sums in float32; the
    tolerance covers the order).
"""

import numpy as np

from .route import round_to


def q6k_parts(blocks: np.ndarray, rows: int, cols: int):
    b = np.asarray(blocks, np.uint8).reshape(-1, 210)
    ql, qh = b[:, :128].reshape(-1, 2, 64), b[:, 128:192].reshape(-1, 2, 32)
    hi = np.stack([(qh >> s) & 3 for s in (0, 2, 4, 6)], axis=2)
    lo = np.stack([ql[..., :32] & 15, ql[..., 32:] & 15, ql[..., :32] >> 4, ql[..., 32:] >> 4], axis=2)
    codes = ((lo | (hi << 4)).astype(np.int16) - 32).astype(np.int8)
    return (codes.reshape(rows, cols), np.ascontiguousarray(b[:, 192:208]).view(np.int8).reshape(rows, cols // 16),
            np.ascontiguousarray(b[:, 208:210]).view("<f2").reshape(rows, cols // 256))


def scaled_weights(codes, scales, d) -> np.ndarray:
    rows, cols = codes.shape
    step = cols // d.shape[1]
    s = np.repeat(scales.astype(np.float64), 16, axis=1) * np.repeat(d.astype(np.float64), step, axis=1)
    return codes.astype(np.float64) * s


def scaled_floats(codes, scales, d, dtype: str) -> np.ndarray:
    rows, cols = codes.shape
    step = cols // d.shape[1]
    s = (np.repeat(d.astype(np.float32), step, axis=1) * np.repeat(scales.astype(np.float32), 16, axis=1))
    return round_to((s.astype(np.float32) * codes.astype(np.float32)).astype(np.float32), dtype)


def scaled_matvec(codes, scales, d, x) -> np.ndarray:
    return np.asarray(x, np.float64) @ scaled_weights(codes, scales, d).T
