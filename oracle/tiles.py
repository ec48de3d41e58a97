"""numpy restatement of the prompt path: pairs laid out in tiles of one expert, and the tile product.

Parity:
  * tiles_of — strata_mlx/blocks.py:539-563, with a stable sort (pairs of one expert keep their order).
    Pinned by the exact invariants of tests/test_blocks.py:177-195 and the layout blocks.py:549-557 fixes,
    checked in tests/test_oracle_route.py.
  * tile_matmul — blocks.py:465-536: out[p] = W[expert of p's tile] . a[p], the weights rounded to a's type,
    float32 sums; pinned against float64 products (tests/test_blocks.py:97-109, 2e-6 relative).
"""

import numpy as np

TOKENS_TILE = 16  # blocks.py:462


def tiles_of(indices: np.ndarray, experts: int):
    """-> (tile_expert (most,), token (most*16,), where (pairs,)), all int64; unused tiles name `experts`."""
    flat = np.asarray(indices).reshape(-1).astype(np.int64)
    k = np.asarray(indices).shape[-1] if np.asarray(indices).ndim else 1
    pairs = flat.size
    order = np.argsort(flat, kind="stable")
    expert = flat[order]
    counts = np.bincount(flat, minlength=experts)[:experts]
    tiles = (counts + TOKENS_TILE - 1) // TOKENS_TILE
    tile_end, pair_end = np.cumsum(tiles), np.cumsum(counts)
    slot = (tile_end - tiles)[expert] * TOKENS_TILE + np.arange(pairs) - (pair_end - counts)[expert]
    most = pairs // TOKENS_TILE + min(experts, pairs)
    token = np.zeros(most * TOKENS_TILE, dtype=np.int64)
    token[slot] = order // k
    where = np.zeros(pairs, dtype=np.int64)
    where[order] = slot
    tile_expert = (tile_end[None, :] <= np.arange(most)[:, None]).sum(axis=1)
    return tile_expert.astype(np.int64), token, where


def tile_matmul(w: np.ndarray, a: np.ndarray, tile_expert: np.ndarray, a_dtype: str) -> np.ndarray:
    """w float32 (E, rows, cols); a (P, cols) values in `a_dtype`; -> (P, rows) float64, rows of tiles that
    name no expert are NaN (the reference leaves them as whatever was in memory)."""
    from .route import round_to

    E = w.shape[0]
    wr = round_to(w, a_dtype).astype(np.float64)
    P = a.shape[0]
    out = np.full((P, w.shape[1]), np.nan)
    for t, e in enumerate(np.asarray(tile_expert)):
        if e < E:
            rows = slice(TOKENS_TILE * t, TOKENS_TILE * t + TOKENS_TILE)
            out[rows] = np.asarray(a[rows], np.float64) @ wr[e].T
    return out
