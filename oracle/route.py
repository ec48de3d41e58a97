"""numpy restatement of the router's choice, SwiGLU and the MoE block's end (strata_mlx/fused.py, blocks.py).

Parity:
  * top_k — the order is a sort by (-value, index), i.e. `argpartition`'s stable order that
    tests/test_fused.py:111-120 checks (fused.py:400-418, ties to the lower index at 411). Pinned in
    tests/test_oracle_route.py against a brute-force sort, ties, equal rows and infinities included.
  * routing_weights — softmax over the chosen float32 logits (fused.py:491). Pinned against the full softmax
    renormalised over the chosen experts and closed forms (equal logits, e^ln3 : e^0).
  * swiglu — the rounding of blocks.py:222-237 (`_MATVEC_GLU`: sigmoid in float32 rounded to the
    activations' type, then two products in that type). Pinned against float64 silu(g)*u within three
    roundings and on closed cases (g = 0, sigma rounding to 1, sigma(1) in each type).
  * moe_combine — the order and roundings of fused.py:448-462 (`_COMBINE`), float32 scalar steps. Pinned
    against float64 sum_k y_k w_k + sigmoid(g) s within the documented roundings, and on hand-built cases
    that a left fold, a fused multiply-add or a missing rounding of the routed sum would change.
"""

import numpy as np

f32 = np.float32


def to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 (round to nearest even), returned as float32 values."""
    x = np.ascontiguousarray(np.asarray(x, dtype=f32))
    u = x.view(np.uint32).astype(np.uint64)
    nan = np.isnan(x)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(f32).reshape(x.shape)
    return np.where(nan, x, out).astype(f32)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float values to the activation type `dtype` ('float32', 'float16', 'bfloat16'), as float32."""
    x = np.asarray(x, dtype=f32)
    if dtype == "float32":
        return x
    if dtype == "float16":
        return x.astype(np.float16).astype(f32)
    if dtype == "bfloat16":
        return to_bf16(x)
    raise ValueError(dtype)


def top_k(logits: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest of each row (..., N), largest first, ties to the lower index.

    strata_mlx/fused.py:400-418 (`_TOPK`) and 424-436 (`top_k`)."""
    logits = np.asarray(logits, dtype=f32)
    n = logits.shape[-1]
    flat = logits.reshape(-1, n)
    out = np.empty((flat.shape[0], k), dtype=np.int64)
    order_idx = np.arange(n)
    for r, row in enumerate(flat):
        out[r] = np.lexsort((order_idx, -row.astype(np.float64)))[:k]
    return out.reshape(*logits.shape[:-1], k)


def routing_weights(logits: np.ndarray, idx: np.ndarray) -> np.ndarray:
    """softmax over the chosen float32 logits (fused.py:491, `mx.softmax(..., precise=True)`), float32."""
    chosen = np.take_along_axis(np.asarray(logits, dtype=np.float64), np.asarray(idx), axis=-1)
    e = np.exp(chosen - chosen.max(axis=-1, keepdims=True))
    return (e / e.sum(axis=-1, keepdims=True)).astype(f32)


def sigmoid32(x: np.ndarray) -> np.ndarray:
    """float32 sigmoid in the form blocks.py:232-234 uses: y = 1/(1+exp(|g|)); g<0 ? y : 1-y."""
    x = np.asarray(x, dtype=f32)
    with np.errstate(over="ignore"):  # exp(|g|) past float32's range: 1 / inf = 0, as the kernel's float32 gives
        y = (f32(1) / (f32(1) + np.exp(np.abs(x).astype(np.float64)).astype(f32))).astype(f32)
    return np.where(x < 0, y, (f32(1) - y)).astype(f32)


def swiglu(gate: np.ndarray, up: np.ndarray, dtype: str) -> np.ndarray:
    """silu(gate) * up with the roundings of blocks.py:222-237: sigma rounded to `dtype`, g*sigma rounded, *up
    rounded. gate/up are values already in `dtype`."""
    g = round_to(gate, dtype)
    u = round_to(up, dtype)
    sig = round_to(sigmoid32(g), dtype)
    a = round_to(g * sig, dtype)
    return round_to(a * u, dtype)


def moe_combine(y: np.ndarray, w: np.ndarray, g: np.ndarray, s: np.ndarray, dtype: str) -> np.ndarray:
    """out = OutT(sum_k y_k w_k) + OutT(OutT(sigmoid(g)) * s), in fused.py:448-462's order and roundings.

    y (T, K, D) in `dtype`, w (T, K) float32, g (T,) in `dtype`, s (T, D) in `dtype` -> (T, D). The experts
    are added as MLX's col_reduce_small adds them: row j of 8 takes k = j, j+8, ...; each product rounded
    before it is added (contract off); then the rows in order."""
    y = np.asarray(y, dtype=f32)
    w = np.asarray(w, dtype=f32)
    T, K, D = y.shape
    acc = np.zeros((T, D), f32)
    for j in range(min(8, K)):
        part = np.zeros((T, D), f32)
        for k in range(j, K, 8):
            prod = (y[:, k, :] * w[:, k][:, None]).astype(f32)
            part = (prod + part).astype(f32)
        acc = part if j == 0 else (part + acc).astype(f32)
    routed = round_to(acc, dtype)
    gate = round_to((f32(1) / (f32(1) + np.exp(-np.asarray(g, dtype=np.float64)).astype(f32))).astype(f32), dtype)
    shared = round_to(gate[:, None] * np.asarray(s, dtype=f32), dtype)
    return round_to(routed + shared, dtype)


def router_logits(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    """The router's product: float16/bfloat16 W (E, d) times x (T, d), float32 sums (fused.py:334-390)."""
    return (np.asarray(x, np.float64) @ np.asarray(w, np.float64).T).astype(f32)
