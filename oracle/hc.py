"""Oracle (test infrastructure only): the hyper-connection read between two blocks, with the write of the block before
folded in — strata_mlx/fused.py:46-131 (`_NORM`, `_DOWN`, `_UP`) and 281-323 (`FusedResidual.__call__`).

For each token, HC streams of D each (the residual, HD = HC * D wide):
    h_s     = before_s + out * inject_in_s                      (float32; the residual is h rounded to the type)
    normed  = h_s * rsqrt(mean(h_s^2) + eps) * norm_s           (float32, a stream at a time)
    z_j     = (down_j . normed) / HC                            (rows j < R of `down`, then the inject rows)
    low_j   = z_j * sigmoid(z_j)        inject_s = 2 sigmoid(z_{R + s}), rounded to the type
    g_sc    = up_{s D + c} . low                                (R terms)
    mixed_c = sum_s normed_{s D + c} * sigmoid(g_sc) / HC       (rounded to the type)
Without inject rows, the inject returned is inject_in. Every sum in float32, whatever the weights' type.

Pinned by tests/test_oracle_hc.py: float64 evaluation of the same formulas on random inputs (to float32's
accuracy), and closed cases that a dropped term, factor or sign would break: nothing before is a plain read (the
residual is `before` bit for bit), zero down and inject weights give low = 0 and inject = 1 exactly and mixed = half
the streams' mean, a constant stream normalizes to its sign, one-hot weight rows pick out single products, and each
token's outputs do not depend on the other tokens of the window.
"""

import numpy as np

from .route import round_to

f32 = np.float32


def _dot(a, w):
    """a (T, K) . w (N, K)^T in float64, each output's sum taken the same way whatever T (no BLAS blocking)."""
    a, w = a.astype(np.float64), w.astype(np.float64)
    return np.stack([np.sum(w * row[None, :], axis=1) for row in a])


def _sigmoid(x):
    with np.errstate(over="ignore"):
        return (f32(1.0) / (f32(1.0) + np.exp(-x.astype(f32)))).astype(f32)


def hc_norm(before, out, inject_in, norm, hc: int, eps: float, dtype: str):
    """residual (T, HC * D) rounded to `dtype`, normed (T, HC * D) float32 (fused.py:46-70)."""
    T = before.shape[0]
    D = out.shape[1]
    b = before.astype(f32).reshape(T, hc, D)
    h = (b + out.astype(f32)[:, None, :] * inject_in.astype(f32)[:, :, None]).astype(f32)
    ms = (np.sum(h.astype(np.float64) ** 2, axis=2) / D).astype(f32)
    scale = (f32(1.0) / np.sqrt(ms + f32(eps))).astype(f32)
    normed = (h * scale[:, :, None] * norm.astype(f32).reshape(1, hc, D)).astype(f32)
    return round_to(h.reshape(T, hc * D), dtype), normed.reshape(T, hc * D)


def hc_down(normed, down, inject_w, hc: int, dtype: str):
    """low (T, R) float32 and inject (T, n_inject) rounded to `dtype` (fused.py:72-98)."""
    rows = down.astype(f32) if inject_w is None else np.concatenate([down, inject_w]).astype(f32)
    R = down.shape[0]
    z = (_dot(normed, rows).astype(f32) / f32(hc)).astype(f32)
    gate = _sigmoid(z)
    low = (z[:, :R] * gate[:, :R]).astype(f32)
    inject = round_to((f32(2.0) * gate[:, R:]).astype(f32), dtype)
    return low, inject


def hc_up(normed, up, low, hc: int, dtype: str):
    """mixed (T, D) rounded to `dtype` (fused.py:100-131)."""
    T, HD = normed.shape
    D = HD // hc
    g = _dot(low, up).astype(f32)  # (T, HD)
    part = (normed.astype(f32) * _sigmoid(g)).astype(f32).reshape(T, hc, D)
    mixed = (np.sum(part.astype(np.float64), axis=1).astype(f32) / f32(hc)).astype(f32)
    return round_to(mixed, dtype)


def fused_residual(before, out, inject_in, norm, down, up, inject_w, hc: int, eps: float, dtype: str):
    """(mixed (T, D), residual (T, HC * D), inject (T, HC)) as FusedResidual returns them (without the leading
    batch axis); inject is inject_in when there are no inject rows."""
    residual, normed = hc_norm(before, out, inject_in, norm, hc, eps, dtype)
    low, inject = hc_down(normed, down, inject_w, hc, dtype)
    mixed = hc_up(normed, up, low, hc, dtype)
    return mixed, residual, (inject if inject_w is not None else round_to(inject_in.astype(f32), dtype))
