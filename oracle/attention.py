"""numpy restatement of decode attention over a cell list / page table (strata_mlx/attention.py).

The reference gathers each query's cells (`_cells` attention.py:132-141, `_gathered` 144-165) and runs SDPA with
the query heads that share a key head as that head's queries. A page table with pages of 16 is the same
contract with cells = page_table[pos // 16] * 16 + pos % 16 and a causal mask among the window's queries
(attention.py:118-129 for the mask's meaning: query t of S sees cells up to kv_len - S + t).

Parity: textbook softmax(q k^T * scale) v in float64 over the gathered keys and values; MLX SDPA's bits are not
reproduced (tolerance 1e-2 of max|want| for bfloat16 outputs, fp32 accumulation).
"""

import numpy as np


def sdpa(q, k, v, mask, scale):
    """q (M, D), k/v (L, D), mask (M, L) bool -> (M, D) float64."""
    s = (np.asarray(q, np.float64) @ np.asarray(k, np.float64).T) * scale
    s = np.where(mask, s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    p = np.exp(s - m)
    p = np.where(mask, p, 0.0)
    return (p / p.sum(axis=-1, keepdims=True)) @ np.asarray(v, np.float64)


def paged_decode(q, k_pages, v_pages, page_table, ctx_len, scale):
    """q (B, Hq, D); k/v pages (n_pages, Hkv, 16, D); page_table (>= ceil(ctx/16),) physical page ids.

    The window's B queries are the last B positions of a context of ctx_len cells; query t sees positions
    0 .. ctx_len - B + t. Returns (B, Hq, D) float64."""
    B, Hq, D = q.shape
    Hkv, P = k_pages.shape[1], k_pages.shape[2]
    group = Hq // Hkv
    pos = np.arange(ctx_len)
    phys = np.asarray(page_table)[pos // P]
    out = np.zeros((B, Hq, D))
    for g in range(Hkv):
        K = np.asarray(k_pages, np.float64)[phys, g, pos % P]
        V = np.asarray(v_pages, np.float64)[phys, g, pos % P]
        for t in range(B):
            visible = pos <= ctx_len - B + t
            rows = q[t, g * group:(g + 1) * group]
            out[t, g * group:(g + 1) * group] = sdpa(rows, K, V, np.broadcast_to(visible, (group, ctx_len)), scale)
    return out


def gathered(q, k, v, cells, real, scale):
    """attention.py:144-165: q (1, H, S, D), k/v (1, G, kv_len, D), cells/real (S, L) -> (1, S, H*D)."""
    _, H, S, D = q.shape
    G = k.shape[1]
    out = np.zeros((1, S, H * D))
    for s in range(S):
        for g in range(G):
            ks, vs = k[0, g, cells[s]], v[0, g, cells[s]]
            rows = q[0, g * (H // G):(g + 1) * (H // G), s]
            o = sdpa(rows, ks, vs, np.broadcast_to(real[s], (H // G, cells.shape[1])), scale)
            out[0, s, g * (H // G) * D:(g + 1) * (H // G) * D] = o.reshape(-1)
    return out


def qk_rope(x, w, cos, sin, heads, head_dim, stride, eps, dtype):
    """attention.py:183-222 (`qk_rope`, kernel `_QK_ROPE`): x (S, heads * stride), each head's head_dim values first;
    w (head_dim,); cos / sin (S, rot) -> (heads, S, head_dim) float32 values of `dtype`. Each head: rms norm (float32
    sum of squares, 1 / sqrt(mean + eps)), normed = T(w * T(x * inv)); then for j < rot: a = T(v c), b = T(o s),
    v = T(a + b) with o = -normed[j + rot/2] below rot/2, normed[j - rot/2] above."""
    from .route import round_to

    x = np.asarray(x, np.float32)
    S = x.shape[0]
    rot = np.asarray(cos).shape[-1]
    xs = x.reshape(S, heads, stride)[..., :head_dim].astype(np.float64)
    inv = 1.0 / np.sqrt((xs * xs).sum(axis=-1, keepdims=True) / head_dim + eps)
    normed = round_to(np.asarray(w, np.float32) * round_to((xs * inv).astype(np.float32), dtype), dtype)
    out = normed.copy()
    if rot:
        half = rot // 2
        other = np.concatenate([-normed[..., half:rot], normed[..., :half]], axis=-1)
        c = np.asarray(cos, np.float32)[:, None, :]
        s = np.asarray(sin, np.float32)[:, None, :]
        a = round_to((normed[..., :rot] * c).astype(np.float32), dtype)
        b = round_to((other * s).astype(np.float32), dtype)
        out[..., :rot] = round_to((a + b).astype(np.float32), dtype)
    return out.transpose(1, 0, 2)


def gate_out(out, gate, dtype):
    """attention.py:261: out * sigmoid(gate), the sigmoid rounded to the type, then the product."""
    from .route import round_to

    g = np.asarray(gate, np.float64)
    sig = round_to((1.0 / (1.0 + np.exp(-g))).astype(np.float32), dtype)
    return round_to((round_to(out, dtype) * sig).astype(np.float32), dtype)
