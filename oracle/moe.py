"""numpy restatement of one MoE block's decode step over GGUF block experts.

The composition follows fused.py:484-497 (`_Routed.__call__`): router logits -> top_k -> softmax of the chosen
logits -> routed experts through switch_glu (blocks.py:801-829; with bfloat16 activations the reference takes
the generic branch 819-829: gate and up products rounded to the activation type, mlx-lm swiglu, down rounded)
-> shared expert and its gate -> moe_combine (fused.py:448-481).

Products are float64 over the exact float32 weights; every value the reference keeps in the activation type is
rounded to it here. Tolerance against this: 1e-2 of max|want| for bfloat16 outputs. The composition is pinned in
tests/test_oracle_route.py on a two-expert block worked out by hand (top-1, and a top-2 tie ending in a bf16 tie).
"""

import numpy as np

from . import blocks as B
from . import route as R


def expert_products(w_gate, w_up, w_down, idx, x, dtype):
    """y[t, k] = down_e(swiglu(gate_e x_t, up_e x_t)) for e = idx[t, k], each stage rounded to `dtype`.

    w_* are float32 stacks (E, rows, cols); idx (T, K); x (T, d) in `dtype`. Returns (T, K, d)."""
    T, K = idx.shape
    flat = idx.reshape(-1)
    g = R.round_to(B.matvec(w_gate, flat, x, K), dtype)
    u = R.round_to(B.matvec(w_up, flat, x, K), dtype)
    h = R.swiglu(g, u, dtype)
    y = R.round_to(B.matvec(w_down, flat, h, 1), dtype)
    return y.reshape(T, K, -1)


def moe_decode(logits, x, k, stacks, shared, shared_gate, dtype="bfloat16"):
    """One MoE block for a window of T tokens.

    logits (T, E) in `dtype`; x (T, d) in `dtype`; stacks = (gate, up, down) float32 (E, ...);
    shared = (gate, up, down) float32 (1, ...); shared_gate (d,) in `dtype`. Returns (out, idx, w)."""
    logits32 = np.asarray(logits, np.float32)
    idx = R.top_k(logits32, k)
    w = R.routing_weights(logits32, idx)
    y = expert_products(*stacks, idx, x, dtype)
    zero = np.zeros((x.shape[0], 1), dtype=np.int64)
    s = expert_products(*shared, zero, x, dtype)[:, 0, :]
    g = R.round_to(np.asarray(x, np.float64) @ np.asarray(shared_gate, np.float64), dtype)
    return R.moe_combine(y, w, g, s, dtype), idx, w


def moe_decode_blocks(logits, x, k, fetch, kinds, dims, shared, shared_gate, tables, dtype="bfloat16"):
    """moe_decode over experts kept as GGUF blocks, dequantizing only the experts the window chooses (a layer of
    512 experts would be 6 GB of float32). fetch = (gate, up, down): callables giving expert e's uint8 blocks;
    kinds = (kind of gate / up, kind of down); dims = (E, d, f); shared = (gate, up, down) float32 (1, ...).
    Returns (out, idx, w)."""
    E, d, f = dims
    logits32 = np.asarray(logits, np.float32)
    idx = R.top_k(logits32, k)
    used = np.unique(idx)
    pos = np.zeros(E, dtype=np.int64)
    pos[used] = np.arange(used.size)

    def take(get, kind, rows, cols):
        part = np.concatenate([np.asarray(get(int(e)), np.uint8).reshape(-1) for e in used])
        return B.dequantize(part, kind, (used.size, rows, cols), tables)

    stacks = (take(fetch[0], kinds[0], f, d), take(fetch[1], kinds[0], f, d), take(fetch[2], kinds[1], d, f))
    w = R.routing_weights(logits32, idx)
    y = expert_products(*stacks, pos[idx], x, dtype)
    zero = np.zeros((x.shape[0], 1), dtype=np.int64)
    s = expert_products(*shared, zero, x, dtype)[:, 0, :]
    g = R.round_to(np.asarray(x, np.float64) @ np.asarray(shared_gate, np.float64), dtype)
    return R.moe_combine(y, w, g, s, dtype), idx, w
