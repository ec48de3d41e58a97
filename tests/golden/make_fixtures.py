"""Writes tests/golden/fixtures.npz: small seeded input / output vectors of the oracle (the reference restated on
the CPU), one group of arrays a function of the path. The reference's own tests regenerate their data from seeds
and commit no vectors; these pin the oracle against change and give the GPU tests fixed expectations.

    python tests/golden/make_fixtures.py      (from the repository root)

Synthetic codebooks (strata_hip.tables.synthetic(0)); their digest is stored beside the vectors."""

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [ROOT, os.path.join(ROOT, "strata-mlx_amd")]

from oracle import attention as OA  # noqa: E402
from oracle import blocks as OB  # noqa: E402
from oracle import moe as OM  # noqa: E402
from oracle import route as OR  # noqa: E402
from oracle import tiles as OT  # noqa: E402
from strata_hip import synth  # noqa: E402
from strata_hip import tables as T  # noqa: E402
from strata_hip.blocks import BLOCK  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "fixtures.npz")


def bf16_values(a: np.ndarray) -> np.ndarray:
    return OR.to_bf16(a.astype(np.float32))


def make() -> dict:
    tables = T.synthetic(0)
    f = {"tables_digest": np.array(T.digest(tables))}
    # dequantize: every kind, 2 rows x 256 weights
    for i, kind in enumerate(sorted(BLOCK)):
        rng = np.random.default_rng(100 + i)
        raw = synth.random_blocks(kind, 2, 256, rng, dist="uniform")
        f[f"dequant/{kind}/blocks"] = raw
        f[f"dequant/{kind}/weights"] = OB.dequantize(raw, kind, (2, 256), tables)
    # expert matvec (share 1), Q2_0 and IQ3_S, bf16 activations: 3 experts x 16 rows x 512
    for kind in ("Q2_0", "IQ3_S"):
        rng = np.random.default_rng(200 + len(kind))
        raw = synth.random_blocks(kind, 3 * 16, 512, rng)
        w = OB.dequantize(raw, kind, (3, 16, 512), tables)
        idx = np.array([2, 0, 2, 1, 1], dtype=np.int32)
        x = bf16_values(rng.standard_normal((5, 512)))
        f[f"matvec/{kind}/blocks"], f[f"matvec/{kind}/idx"], f[f"matvec/{kind}/x"] = raw, idx, x
        f[f"matvec/{kind}/out"] = OB.matvec(w, idx, x, 1).astype(np.float32)
    # top-k with ties, and the routing weights
    rng = np.random.default_rng(300)
    logits = rng.standard_normal((4, 64)).astype(np.float32)
    logits[1, 10] = logits[1, 20]
    logits[2, :] = 0.5
    idx = OR.top_k(logits, 10)
    f["topk/logits"], f["topk/idx"] = logits, idx.astype(np.int32)
    f["topk/weights"] = OR.routing_weights(logits, idx).astype(np.float32)
    # combine, bf16
    rng = np.random.default_rng(301)
    y = bf16_values(rng.standard_normal((3, 10, 64)) * 0.5)
    wl = rng.standard_normal((3, 10))
    wts = (np.exp(wl) / np.exp(wl).sum(-1, keepdims=True)).astype(np.float32)
    g = bf16_values(rng.standard_normal((3,)) * 2)
    s = bf16_values(rng.standard_normal((3, 64)) * 0.5)
    f["combine/y"], f["combine/w"], f["combine/g"], f["combine/s"] = y, wts, g, s
    f["combine/out"] = OR.moe_combine(y, wts, g, s, "bfloat16").astype(np.float32)
    # tiles of a small routing
    rng = np.random.default_rng(302)
    ind = rng.integers(0, 6, (1, 23, 3))
    ind[0, :8, 0] = 2
    te, tok, where = OT.tiles_of(ind, 6)
    f["tiles/indices"], f["tiles/tile_expert"], f["tiles/token"], f["tiles/where"] = (
        ind.astype(np.int32), te.astype(np.int32), tok.astype(np.int32), where.astype(np.int32))
    # paged decode attention: 37 positions in 3 shuffled pages (of 5), 3 queries, 4 / 2 heads of 128
    rng = np.random.default_rng(303)
    q = bf16_values(rng.standard_normal((3, 4, 128)))
    kp = bf16_values(rng.standard_normal((5, 2, 16, 128)))
    vp = bf16_values(rng.standard_normal((5, 2, 16, 128)))
    table = np.array([4, 0, 2], dtype=np.int32)
    f["paged/q"], f["paged/k"], f["paged/v"], f["paged/table"] = q, kp, vp, table
    f["paged/out"] = OA.paged_decode(q, kp, vp, table, 37, 0.0884).astype(np.float32)
    # one MoE block decode step: 8 experts, d 256, ffn 128, top 4, 2 tokens, Q2_0
    rng = np.random.default_rng(304)
    E, D, F, K = 8, 256, 128, 4
    raw = {n: synth.random_blocks("Q2_0", r, c, rng) for n, r, c in
           (("gate", E * F, D), ("up", E * F, D), ("down", E * D, F), ("sgate", F, D), ("sup", F, D),
            ("sdown", D, F))}
    shapes = {"gate": (E, F, D), "up": (E, F, D), "down": (E, D, F), "sgate": (1, F, D), "sup": (1, F, D),
              "sdown": (1, D, F)}
    w = {n: OB.dequantize(raw[n], "Q2_0", shapes[n], tables) for n in raw}
    x = bf16_values(rng.standard_normal((2, D)))
    lg = bf16_values(rng.standard_normal((2, E)))
    wg = bf16_values(rng.standard_normal(D) * 0.05)
    out, oidx, ow = OM.moe_decode(lg, x, K, (w["gate"], w["up"], w["down"]), (w["sgate"], w["sup"], w["sdown"]),
                                  wg, "bfloat16")
    for n in raw:
        f[f"moe/{n}"] = raw[n]
    f["moe/x"], f["moe/logits"], f["moe/shared_gate_w"] = x, lg, wg
    f["moe/out"], f["moe/idx"], f["moe/weights"] = out.astype(np.float32), oidx.astype(np.int32), ow.astype(np.float32)
    return f


if __name__ == "__main__":
    np.savez_compressed(OUT, **make())
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")
