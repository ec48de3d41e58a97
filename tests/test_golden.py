"""The committed fixtures (tests/golden/fixtures.npz, written by tests/golden/make_fixtures.py from the oracle):
the oracle must still produce them exactly (CPU), and the HIP path must match them (GPU) — dequantized weights,
top-k and the tiles bit for bit, products within the path's tolerances."""

import os

import numpy as np
import pytest
import torch

from conftest import rel_err
from oracle import attention as OA
from oracle import blocks as OB
from oracle import moe as OM
from oracle import route as OR
from oracle import tiles as OT
from strata_hip import tables as T
from strata_hip.blocks import BLOCK

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fixtures.npz")


@pytest.fixture(scope="module")
def fx():
    with np.load(FIX, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_fixture_tables_are_the_synthetic_ones(fx, tables):
    assert str(fx["tables_digest"]) == T.digest(tables)


def test_oracle_reproduces_the_fixtures(fx, tables):
    for kind in sorted(BLOCK):
        np.testing.assert_array_equal(OB.dequantize(fx[f"dequant/{kind}/blocks"], kind, (2, 256), tables),
                                      fx[f"dequant/{kind}/weights"])
    for kind in ("Q2_0", "IQ3_S"):
        w = OB.dequantize(fx[f"matvec/{kind}/blocks"], kind, (3, 16, 512), tables)
        np.testing.assert_array_equal(OB.matvec(w, fx[f"matvec/{kind}/idx"], fx[f"matvec/{kind}/x"], 1)
                                      .astype(np.float32), fx[f"matvec/{kind}/out"])
    idx = OR.top_k(fx["topk/logits"], 10)
    np.testing.assert_array_equal(idx, fx["topk/idx"])
    np.testing.assert_array_equal(OR.routing_weights(fx["topk/logits"], idx).astype(np.float32), fx["topk/weights"])
    np.testing.assert_array_equal(OR.moe_combine(fx["combine/y"], fx["combine/w"], fx["combine/g"], fx["combine/s"],
                                                 "bfloat16").astype(np.float32), fx["combine/out"])
    for got, name in zip(OT.tiles_of(fx["tiles/indices"], 6), ("tile_expert", "token", "where")):
        np.testing.assert_array_equal(got, fx[f"tiles/{name}"])
    np.testing.assert_array_equal(OA.paged_decode(fx["paged/q"], fx["paged/k"], fx["paged/v"], fx["paged/table"],
                                                  37, 0.0884).astype(np.float32), fx["paged/out"])


@pytest.mark.gpu
def test_hip_path_matches_the_fixtures(fx, tables, dev):
    from strata_hip import attention as SA
    from strata_hip import blocks as SB
    from strata_hip import fused as SF

    for kind in sorted(BLOCK):
        got = SB.dequantize(torch.from_numpy(fx[f"dequant/{kind}/blocks"]).to(dev), kind, (2, 256), torch.float32)
        np.testing.assert_array_equal(got.cpu().numpy(), fx[f"dequant/{kind}/weights"])
    for kind in ("Q2_0", "IQ3_S"):
        x = torch.from_numpy(fx[f"matvec/{kind}/x"]).to(torch.bfloat16).to(dev)
        got = SB.switch_matvec(torch.from_numpy(fx[f"matvec/{kind}/blocks"]).to(dev), kind, (3, 16, 512),
                               torch.from_numpy(fx[f"matvec/{kind}/idx"]).to(dev), x, 1)
        assert rel_err(got.float().cpu(), fx[f"matvec/{kind}/out"]) <= 1e-2
    idx, w = SF.top_k(torch.from_numpy(fx["topk/logits"]).to(dev), 10, weights=True)
    np.testing.assert_array_equal(idx.cpu().numpy(), fx["topk/idx"])
    np.testing.assert_allclose(w.cpu().numpy(), fx["topk/weights"], rtol=2e-6, atol=1e-7)
    bf = lambda a: torch.from_numpy(a).to(torch.bfloat16).to(dev)  # noqa: E731
    got = SF.moe_combine(bf(fx["combine/y"]), torch.from_numpy(fx["combine/w"]).to(dev), bf(fx["combine/g"])[:, None],
                         bf(fx["combine/s"]))
    assert rel_err(got.float().cpu(), fx["combine/out"]) <= 1e-2
    te, tok, where = SB.tiles_of(torch.from_numpy(fx["tiles/indices"]).to(dev), 6)
    for got_a, name in zip((te, tok, where), ("tile_expert", "token", "where")):
        np.testing.assert_array_equal(got_a.cpu().numpy(), fx[f"tiles/{name}"])
    got = SA.paged_decode_attention(bf(fx["paged/q"]), bf(fx["paged/k"]), bf(fx["paged/v"]),
                                    torch.from_numpy(fx["paged/table"]).to(dev), 37, scale=0.0884)
    assert rel_err(got.float().cpu(), fx["paged/out"]) <= 1e-2
    E, D, F, K = 8, 256, 128, 4
    shapes = {"gate": (E, F, D), "up": (E, F, D), "down": (E, D, F), "sgate": (1, F, D), "sup": (1, F, D),
              "sdown": (1, D, F)}
    lin = {n: SB.BlockSwitchLinear(torch.from_numpy(fx[f"moe/{n}"]).to(dev), "Q2_0", shapes[n]) for n in shapes}
    # the block of 8 experts through the reference's composition (strata_mlx/fused.py:484-497): top-k, switch_glu
    # of the routed and of the shared expert, the shared gate's logit rounded to bf16, moe_combine
    x = bf(fx["moe/x"])
    oidx, ow = SF.top_k(bf(fx["moe/logits"]), K, weights=True)
    np.testing.assert_array_equal(oidx.cpu().numpy(), fx["moe/idx"])
    np.testing.assert_allclose(ow.cpu().numpy(), fx["moe/weights"], rtol=2e-6, atol=1e-7)
    y = SB.BlockSwitchGLU(lin["gate"], lin["up"], lin["down"])(x, oidx)
    zero = torch.zeros((x.shape[0], 1), dtype=torch.int32, device=dev)
    sh = SB.BlockSwitchGLU(lin["sgate"], lin["sup"], lin["sdown"])(x, zero)[:, 0, :]
    g = (x.float() @ bf(fx["moe/shared_gate_w"]).float()).to(torch.bfloat16)
    out = SF.moe_combine(y, ow, g[:, None], sh)
    assert rel_err(out.float().cpu(), fx["moe/out"]) <= 1e-2
