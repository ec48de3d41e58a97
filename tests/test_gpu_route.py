"""Router product, top-k, the MoE combine and tiles_of on the GPU against the oracle."""

import numpy as np
import pytest
import torch

from conftest import rel_err
from oracle import route as OR
from oracle import tiles as OT
from strata_hip import blocks as SB
from strata_hip import fused as SF

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("tokens", [1, 3, 8, 40])
@pytest.mark.parametrize("ties", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_top_k_is_the_oracles_choice(tokens, ties, dtype, dev):
    """tests/test_fused.py:111-120: the k largest, largest first, ties to the lower index; and the routing
    weights, the softmax of the chosen logits."""
    rng = np.random.default_rng(tokens + 10 * ties)
    for _ in range(5):
        logits = rng.standard_normal((tokens, 512)).astype(np.float32)
        if ties:
            logits = np.round(logits * 4) / 4
        lt = torch.from_numpy(logits).to(dtype)
        idx, w = SF.top_k(lt.to(dev), 10, weights=True)
        want = OR.top_k(lt.float().numpy(), 10)
        np.testing.assert_array_equal(idx.cpu().numpy(), want)
        np.testing.assert_allclose(w.cpu().numpy(), OR.routing_weights(lt.float().numpy(), want), rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_top_k_takes_signed_zeros_as_equal(dtype, dev):
    """-0 and +0 compare equal in the reference's choice (fused.py:400-418: float comparisons, ties to the lower
    index): a row of signed zeros around the k-th place is chosen by index, not by sign."""
    rng = np.random.default_rng(5)
    logits = np.zeros((6, 96), dtype=np.float32)
    logits[:, :4] = rng.uniform(1, 2, (6, 4))
    logits[:, 40:] = -rng.uniform(1, 2, (6, 56))
    logits[:, 4:40] = np.where(rng.random((6, 36)) < 0.5, -0.0, 0.0)
    lt = torch.from_numpy(logits).to(dtype)
    for k in (6, 10, 20):
        idx, w = SF.top_k(lt.to(dev), k, weights=True)
        want = OR.top_k(lt.float().numpy(), k)
        np.testing.assert_array_equal(idx.cpu().numpy(), want)
        np.testing.assert_array_equal(want[:, 4:k], np.tile(np.arange(4, k), (6, 1)))  # zeros by index


@pytest.mark.parametrize("n, k", [(64, 1), (2048, 10), (96, 96), (100, 7)])
def test_top_k_shapes(n, k, dev):
    rng = np.random.default_rng(n)
    logits = rng.standard_normal((5, n)).astype(np.float32)
    idx = SF.top_k(torch.from_numpy(logits).to(dev), k)
    np.testing.assert_array_equal(idx.cpu().numpy(), OR.top_k(logits, k))


@pytest.mark.parametrize("tokens", [1, 3, 8, 16])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_moe_combine(tokens, dtype, dev):
    rng = np.random.default_rng(tokens)
    name = "float16" if dtype == torch.float16 else "bfloat16"
    y = torch.from_numpy(rng.standard_normal((tokens, 10, 2048)).astype(np.float32) * 0.5).to(dtype)
    wl = rng.standard_normal((tokens, 10))
    w = torch.from_numpy((np.exp(wl) / np.exp(wl).sum(-1, keepdims=True)).astype(np.float32))
    g = torch.from_numpy(rng.standard_normal((tokens, 1)).astype(np.float32) * 2).to(dtype)
    s = torch.from_numpy(rng.standard_normal((tokens, 2048)).astype(np.float32) * 0.5).to(dtype)
    got = SF.moe_combine(y.to(dev), w.to(dev), g.to(dev), s.to(dev)).cpu()
    want = OR.moe_combine(y.float().numpy(), w.numpy(), g.float().numpy()[:, 0], s.float().numpy(), name)
    gotf = got.float().numpy()
    # the reference's order and roundings: equal but where exp's last bit tips the gate's rounding
    assert (gotf == want).mean() > 0.999
    assert rel_err(gotf, want) <= 1e-2


@pytest.mark.parametrize("tokens", [1, 3, 8])
@pytest.mark.parametrize("wdtype", [torch.float16, torch.bfloat16])
def test_router_product(tokens, wdtype, dev):
    """tests/test_fused.py:91-106: float32 sums within 1e-5, and a token's bits the same alone or in a window."""
    rng = np.random.default_rng(tokens)
    w = torch.from_numpy(rng.standard_normal((48, 256)).astype(np.float32) * 0.1).to(wdtype)

    class Lin:
        weight = w.to(dev)

    router = SF.WindowLinear(Lin())
    x = torch.from_numpy(rng.standard_normal((1, tokens, 256)).astype(np.float32)).to(torch.bfloat16)
    got = router(x.to(dev)).cpu()
    assert got.dtype == torch.float32 and got.shape == (1, tokens, 48)
    want = x.float().numpy()[0].astype(np.float64) @ w.float().numpy().T.astype(np.float64)
    assert rel_err(got[0], want) <= 1e-5
    alone = torch.cat([router(x[:, t:t + 1].to(dev)).cpu() for t in range(tokens)], dim=1)
    assert torch.equal(alone, got)


@pytest.mark.parametrize("tokens, k, experts", [(211, 3, 7), (5, 2, 40), (64, 10, 512), (1, 1, 3), (2048, 10, 512)])
def test_tiles_hold_every_pair_with_its_expert(tokens, k, experts, dev):
    """tests/test_blocks.py:177-195, and the oracle's layout exactly (pairs of an expert in order)."""
    rng = np.random.default_rng(tokens)
    idx = rng.integers(0, experts, (1, tokens, k))
    idx[0, : tokens // 3] = 1
    if tokens >= 33 and experts > 4:
        idx[0, -33:, 0] = np.repeat([3, 4], [16, 17])
    tile_expert, token, where = (a.cpu().numpy() for a in SB.tiles_of(torch.from_numpy(idx).to(dev), experts))
    flat = idx.reshape(-1)
    assert len(tile_expert) * 16 == len(token) and len(where) == len(flat)
    assert len(set(where.tolist())) == len(flat)
    np.testing.assert_array_equal(tile_expert[where // 16], flat)
    np.testing.assert_array_equal(token[where], np.arange(len(flat)) // k)
    used = np.zeros(len(tile_expert), dtype=bool)
    used[where // 16] = True
    assert (tile_expert[~used] == experts).all() and (tile_expert[used] < experts).all()
    assert used.sum() == sum(-(-c // 16) for c in np.bincount(flat))
    want = OT.tiles_of(idx, experts)
    for got_a, want_a in zip((tile_expert, token, where), want):
        np.testing.assert_array_equal(got_a, want_a)
