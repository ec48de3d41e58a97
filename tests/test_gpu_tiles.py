"""The prompt path's grouped expert GEMM on the GPU (strata_mlx/blocks.py:465-536): tiles in any order, every
kind, the weights rounded to the activations' type; float32 sums within 2e-6 of max|want| as the reference's own
test asks (tests/test_blocks.py:97-109). And a prompt through the tiles against the oracle pair by pair."""

import numpy as np
import pytest
import torch

from oracle import blocks as OB
from oracle import moe as OM
from oracle import route as OR
from oracle import tiles as OT
from strata_hip import blocks as SB
from strata_hip import synth

pytestmark = pytest.mark.gpu

KINDS = sorted(SB.BLOCK)
NAME = {torch.float16: "float16", torch.bfloat16: "bfloat16"}


def stack(kind, experts, rows, cols, seed, tables):
    rng = np.random.default_rng(seed)
    raw = synth.random_blocks(kind, experts * rows, cols, rng)
    return raw, OB.dequantize(raw, kind, (experts, rows, cols), tables), rng


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_the_tile_product_is_the_product_with_the_weights(kind, dtype, tables, dev):
    shape = (4, 128, 512)
    raw, w, rng = stack(kind, *shape, 0, tables)
    tiles = np.array([3, 0, 0, 2, 3])  # tiles of 16 rows, each for one expert, in no particular order
    a = torch.from_numpy(rng.standard_normal((16 * len(tiles), shape[2])).astype(np.float32)).to(dtype)
    got = SB.tile_matmul(torch.from_numpy(raw).to(dev), kind, shape, a.to(dev),
                         torch.from_numpy(tiles.astype(np.int32)).to(dev)).cpu().numpy()
    want = OT.tile_matmul(w, a.float().numpy(), tiles, NAME[dtype])
    assert got.shape == want.shape and got.dtype == np.float32
    assert np.abs(got - want).max() <= 2e-6 * np.abs(want).max()


def test_tiles_naming_no_expert_are_left_as_they_were(tables, dev):
    shape = (3, 64, 256)
    raw, w, rng = stack("IQ3_S", *shape, 1, tables)
    tiles = np.array([1, 3, 0, 3, 2, 7], dtype=np.int32)  # 3 and 7: no expert
    a = torch.from_numpy(rng.standard_normal((16 * len(tiles), 256)).astype(np.float32)).to(torch.bfloat16)
    got = SB.tile_matmul(torch.from_numpy(raw).to(dev), "IQ3_S", shape, a.to(dev), torch.from_numpy(tiles).to(dev))
    want = OT.tile_matmul(w, a.float().numpy(), tiles, "bfloat16")
    real = ~np.isnan(want)
    assert np.abs(got.cpu().numpy()[real] - want[real]).max() <= 2e-6 * np.abs(want[real]).max()


@pytest.mark.parametrize("kind", ["IQ3_S", "Q2_0"])
def test_a_prompt_in_tiles_of_skewed_routing(kind, tables, dev):
    """C5's form at a smaller size: 256 tokens x top-10 of 64 experts under Zipf(1.1) popularity, d 2048 -> 512,
    tiles from tiles_of; every pair's row against the oracle."""
    E, R, C, T, K = 64, 512, 2048, 256, 10
    raw, w, rng = stack(kind, E, R, C, 3, tables)
    logits = synth.zipf_logits(rng, T, E)
    idx = OR.top_k(logits.float().numpy(), K)
    x = torch.from_numpy(rng.standard_normal((T, C)).astype(np.float32)).to(torch.bfloat16)
    te, token, where = SB.tiles_of(torch.from_numpy(idx).to(dev), E)
    a = x.to(dev)[token.long()]
    got = SB.tile_matmul(torch.from_numpy(raw).to(dev), kind, (E, R, C), a, te)[where.long()].cpu().numpy()
    wr = OR.round_to(w, "bfloat16").astype(np.float64)
    flat, xs = idx.reshape(-1), x.float().numpy().astype(np.float64)
    want = np.zeros((flat.size, R))
    for e in np.unique(flat):
        pairs = np.nonzero(flat == e)[0]
        want[pairs] = xs[pairs // K] @ wr[e].T
    assert np.abs(got - want).max() <= 2e-6 * np.abs(want).max()
