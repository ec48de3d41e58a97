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


@pytest.mark.parametrize("kind", ["IQ3_S", "Q2_0"])
def test_long_runs_and_gaps_of_tiles(kind, tables, dev):
    """Runs of one expert longer than a unit of eight tiles, a run broken by a tile naming no expert, a run at the
    end: every real tile's rows against the oracle, the others left as they were."""
    shape = (3, 128, 512)
    raw, w, rng = stack(kind, *shape, 4, tables)
    tiles = np.array([0] * 19 + [3] + [0] * 3 + [2, 1, 1] + [7] * 2 + [1] * 9, dtype=np.int32)
    a = torch.from_numpy(rng.standard_normal((16 * len(tiles), shape[2])).astype(np.float32)).to(torch.bfloat16)
    got = SB.tile_matmul(torch.from_numpy(raw).to(dev), kind, shape, a.to(dev), torch.from_numpy(tiles).to(dev))
    want = OT.tile_matmul(w, a.float().numpy(), tiles, "bfloat16")
    real = ~np.isnan(want)
    assert real.any() and np.abs(got.cpu().numpy()[real] - want[real]).max() <= 2e-6 * np.abs(want[real]).max()


def prompt_want(wg, wu, wd, x, idx, dtype):
    """The reference's composition (strata_mlx/blocks.py:566-576) in float64 from the rounded weights: h =
    swiglu(gate . a, up . a) rounded to x's type, out = down . h rounded to x's type; pair by pair."""
    K = idx.shape[-1]
    flat, xs = idx.reshape(-1), x.float().numpy().astype(np.float64)
    r = {n: OR.round_to(m, dtype).astype(np.float64) for n, m in (("g", wg), ("u", wu), ("d", wd))}
    out = np.zeros((flat.size, wd.shape[1]))
    hs = np.zeros((flat.size, wg.shape[1]), dtype=np.float32)
    for e in np.unique(flat):
        pairs = np.nonzero(flat == e)[0]
        a = xs[pairs // K]
        g, u = a @ r["g"][e].T, a @ r["u"][e].T
        with np.errstate(over="ignore"):
            h = OR.round_to((g / (1.0 + np.exp(-g)) * u).astype(np.float32), dtype)
        hs[pairs] = h
        out[pairs] = h.astype(np.float64) @ r["d"][e].T
    return out, hs


@pytest.mark.parametrize("kind,dtype,T,E", [("IQ3_S", torch.bfloat16, 256, 64), ("Q2_0", torch.float16, 256, 64),
                                           ("IQ3_S", torch.bfloat16, 4096, 64)])
def test_the_prompt_layer_through_the_fused_products(kind, dtype, T, E, tables, dev):
    """switch_glu's prompt branch (gate / up / SwiGLU in one pass, down and the un-permutation in another) against
    the reference's composition pair by pair: Zipf(1.1) routing, top-10; 4096 tokens make more than one window
    of 2048 tiles. Within 1e-2 of the largest output (bfloat16 / float16), most much closer."""
    F, D, K = 256, 512, 10
    rng = np.random.default_rng(6)
    raws, ws = {}, {}
    for n, (r, c) in (("g", (F, D)), ("u", (F, D)), ("d", (D, F))):
        raws[n], ws[n], _ = stack(kind, E, r, c, 7 + len(raws), tables)
    lin = {n: SB.BlockSwitchLinear(torch.from_numpy(raws[n]).to(dev), kind, (E,) + ws[n].shape[1:]) for n in raws}
    logits = synth.zipf_logits(rng, T, E)
    idx = OR.top_k(logits.float().numpy(), K)
    x = torch.from_numpy(rng.standard_normal((T, D)).astype(np.float32)).to(dtype)
    got = SB.BlockSwitchGLU(lin["g"], lin["u"], lin["d"])(x.to(dev), torch.from_numpy(idx).to(dev))
    assert got.shape == (T, K, D) and got.dtype == dtype
    want, _ = prompt_want(ws["g"], ws["u"], ws["d"], x, idx, NAME[dtype])
    err = np.abs(got.float().cpu().numpy().reshape(-1, D) - want)
    scale = np.abs(want).max()
    assert err.max() <= 1e-2 * scale
    assert np.median(err) <= 2e-3 * scale


def test_the_fused_gate_up_is_swiglu_of_the_tile_products(tables, dev):
    """tile_glu against tile_matmul's two products and the reference's swiglu order (float32 swiglu, then
    rounded): equal but for the last bit of the rounding."""
    kind, E, F, D, T, K = "IQ3_S", 16, 128, 512, 64, 4
    rng = np.random.default_rng(8)
    raws = {n: synth.random_blocks(kind, E * F, D, rng) for n in ("g", "u")}
    lin = {n: SB.BlockSwitchLinear(torch.from_numpy(raws[n]).to(dev), kind, (E, F, D)) for n in raws}
    idx = torch.from_numpy(rng.integers(0, E, (T, K)).astype(np.int32)).to(dev)
    x = torch.from_numpy(rng.standard_normal((T, D)).astype(np.float32)).to(torch.bfloat16).to(dev)
    te, token, where = SB.tiles_of(idx, E)
    h = SB.tile_glu(lin["g"], lin["u"], x, token, te)
    a = x[token.long()]
    g = SB.tile_matmul(lin["g"].blocks, kind, (E, F, D), a, te)
    u = SB.tile_matmul(lin["u"].blocks, kind, (E, F, D), a, te)
    want = (torch.nn.functional.silu(g) * u).to(torch.bfloat16)
    real = torch.zeros(h.shape[0], dtype=torch.bool, device=dev)
    real[where.long()] = True
    diff = (h[real].float() - want[real].float()).abs()
    assert diff.max().item() <= 2 ** -7 * want[real].float().abs().max().item()
    assert (diff == 0).float().mean().item() > 0.99


@pytest.mark.parametrize("kind", ["IQ3_S", "Q2_0", "Q3_K"])
def test_float32_activations_take_the_weights_exactly(kind, tables, dev):
    """tile_matmul with float32 activations (the weights exact, float32 sums) against float64 products, tiles in
    any order; tiles naming no expert are not compared."""
    shape = (3, 64, 512)
    raw, w, rng = stack(kind, *shape, 9, tables)
    tiles = np.array([2, 0, 3, 0, 1], dtype=np.int32)  # 3: no expert
    a = torch.from_numpy(rng.standard_normal((16 * len(tiles), shape[2])).astype(np.float32))
    got = SB.tile_matmul(torch.from_numpy(raw).to(dev), kind, shape, a.to(dev), torch.from_numpy(tiles).to(dev))
    assert got.dtype == torch.float32
    want = OT.tile_matmul(w, a.numpy(), tiles, "float32")
    real = ~np.isnan(want)
    assert np.abs(got.cpu().numpy()[real] - want[real]).max() <= 1e-5 * np.abs(want[real]).max()


def test_a_float32_prompt_through_the_tiles(tables, dev):
    """switch_glu's prompt branch in float32 (the reference tiles float16 and float32 prompts) against the
    composition pair by pair."""
    kind, E, F, D, T, K = "IQ3_S", 16, 256, 256, 256, 8
    rng = np.random.default_rng(10)
    raws, ws = {}, {}
    for n, (r, c) in (("g", (F, D)), ("u", (F, D)), ("d", (D, F))):
        raws[n], ws[n], _ = stack(kind, E, r, c, 20 + len(raws), tables)
    lin = {n: SB.BlockSwitchLinear(torch.from_numpy(raws[n]).to(dev), kind, (E,) + ws[n].shape[1:]) for n in raws}
    idx = OR.top_k(rng.standard_normal((T, E)).astype(np.float32), K)
    assert idx.size >= SB.TILES_FROM
    x = torch.from_numpy(rng.standard_normal((T, D)).astype(np.float32))
    got = SB.BlockSwitchGLU(lin["g"], lin["u"], lin["d"])(x.to(dev), torch.from_numpy(idx).to(dev))
    assert got.shape == (T, K, D) and got.dtype == torch.float32
    want, _ = prompt_want(ws["g"], ws["u"], ws["d"], x, idx, "float32")
    assert np.abs(got.cpu().numpy().reshape(-1, D) - want).max() <= 1e-4 * np.abs(want).max()


@pytest.mark.parametrize("kind, dtype", [("IQ3_S", torch.bfloat16), ("Q2_0", torch.float16)])
def test_shared_tiles_give_one_wave_a_tiles_bits(kind, dtype, tables, dev):
    """Experts' runs of 1-8 tiles (Zipf routing over few experts): the streamed products with a short run's tiles
    shared among waves (each wave some of the 64 rows) give the bits of one wave a tile, for tile_matmul, the fused
    gate / up + SwiGLU and the down pass, call after call."""
    from strata_hip import _lib

    E, F, D, T, K = 24, 256, 512, 96, 6
    rng = np.random.default_rng(12)
    raws = {n: torch.from_numpy(synth.random_blocks(kind, E * r, c, rng)).to(dev)
            for n, (r, c) in (("g", (F, D)), ("u", (F, D)), ("d", (D, F)))}
    lin = {n: SB.BlockSwitchLinear(raws[n], kind, (E, F, D) if n != "d" else (E, D, F)) for n in raws}
    idx = torch.from_numpy(OR.top_k(synth.zipf_logits(rng, T, E).float().numpy(), K)).to(dev)
    x = torch.from_numpy(rng.standard_normal((T, D)).astype(np.float32)).to(dtype).to(dev)
    te, token, where = SB.tiles_of(idx, E)
    runs = torch.bincount(te[te < E].long(), minlength=E)
    assert runs.max() >= 5 and (runs[runs > 0] <= 4).any()  # long and short runs both
    a = x[token.long()]
    valid = (te < E).repeat_interleave(16)
    lib = _lib.load()
    before = lib.sh_tiles_set_share(1)
    try:
        h = SB.tile_glu(lin["g"], lin["u"], x, token, te)
        shared = (SB.tile_matmul(raws["g"], kind, (E, F, D), a, te)[valid], h[valid],
                  SB.tile_down(lin["d"], h, te, where))
        torch.cuda.synchronize()
        lib.sh_tiles_set_share(0)
        alone = (SB.tile_matmul(raws["g"], kind, (E, F, D), a, te)[valid],
                 SB.tile_glu(lin["g"], lin["u"], x, token, te)[valid], SB.tile_down(lin["d"], h, te, where))
        torch.cuda.synchronize()
        lib.sh_tiles_set_share(1)
        again = SB.tile_glu(lin["g"], lin["u"], x, token, te)[valid]
    finally:
        lib.sh_tiles_set_share(before)
    assert torch.equal(shared[0], alone[0])
    assert torch.equal(shared[1].view(torch.int16), alone[1].view(torch.int16))
    assert torch.equal(shared[2].view(torch.int16), alone[2].view(torch.int16))
    assert torch.equal(again.view(torch.int16), shared[1].view(torch.int16))
