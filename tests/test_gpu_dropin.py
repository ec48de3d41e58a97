"""The drop-in's Python level on the GPU against the oracle: the routed MoE block called as the reference calls it
(`_Routed.__call__(x)` after `install_routers`, strata_mlx/fused.py:484-507) on the fused two-kernel path and on the
composition; prompts whose rows end inside a chunk of 256 columns (the reference model's ffn of 640) through the
tiles; many pairs of a plain expert product through the grouped GEMM; and the dense layers of dense.py."""

import numpy as np
import pytest
import torch

from conftest import rel_err
from oracle import blocks as OB
from oracle import dense as OD
from oracle import moe as OM
from oracle import route as OR
from oracle import tiles as OT
from strata_hip import blocks as SB
from strata_hip import dense as SD
from strata_hip import fused as SF
from strata_hip import synth

pytestmark = pytest.mark.gpu
TOL = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 1e-2}
NAME = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}


@pytest.mark.parametrize("kind", ["Q2_0", "IQ4_NL"])
@pytest.mark.parametrize("cols", [192, 320, 640])
def test_tile_product_with_a_partial_last_chunk(kind, cols, tables, dev):
    """Rows of 64-column blocks that end inside a chunk of 256: the chunk's missing columns contribute nothing."""
    shape = (4, 128, cols)
    rng = np.random.default_rng(cols)
    raw = synth.random_blocks(kind, 4 * 128, cols, rng)
    w = OB.dequantize(raw, kind, shape, tables)
    tiles = np.array([3, 0, 0, 2, 9, 1], dtype=np.int32)  # 9: no expert
    a = torch.from_numpy(rng.standard_normal((16 * len(tiles), cols)).astype(np.float32)).to(torch.bfloat16)
    got = SB.tile_matmul(torch.from_numpy(raw).to(dev), kind, shape, a.to(dev), torch.from_numpy(tiles).to(dev))
    want = OT.tile_matmul(w, a.float().numpy(), tiles, "bfloat16")
    real = ~np.isnan(want)
    assert np.abs(got.cpu().numpy()[real] - want[real]).max() <= 2e-6 * np.abs(want[real]).max()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_a_prompt_at_the_reference_models_shape(dtype, tables, dev):
    """d 2560, ffn 640 (bench/blocks_matvec.py:18), Q2_0, 256 tokens x top-10 of 64 experts: tiles, as the reference
    tiles it (down's rows of 640 end inside a chunk), against the reference's composition pair by pair."""
    E, D, F, T, K = 64, 2560, 640, 256, 10
    rng = np.random.default_rng(3)
    raws, ws = {}, {}
    for n, (r, c) in (("g", (F, D)), ("u", (F, D)), ("d", (D, F))):
        raws[n] = synth.random_blocks("Q2_0", E * r, c, rng, sigma=0.005)
        ws[n] = OB.dequantize(raws[n], "Q2_0", (E, r, c), tables)
    lin = {n: SB.BlockSwitchLinear(torch.from_numpy(raws[n]).to(dev), "Q2_0", (E,) + ws[n].shape[1:]) for n in raws}
    assert all(SB.tileable("Q2_0", l.output_dims, l.input_dims) for l in lin.values())
    idx = OR.top_k(rng.standard_normal((T, E)).astype(np.float32), K)
    x = torch.from_numpy(rng.standard_normal((T, D)).astype(np.float32)).to(dtype)
    got = SB.BlockSwitchGLU(lin["g"], lin["u"], lin["d"])(x.to(dev), torch.from_numpy(idx).to(dev))
    flat, xs = idx.reshape(-1), x.float().numpy().astype(np.float64)
    r = {n: OR.round_to(m, NAME[dtype]).astype(np.float64) for n, m in ws.items()}
    want = np.zeros((flat.size, D))
    for e in np.unique(flat):
        pairs = np.nonzero(flat == e)[0]
        g, u = xs[pairs // K] @ r["g"][e].T, xs[pairs // K] @ r["u"][e].T
        h = OR.round_to(g / (1 + np.exp(-g)) * u, NAME[dtype]).astype(np.float64)
        want[pairs] = h @ r["d"][e].T
    assert got.shape == (T, K, D)
    assert rel_err(got.float().cpu().numpy().reshape(-1, D), want) <= 1e-2


def test_many_pairs_of_one_product_go_through_the_grouped_gemm(tables, dev):
    """BlockSwitchLinear with more pairs than `unpack_from` (the reference's unpack + gather_mm route): the tiles,
    the weights rounded to x's type, float32 sums."""
    E, R, C, P = 16, 128, 512, 6000
    rng = np.random.default_rng(4)
    raw = synth.random_blocks("IQ3_S", E * R, C, rng)
    w = OB.dequantize(raw, "IQ3_S", (E, R, C), tables)
    lin = SB.BlockSwitchLinear(torch.from_numpy(raw).to(dev), "IQ3_S", (E, R, C))
    idx = rng.integers(0, E, (P, 1))
    x = torch.from_numpy(rng.standard_normal((P, 1, 1, C)).astype(np.float32)).to(torch.bfloat16)
    got = lin(x.to(dev), torch.from_numpy(idx).to(dev)).float().cpu().numpy().reshape(P, R)
    wr = OR.round_to(w, "bfloat16").astype(np.float64)
    want = np.einsum("prc,pc->pr", wr[idx[:, 0]], x.float().numpy().reshape(P, C).astype(np.float64))
    assert rel_err(got, want) <= 1e-2


class Linear(torch.nn.Module):
    def __init__(self, weight):
        super().__init__()
        self.weight = torch.nn.Parameter(weight, requires_grad=False)

    def forward(self, x):
        return (x.float() @ self.weight.float().T).to(x.dtype)


class MoEBlock(torch.nn.Module):
    """A block with mlx-lm SparseMoeBlock's attributes: a float16 router, routed experts as BlockSwitchGLU, a shared
    expert of block layers and its gate."""

    def __init__(self, router_w, switch_mlp, shared, shared_gate_w, k):
        super().__init__()
        self.gate = Linear(router_w)
        self.switch_mlp = switch_mlp
        self.shared_expert = shared
        self.shared_expert_gate = Linear(shared_gate_w[None])
        self.top_k = k

    def forward(self, x):
        raise AssertionError("not swapped")


@pytest.fixture(scope="module")
def moe_block(tables, dev):
    """512 experts, d 2048, ffn 512, Q2_0 (the benchmark's layer), random blocks made on the GPU."""
    E, D, F, K = 512, 2048, 512, 10
    shapes = {"gate": (E, F, D), "up": (E, F, D), "down": (E, D, F)}
    raw = {n: synth.random_blocks_gpu("Q2_0", s[0] * s[1], s[2], 90 + i, dev, sigma=0.01)
           for i, (n, s) in enumerate(shapes.items())}
    lin = {n: SB.BlockSwitchLinear(raw[n], "Q2_0", shapes[n]) for n in raw}
    sraw = {n: synth.random_blocks_gpu("Q2_0", s[1], s[2], 95 + i, dev, sigma=0.01)
            for i, (n, s) in enumerate(shapes.items())}
    shared = SF.SwiGLUExpert(*(SD.BlockLinear(sraw[n], "Q2_0", shapes[n][1:]) for n in ("gate", "up", "down")))
    gen = torch.Generator(device=dev)
    gen.manual_seed(99)
    router_w = (torch.randn((E, D), generator=gen, device=dev) * 0.05).to(torch.float16)
    sgw = (torch.randn(D, generator=gen, device=dev) * 0.05).to(torch.float16)
    block = MoEBlock(router_w, SB.BlockSwitchGLU(lin["gate"], lin["up"], lin["down"]), shared, sgw, K)

    def per_rows(name, rows, cols, stacks=raw):
        n = rows * OB.row_bytes("Q2_0", cols)
        return lambda e: stacks[name][e * n:(e + 1) * n].cpu().numpy()

    fetch = (per_rows("gate", F, D), per_rows("up", F, D), per_rows("down", D, F))
    sh = tuple(OB.dequantize(sraw[n].cpu().numpy(), "Q2_0", (1,) + shapes[n][1:], tables)
               for n in ("gate", "up", "down"))
    return block, fetch, sh, sgw


@pytest.mark.parametrize("tokens", [1, 4, 16])
def test_the_routed_block_after_install_routers(tokens, moe_block, tables, dev):
    """install_routers swaps the block's class; its call is then the router's product and the fused decode, and
    with the fused path off the reference's composition: both against the oracle from the router's own logits."""
    block, fetch, sh, sgw = moe_block
    SF.install_routers([type("L", (), {"mlp": block})()])
    assert isinstance(block, SF._RoutedCall) and isinstance(block.gate, SF.WindowLinear)
    E, D, F, K = 512, 2048, 512, 10
    gen = torch.Generator(device=dev)
    gen.manual_seed(tokens)
    x = torch.randn((1, tokens, D), generator=gen, device=dev).to(torch.float16)
    fused = block(x)
    assert block._fused_for(x) is not None and fused.shape == x.shape and fused.dtype == x.dtype
    logits = block.gate(x if block.gate.takes(x) else x.float()).reshape(tokens, E)  # as the block routes
    assert logits.dtype == torch.float32
    want, _, _ = OM.moe_decode_blocks(logits.cpu().numpy(), x.float().cpu().numpy()[0], K, fetch, ("Q2_0", "Q2_0"),
                                      (E, D, F), sh, sgw.float().cpu().numpy(), tables, "float16")
    assert rel_err(fused.float().cpu().numpy()[0], want) <= 1e-2
    SF.FUSED = False
    try:
        composed = block(x)
    finally:
        SF.FUSED = True
    assert rel_err(composed.float().cpu().numpy()[0], want) <= 1e-2
    assert rel_err(composed.float().cpu().numpy(), fused.float().cpu().numpy()) <= 1e-2


def test_a_routed_block_the_fused_path_does_not_take(tables, dev):
    """64 experts, d 512, ffn 256, IQ3_S routed, window of 3: MoEDecode's three-kernel shape through _Routed; a
    window of 20 tokens (more than the fused decode takes) through the composition."""
    E, D, F, K = 64, 512, 256, 4
    rng = np.random.default_rng(8)
    shapes = {"gate": (E, F, D), "up": (E, F, D), "down": (E, D, F)}
    raw = {n: synth.random_blocks("IQ3_S", s[0] * s[1], s[2], rng, sigma=0.002) for n, s in shapes.items()}
    w = {n: OB.dequantize(raw[n], "IQ3_S", shapes[n], tables) for n in raw}
    lin = {n: SB.BlockSwitchLinear(torch.from_numpy(raw[n]).to(dev), "IQ3_S", shapes[n]) for n in raw}
    sraw = {n: synth.random_blocks("IQ3_S", s[1], s[2], rng, sigma=0.002) for n, s in shapes.items()}
    sw = tuple(OB.dequantize(sraw[n], "IQ3_S", (1,) + shapes[n][1:], tables) for n in ("gate", "up", "down"))
    shared = SF.SwiGLUExpert(*(SD.BlockLinear(torch.from_numpy(sraw[n]).to(dev), "IQ3_S", shapes[n][1:])
                               for n in ("gate", "up", "down")))
    router_w = torch.from_numpy(rng.standard_normal((E, D)).astype(np.float32) * 0.05).to(torch.bfloat16)
    sgw = torch.from_numpy(rng.standard_normal(D).astype(np.float32) * 0.05).to(torch.bfloat16)
    block = SF._Routed(SF.WindowLinear(Linear(router_w.to(dev))), SB.BlockSwitchGLU(lin["gate"], lin["up"],
                       lin["down"]), shared, Linear(sgw[None].to(dev)), K)
    for tokens in (3, 20):
        x = torch.from_numpy(rng.standard_normal((1, tokens, D)).astype(np.float32)).to(torch.bfloat16).to(dev)
        got = block(x)
        assert (block._fused_for(x) is not None) == (tokens <= 16)
        logits = (x.float() @ router_w.to(dev).float().T)[0] if tokens > 8 else block.gate(x)[0]
        # past a window the shared expert's block layers multiply weights unpacked to bf16 (dense.py:222-226)
        swr = sw if tokens <= SD.MAX_TOKENS else tuple(OR.round_to(m, "bfloat16") for m in sw)
        want, _, _ = OM.moe_decode(logits.cpu().numpy(), x.float().cpu().numpy()[0], K,
                                   (w["gate"], w["up"], w["down"]), swr, sgw.float().numpy(), "bfloat16")
        assert rel_err(got.float().cpu().numpy()[0], want) <= 1e-2


@pytest.mark.parametrize("kind", ["Q2_0", "IQ3_S", "Q3_K", "IQ4_XS"])
@pytest.mark.parametrize("tokens", [1, 8, 40])
def test_block_linear(kind, tokens, tables, dev):
    """dense.py:197-228: a window on the blocks, a prompt chunk on the weights unpacked to x's type."""
    R, C = 256, 1024
    rng = np.random.default_rng(tokens)
    raw = synth.random_blocks(kind, R, C, rng)
    w = OB.dequantize(raw, kind, (R, C), tables).astype(np.float64)
    layer = SD.BlockLinear(torch.from_numpy(raw).to(dev), kind, (R, C))
    x = torch.from_numpy(rng.standard_normal((1, tokens, C)).astype(np.float32)).to(torch.bfloat16)
    got = layer(x.to(dev))
    assert got.shape == (1, tokens, R) and got.dtype == torch.bfloat16
    wr = w if tokens <= SD.MAX_TOKENS else OR.round_to(w, "bfloat16").astype(np.float64)
    assert rel_err(got.float().cpu().numpy()[0], x.float().numpy()[0].astype(np.float64) @ wr.T) <= 1e-2


def test_block_linear_with_reordered_inputs(tables, dev):
    R, C = 64, 512
    rng = np.random.default_rng(5)
    raw = synth.random_blocks("Q2_0", R, C, rng)
    w = OB.dequantize(raw, "Q2_0", (R, C), tables).astype(np.float64)
    inputs = rng.permutation(C)  # input i of the layer sits at inputs[i] in the file's row
    layer = SD.BlockLinear(torch.from_numpy(raw).to(dev), "Q2_0", (R, C), inputs=inputs)
    x = rng.standard_normal((2, C)).astype(np.float32)
    got = layer(torch.from_numpy(x).to(dev)).cpu().numpy()
    want = x.astype(np.float64) @ w[:, inputs].T
    assert rel_err(got, want) <= 1e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("tokens", [1, 2, 3, 4, 5, 6, 7, 8, 24])
def test_scaled_linear(dtype, tokens, dev):
    """Q6_K as codes, scales and d (dense.py:109-167): a window on the three parts, a chunk on the floats."""
    R, C = 192, 768
    rng = np.random.default_rng(tokens)
    b = rng.integers(0, 256, (R * C // 256, 210), dtype=np.uint8)
    b[:, 208:210] = rng.uniform(-0.05, 0.05, (len(b), 1)).astype("<f2").view(np.uint8)
    layer = SD.ScaledLinear.from_blocks(b, R, C, dev)
    parts = OD.q6k_parts(b, R, C)
    x = torch.from_numpy(rng.standard_normal((tokens, C)).astype(np.float32)).to(dtype)
    got = layer(x.to(dev))
    assert got.dtype == dtype and got.shape == (tokens, R)
    if tokens <= SD.MAX_TOKENS:
        want = OD.scaled_matvec(*parts, x.float().numpy())
    else:
        want = x.float().numpy().astype(np.float64) @ OD.scaled_floats(*parts, NAME[dtype]).astype(np.float64).T
    assert rel_err(got.float().cpu().numpy(), want) <= TOL[dtype]
    floats = layer.floats(dtype).float().cpu().numpy()
    np.testing.assert_array_equal(floats, OD.scaled_floats(*parts, NAME[dtype]))  # one rounding, as the kernel


def test_block_embedding(tables, dev):
    V, Dm = 100, 512
    rng = np.random.default_rng(6)
    raw = synth.random_blocks("IQ4_XS", V, Dm, rng)
    table = OB.dequantize(raw, "IQ4_XS", (V, Dm), tables)
    emb = SD.BlockEmbedding(torch.from_numpy(raw).to(dev), "IQ4_XS", (V, Dm), torch.float16)
    ids = torch.tensor([[3, 99, 0, 3]], device=dev)
    got = emb(ids).cpu()
    assert got.shape == (1, 4, Dm) and got.dtype == torch.float16
    np.testing.assert_array_equal(got.float().numpy()[0], OR.round_to(table[[3, 99, 0, 3]], "float16"))
