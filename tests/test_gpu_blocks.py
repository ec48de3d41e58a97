"""Block products on the GPU against the oracle: dequantized weights bit for bit, products within the path's
tolerances (1e-5 of max|want| with float32 activations, 1e-2 with bf16/fp16), for all ten kinds."""

import numpy as np
import pytest
import torch

from conftest import rel_err
from oracle import blocks as OB
from oracle import lookup as OL
from oracle import route as OR
from strata_hip import blocks as SB
from strata_hip import synth

pytestmark = pytest.mark.gpu

KINDS = sorted(SB.BLOCK)
TORCH = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}
TOL = {"float32": 1e-5, "float16": 1e-2, "bfloat16": 1e-2}


def stack(kind, experts, rows, cols, seed, tables):
    rng = np.random.default_rng(seed)
    raw = synth.random_blocks(kind, experts * rows, cols, rng)
    w = OB.dequantize(raw, kind, (experts, rows, cols), tables)
    return raw, w


def act(rng, shape, dtype):
    """activations already in `dtype`, as (torch CPU tensor, float32 numpy values)"""
    t = torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).to(TORCH[dtype])
    return t, t.float().numpy()


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
def test_dequantize_is_the_oracle_bit_for_bit(kind, dtype, tables, dev):
    raw, w = stack(kind, 3, 8, 512, 1, tables)
    got = SB.dequantize(torch.from_numpy(raw).to(dev), kind, (3, 8, 512), TORCH[dtype]).cpu()
    want = torch.from_numpy(w).to(TORCH[dtype])  # one rounding of the exact weights
    assert got.dtype == TORCH[dtype] and got.shape == want.shape
    assert torch.equal(got.view(torch.int16 if dtype != "float32" else torch.int32),
                       want.view(torch.int16 if dtype != "float32" else torch.int32))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("share", [1, 2])
def test_switch_matvec(kind, dtype, share, tables, dev):
    E, R, C = 5, 48, 512
    raw, w = stack(kind, E, R, C, 2, tables)
    rng = np.random.default_rng(3)
    idx = np.array([4, 0, 0, 2, 3, 3, 3, 1, 4, 2])  # repeats: tokens share experts
    x, xv = act(rng, (len(idx) // share, C), dtype)
    got = SB.switch_matvec(torch.from_numpy(raw).to(dev), kind, (E, R, C), torch.from_numpy(idx).to(dev),
                           x.to(dev), share)
    assert got.dtype == TORCH[dtype] and got.shape == (len(idx), R)
    want = OB.matvec(w, idx, xv, share)
    assert rel_err(got.float().cpu(), want) <= TOL[dtype]


@pytest.mark.parametrize("kind", ["Q2_0", "IQ3_S"])
@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("pairs", [1, 3, 16, 40, 80, 200])
def test_mfma_path_against_the_oracle(kind, dtype, pairs, tables, dev):
    """The MFMA decode path at decode shapes: 2048 columns, pairs grouped by expert (up to 128) or one a block,
    experts chosen by many tokens (more than a group holds) and by one."""
    E, R, C = 24, 64, 2048
    raw, w = stack(kind, E, R, C, 4, tables)
    rng = np.random.default_rng(pairs)
    idx = rng.integers(0, E, pairs)
    if pairs >= 40:
        idx[: pairs // 3] = 7  # one expert chosen by many tokens
    x, xv = act(rng, (pairs, C), dtype)
    got = SB.switch_matvec(torch.from_numpy(raw).to(dev), kind, (E, R, C), torch.from_numpy(idx).to(dev),
                           x.to(dev), 1)
    assert rel_err(got.float().cpu(), OB.matvec(w, idx, xv, 1)) <= TOL[dtype]


def test_a_pair_naming_no_expert_gets_zeros(tables, dev):
    E, R, C = 3, 32, 256
    raw, w = stack("Q2_0", E, R, C, 5, tables)
    idx = np.array([1, 7, 0, -2])
    x = torch.randn(4, C).to(torch.bfloat16)
    got = SB.switch_matvec(torch.from_numpy(raw).to(dev), "Q2_0", (E, R, C), torch.from_numpy(idx).to(dev),
                           x.to(dev), 1).float().cpu()
    assert (got[1] == 0).all() and (got[3] == 0).all()
    assert rel_err(got[[0, 2]], OB.matvec(w, idx[[0, 2]], x.float().numpy()[[0, 2]], 1)) <= 1e-2


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("per", [1, 2])
def test_block_switch_linear_share_modes(kind, per, tables, dev):
    """tests/test_blocks.py:22-39: a row to each token (gate/up) and a row to each pair (down)."""
    E, R, C = 3, 16, 512
    raw, w = stack(kind, E, R, C, 6, tables)
    layer = SB.BlockSwitchLinear(torch.from_numpy(raw).to(dev), kind, (E, R, C))
    idx = np.array([[2, 0], [1, 1], [0, 2], [2, 2], [0, 1]])
    rng = np.random.default_rng(7)
    x = rng.standard_normal((5, per, 1, C)).astype(np.float32)
    got = layer(torch.from_numpy(x).to(dev), torch.from_numpy(idx).to(dev)).cpu().numpy()
    assert got.shape == (5, 2, 1, R)
    xs = x[:, 0, 0] if per == 1 else x[:, :, 0]
    want = np.einsum("tkoi,ti->tko", w[idx], xs) if per == 1 else np.einsum("tkoi,tki->tko", w[idx], xs)
    assert rel_err(got[:, :, 0], want) <= 1e-5


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("tokens", [1, 3, 8])
def test_window_matvec(kind, tokens, tables, dev):
    raw, w = stack(kind, 1, 40, 512, 8, tables)
    rng = np.random.default_rng(9)
    x, xv = act(rng, (tokens, 512), "float32")
    got = SB.window_matvec(torch.from_numpy(raw).to(dev), kind, 40, 512, x.to(dev)).cpu()
    assert rel_err(got, xv.astype(np.float64) @ w[0].T.astype(np.float64)) <= 1e-5
    # a token's bits do not depend on the window it is in
    alone = torch.cat([SB.window_matvec(torch.from_numpy(raw).to(dev), kind, 40, 512, x[t:t + 1].to(dev)).cpu()
                       for t in range(tokens)])
    assert torch.equal(alone, got)


@pytest.mark.parametrize("kind", ["Q2_0", "IQ4_XS", "IQ1_M", "IQ3_S"])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
def test_matvec_separate(kind, dtype, tables, dev):
    E, R, C = 4, 24, 512
    raw, w = stack(kind, E, R, C, 10, tables)
    per = len(raw) // E
    experts = [torch.from_numpy(raw[e * per:(e + 1) * per].copy()).to(dev) for e in (2, 0, 3, 3)]
    rng = np.random.default_rng(11)
    x, xv = act(rng, (2, C), dtype)
    got = SB.matvec_separate(experts, kind, R, C, x.to(dev), 2).cpu()
    assert got.dtype == TORCH[dtype]
    assert rel_err(got.float(), OB.matvec(w, np.array([2, 0, 3, 3]), xv, 2)) <= TOL[dtype]


@pytest.mark.parametrize("kind", ["Q2_0", "IQ3_S", "IQ2_XS"])
@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
def test_matvec_glu_takes_swiglu_itself(kind, dtype, tables, dev):
    E, R, C = 4, 32, 256
    raw, w = stack(kind, E, R, C, 12, tables)
    rng = np.random.default_rng(13)
    idx = np.array([1, 3, 3, 0, 2])
    g, gv = act(rng, (5, C), dtype)
    u, uv = act(rng, (5, C), dtype)
    layer = SB.BlockSwitchLinear(torch.from_numpy(raw).to(dev), kind, (E, R, C))
    got = SB.matvec_glu(layer, torch.from_numpy(idx).to(dev), g.to(dev), u.to(dev)).float().cpu()
    h = OR.swiglu(gv, uv, dtype)
    assert rel_err(got, OB.matvec(w, idx, h, 1)) <= TOL[dtype]


@pytest.mark.parametrize("pairs", [1, 10, 30])
@pytest.mark.parametrize("rows, cols", [(256, 640), (96, 128), (40, 2048)])
def test_the_glu_table_built_in_down_gives_the_bits_of_its_own_kernel(pairs, rows, cols, tables, dev):
    """tests/test_blocks.py:215-229."""
    rng = np.random.default_rng(pairs + rows)
    raw = synth.random_blocks("Q2_0", 3 * rows, cols, rng, dist="uniform")
    down = SB.BlockSwitchLinear(torch.from_numpy(raw).to(dev), "Q2_0", (3, rows, cols))
    idx = torch.from_numpy(rng.integers(0, 3, pairs)).to(dev)
    gate = torch.from_numpy(rng.standard_normal((pairs, cols)).astype(np.float16)).to(dev)
    up = torch.from_numpy(rng.standard_normal((pairs, cols)).astype(np.float16)).to(dev)
    got = SB.lookup_down_glu(down, idx, gate, up)
    assert got is not None and got.dtype == torch.float16
    assert torch.equal(got, SB.lookup_matvec(down, idx, SB.lookup_table_glu(gate, up), 1))


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_lookup_table_is_the_oracles_bit_for_bit(dtype, dev):
    rng = np.random.default_rng(16)
    x, xv = act(rng, (3, 640), dtype)
    got = SB.lookup_table(x.to(dev)).float().cpu().numpy()
    np.testing.assert_array_equal(got, OL.lookup_table(xv, dtype))


@pytest.mark.parametrize("cols", [512, 640])
@pytest.mark.parametrize("share", [1, 2])
def test_lookup_matvec_is_the_oracles_table_product(cols, share, tables, dev):
    """The table's float16 rounding modelled (blocks.py:595-603, 618-643): only the float32 sums' order and the
    output's rounding are left."""
    E, R = 3, 64
    raw, _ = stack("Q2_0", E, R, cols, 17, tables)
    lin = SB.BlockSwitchLinear(torch.from_numpy(raw).to(dev), "Q2_0", (E, R, cols))
    rng = np.random.default_rng(18)
    idx = np.array([0, 2, 1, 1, 2, 0])
    x, xv = act(rng, (len(idx) // share, cols), "float16")
    got = SB.lookup_matvec(lin, torch.from_numpy(idx).to(dev), SB.lookup_table(x.to(dev)), share).float().cpu().numpy()
    want = OL.lookup_matvec(raw, (E, R, cols), idx, OL.lookup_table(xv, "float16"), share)
    assert (np.abs(got - want) <= 2.0 ** -11 * np.abs(want) + 1e-6 * np.abs(want).max()).all()


@pytest.mark.parametrize("pairs", [1, 10])
def test_lookup_down_glu_is_the_oracles(pairs, tables, dev):
    """silu(gate) * up in float32 into the float16 table (blocks.py:606-616, 702-760); the exponential's last bit
    may move an entry by one float16 step."""
    E, R, C = 3, 96, 640
    raw, _ = stack("Q2_0", E, R, C, 19, tables)
    down = SB.BlockSwitchLinear(torch.from_numpy(raw).to(dev), "Q2_0", (E, R, C))
    rng = np.random.default_rng(20 + pairs)
    idx = rng.integers(0, E, pairs)
    g, gv = act(rng, (pairs, C), "float16")
    u, uv = act(rng, (pairs, C), "float16")
    tab = SB.lookup_table_glu(g.to(dev), u.to(dev)).float().cpu().numpy()
    want_tab = OL.lookup_table_glu(gv, uv, "float16")
    step = np.abs(want_tab) * 2.0 ** -10 + 2.0 ** -24
    assert (np.abs(tab - want_tab) <= step).all() and (tab == want_tab).mean() > 0.99
    got = SB.lookup_down_glu(down, torch.from_numpy(idx).to(dev), g.to(dev), u.to(dev)).float().cpu().numpy()
    want = OL.lookup_down_glu(raw, (E, R, C), idx, gv, uv, "float16")
    assert rel_err(got, want) <= 2e-3


def test_lookup_matvec_is_the_product(tables, dev):
    E, R, C = 3, 64, 512
    raw, w = stack("Q2_0", E, R, C, 14, tables)
    lin = SB.BlockSwitchLinear(torch.from_numpy(raw).to(dev), "Q2_0", (E, R, C))
    rng = np.random.default_rng(15)
    x, xv = act(rng, (2, C), "float16")
    idx = np.array([0, 2, 1, 1])
    table = SB.lookup_table(x.to(dev))
    got = SB.lookup_matvec(lin, torch.from_numpy(idx).to(dev), table, 2).float().cpu()
    assert rel_err(got, OB.matvec(w, idx, xv, 2)) <= 1e-2


@pytest.mark.parametrize("kind", ["Q2_0", "IQ3_S"])
@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("tokens", [1, 4, 8, 16])
def test_stack_matvec_streams_many_matrices(kind, dtype, tokens, tables, dev):
    """The streaming window matvec: every matrix of a stack times its own tokens, rows not a multiple of a tile."""
    n, R, C = 7, 200, 512
    raw, w = stack(kind, n, R, C, 20 + tokens, tables)
    rng = np.random.default_rng(tokens)
    x, xv = act(rng, (n, tokens, C), dtype)
    got = SB.stack_matvec(torch.from_numpy(raw).to(dev), kind, (n, R, C), x.to(dev)).float().cpu().numpy()
    want = np.einsum("mrc,mtc->mtr", w.astype(np.float64), xv.astype(np.float64))
    assert got.shape == (n, tokens, R)
    assert rel_err(got, want) <= TOL[dtype]


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("tokens", [1, 2])
@pytest.mark.parametrize("kind, shape", [("Q2_0", (40, 512, 1024)), ("Q2_0", (12, 1536, 2048)),
                                         ("Q2_0", (36, 528, 1024)), ("IQ3_S", (40, 512, 2048)),
                                         ("IQ3_S", (12, 1536, 2048))])
def test_long_stacks_stream_by_waves(kind, shape, tokens, dtype, tables, dev):
    """Stacks of more than a thousand 16-row groups: Q2_0 in the wave-streamed form (blocks whose row tiles cross
    matrix boundaries, waves with no row tile in a block, 2 and 4 K-chunks a row, tiles of 32 rows and, for 528
    rows a matrix, of 16), IQ3_S in the block-ring form."""
    n, R, C = shape
    raw, w = stack(kind, n, R, C, 40 + tokens, tables)
    rng = np.random.default_rng(50 + tokens)
    x, xv = act(rng, (n, tokens, C), dtype)
    got = SB.stack_matvec(torch.from_numpy(raw).to(dev), kind, (n, R, C), x.to(dev)).float().cpu().numpy()
    want = np.stack([xv[m].astype(np.float64) @ w[m].T.astype(np.float64) for m in range(n)])
    assert got.shape == (n, tokens, R)
    assert rel_err(got, want) <= TOL[dtype]
    for m in (0, n // 2, n - 1):  # every matrix's own rows
        assert rel_err(got[m], want[m]) <= TOL[dtype]


@pytest.mark.parametrize("kind, cols", [("IQ3_S", 4352), ("IQ3_S", 4608), ("IQ3_S", 8192), ("Q2_0", 6400),
                                        ("Q2_0", 8192)])
@pytest.mark.parametrize("tokens", [1, 4, 9])
def test_window_matvec_of_wide_rows(kind, cols, tokens, tables, dev):
    """Rows past 4096 columns: the streaming kernel where its waves split the row evenly and its ring fits in LDS,
    the generic window kernel otherwise; the stack form refuses the rows it cannot split instead of dropping the
    remainder (IQ3_S at 4352: 136 runs, not a multiple of the 16 a wave)."""
    R = 48
    raw, w = stack(kind, 1, R, cols, cols + tokens, tables)
    rng = np.random.default_rng(cols + tokens)
    x, xv = act(rng, (tokens, cols), "bfloat16")
    got = SB.window_matvec(torch.from_numpy(raw).to(dev), kind, R, cols, x.to(dev)).float().cpu().numpy()
    want = xv.astype(np.float64) @ w[0].T.astype(np.float64)
    assert rel_err(got, want) <= TOL["bfloat16"]
    if kind == "IQ3_S" and cols == 4352:
        with pytest.raises(Exception, match="columns"):
            SB.stack_matvec(torch.from_numpy(raw).to(dev), kind, (1, R, cols), x[None].to(dev))


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("tokens", [3, 4])
@pytest.mark.parametrize("shape", [(40, 512, 1024), (12, 1536, 2048), (36, 528, 1024)])
def test_q2_stacks_of_three_and_four_tokens(shape, tokens, dtype, tables, dev):
    """Q2_0 stacks of many 32-row items at 3 and 4 tokens: the block-ring form whose waves each take both row groups
    of an item over a quarter or an eighth of the columns (one set of activation registers for 32 rows), the other
    column splits' sums added by the first split's wave; for 528 rows a matrix the last item has one row group."""
    n, R, C = shape
    raw, w = stack("Q2_0", n, R, C, 60 + tokens, tables)
    rng = np.random.default_rng(70 + tokens)
    x, xv = act(rng, (n, tokens, C), dtype)
    got = SB.stack_matvec(torch.from_numpy(raw).to(dev), "Q2_0", (n, R, C), x.to(dev)).float().cpu().numpy()
    want = np.stack([xv[m].astype(np.float64) @ w[m].T.astype(np.float64) for m in range(n)])
    for m in (0, n // 2, n - 1):
        assert rel_err(got[m], want[m]) <= TOL[dtype]
    assert rel_err(got, want) <= TOL[dtype]


@pytest.mark.parametrize("kind", ["Q2_0", "IQ3_S"])
def test_window_matvec_bits_do_not_depend_on_the_window(kind, tables, dev):
    raw, w = stack(kind, 1, 96, 2048, 30, tables)
    x = torch.randn(8, 2048).to(torch.bfloat16)
    b = torch.from_numpy(raw).to(dev)
    got = SB.window_matvec(b, kind, 96, 2048, x.to(dev)).cpu()
    alone = torch.cat([SB.window_matvec(b, kind, 96, 2048, x[t:t + 1].to(dev)).cpu() for t in range(8)])
    assert torch.equal(alone, got)
    assert rel_err(got.float(), x.float().numpy().astype(np.float64) @ w[0].T.astype(np.float64)) <= 1e-2


@pytest.mark.parametrize("kind, dtype", [("Q2_0", "bfloat16"), ("IQ3_S", "float16"), ("IQ4_NL", "bfloat16"),
                                         ("Q2_0", "float32"), ("Q3_K", "float16")])
def test_pairs_naming_no_expert_get_zeros(kind, dtype, tables, dev):
    """A pair whose index is outside 0..experts-1 reads no weights and gets a zero row (every product kernel: the
    MFMA and generic matvecs, the GLU matvec, the table-of-sums products); the other pairs are the oracle's."""
    E, R, C = 4, 48, 512
    raw, w = stack(kind, E, R, C, 31, tables)
    rng = np.random.default_rng(32)
    idx = np.array([2, -1, 0, E, 3, 1 << 20, 1])
    x, xv = act(rng, (len(idx), C), dtype)
    lin = SB.BlockSwitchLinear(torch.from_numpy(raw).to(dev), kind, (E, R, C))
    ti = torch.from_numpy(idx).to(dev)
    real = (idx >= 0) & (idx < E)
    got = SB.switch_matvec(lin.blocks, kind, (E, R, C), ti, x.to(dev), 1).float().cpu().numpy()
    assert (got[~real] == 0).all()
    assert rel_err(got[real], OB.matvec(w, idx[real], xv[real], 1)) <= TOL[dtype]
    if dtype == "float32":
        return
    u, uv = act(rng, (len(idx), C), dtype)
    glu = SB.matvec_glu(lin, ti, x.to(dev), u.to(dev)).float().cpu().numpy()
    assert (glu[~real] == 0).all()
    assert rel_err(glu[real], OB.matvec(w, idx[real], OR.swiglu(xv, uv, dtype)[real], 1)) <= TOL[dtype]
    if kind == "Q2_0" and dtype == "bfloat16":
        xh = x.to(torch.float16)
        look = SB.lookup_matvec(lin, ti, SB.lookup_table(xh.to(dev)), 1).float().cpu().numpy()
        assert (look[~real] == 0).all()
        assert rel_err(look[real], OB.matvec(w, idx[real], xh.float().numpy()[real], 1)) <= 1e-2
        down = SB.lookup_down_glu(lin, ti, xh.to(dev), u.to(torch.float16).to(dev)).float().cpu().numpy()
        assert (down[~real] == 0).all()
