"""The streaming matvec of exact weights (every kind, float32 / bf16 / fp16 activations, one layer or a stack of
matrices): the oracle's products within the path's tolerances; for the kinds whose runs it takes as the generic
kernels do (not Q2_0, IQ4_NL, IQ4_XS, Q3_K, whose scales and offsets it takes out of the sums) the generic expert
kernel's bits exactly (the same runs a lane, the same order of sums); a token's bits whatever its window, and a
layer's the same alone or in a stack."""

import numpy as np
import pytest
import torch

from conftest import rel_err
from oracle import blocks as OB
from strata_hip import blocks as SB
from strata_hip import synth

pytestmark = pytest.mark.gpu

KINDS = sorted(SB.BLOCK)
TORCH = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}
TOL = {"float32": 1e-5, "float16": 1e-2, "bfloat16": 1e-2}


def mats(kind, n, rows, cols, seed, tables):
    rng = np.random.default_rng(seed)
    raw = synth.random_blocks(kind, n * rows, cols, rng)
    return raw, OB.dequantize(raw, kind, (n, rows, cols), tables)


def act(rng, shape, dtype):
    t = torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).to(TORCH[dtype])
    return t, t.float().numpy()


FACTORED = ("Q2_0", "IQ4_NL", "IQ4_XS", "Q3_K")  # kinds whose runs the stream takes with the scales outside


def streamed(kind, dtype):
    """Whether window_matvec takes the exact-weight stream (not the MFMA kernels) for this kind and dtype, with the
    generic kernel's bits (its runs' arithmetic)."""
    return kind not in FACTORED and not (kind == "IQ3_S" and dtype != "float32")


def off16(x):
    """x's values in a buffer that does not start on 16 bytes (one element in): the stream does not take it."""
    flat = torch.empty(x.numel() + 1, dtype=x.dtype, device=x.device)
    out = flat[1:].view(x.shape)
    out.copy_(x)
    assert out.data_ptr() % 16
    return out


def generic(b, kind, shape, x, dev):
    """The generic expert kernel (matvec_separate, a buffer a pair, activations off 16 bytes), pair t = matrix m's
    token t: the reference bits of the stream."""
    n, rows, cols = shape
    tokens = x.shape[-2]
    mat = rows * SB.row_bytes(kind, cols)
    experts = [b[m * mat : (m + 1) * mat] for m in range(n) for _ in range(tokens)]
    x1 = off16(x.reshape(-1, cols))
    return SB.matvec_separate(experts, kind, rows, cols, x1, 1).reshape(n, tokens, rows)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("tokens", [1, 3, 8])
def test_window_matvec_of_every_kind(kind, dtype, tokens, tables, dev):
    R, C = 200, 512  # rows not a multiple of an item's
    raw, w = mats(kind, 1, R, C, 300 + tokens, tables)
    rng = np.random.default_rng(310 + tokens)
    x, xv = act(rng, (tokens, C), dtype)
    b = torch.from_numpy(raw).to(dev)
    got = SB.window_matvec(b, kind, R, C, x.to(dev)).cpu()
    want = xv.astype(np.float64) @ w[0].T.astype(np.float64)
    assert got.shape == (tokens, R) and got.dtype == TORCH[dtype]
    assert rel_err(got.float().numpy(), want) <= TOL[dtype]
    if streamed(kind, dtype):
        assert torch.equal(got, generic(b, kind, (1, R, C), x[None].to(dev), dev)[0].cpu())


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("tokens", [1, 5])
def test_stack_matvec_of_every_kind(kind, dtype, tokens, tables, dev):
    """Many matrices in one launch: items crossing from one matrix to the next, each matrix its own tokens."""
    n, R, C = 6, 72, 1024
    raw, w = mats(kind, n, R, C, 320 + tokens, tables)
    rng = np.random.default_rng(330 + tokens)
    x, xv = act(rng, (n, tokens, C), dtype)
    b = torch.from_numpy(raw).to(dev)
    got = SB.stack_matvec(b, kind, (n, R, C), x.to(dev)).cpu()
    want = np.einsum("mrc,mtc->mtr", w.astype(np.float64), xv.astype(np.float64))
    assert got.shape == (n, tokens, R)
    assert rel_err(got.float().numpy(), want) <= TOL[dtype]
    for m in (0, n - 1):
        assert rel_err(got[m].float().numpy(), want[m]) <= TOL[dtype]
    if streamed(kind, dtype):
        assert torch.equal(got, generic(b, kind, (n, R, C), x.to(dev), dev).cpu())


@pytest.mark.parametrize("kind, cols", [("Q2_0", 192), ("Q2_0", 2880), ("IQ4_NL", 96), ("Q3_K", 2560),
                                        ("IQ1_M", 768), ("IQ2_XXS", 1280)])
@pytest.mark.parametrize("tokens", [1, 2])
def test_rows_not_whole_chunks(kind, cols, tokens, tables, dev):
    """Rows whose bytes are not whole 16-byte chunks (Q2_0 at 54 and 810 bytes, IQ4_NL at 54, Q3_K at the reference
    model's d 2560: 1,100): items start inside a chunk and end with loose bytes; rows of fewer runs than a wave."""
    n, R = 3, 37
    raw, w = mats(kind, n, R, cols, cols + tokens, tables)
    rng = np.random.default_rng(cols + 7 * tokens)
    x, xv = act(rng, (n, tokens, cols), "float32")
    b = torch.from_numpy(raw).to(dev)
    got = SB.stack_matvec(b, kind, (n, R, cols), x.to(dev)).cpu()
    want = np.einsum("mrc,mtc->mtr", w.astype(np.float64), xv.astype(np.float64))
    assert rel_err(got.numpy(), want) <= TOL["float32"]
    if kind not in FACTORED:
        assert torch.equal(got, generic(b, kind, (n, R, cols), x.to(dev), dev).cpu())
    one = SB.window_matvec(b[: R * SB.row_bytes(kind, cols)], kind, R, cols, x[0].to(dev)).cpu()
    assert torch.equal(one, got[0])


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("kind, cols, block, d_at", [("Q2_0", 576, 18, 0), ("IQ4_NL", 576, 18, 0),
                                                     ("IQ4_XS", 768, 136, 0), ("Q3_K", 768, 110, 108)])
def test_negative_scales(kind, cols, block, d_at, dtype, tables, dev):
    """Blocks with negative scales (the stream takes the scales out of each run's sums): rows of both signs against
    the oracle, a layer alone the bits of the same layer in the stack."""
    n, R, C = 2, 64, cols  # Q2_0 at 9 blocks a row: the MFMA kernels do not take it in bf16 either
    raw, _ = mats(kind, n, R, C, 370, tables)
    blk = raw.reshape(-1, block)
    blk[::2, d_at + 1] |= 0x80  # every other block's fp16 scale negative
    w = OB.dequantize(raw, kind, (n, R, C), tables)
    rng = np.random.default_rng(371)
    x, xv = act(rng, (n, 3, C), dtype)
    b = torch.from_numpy(raw).to(dev)
    got = SB.stack_matvec(b, kind, (n, R, C), x.to(dev)).cpu()
    want = np.einsum("mrc,mtc->mtr", w.astype(np.float64), xv.astype(np.float64))
    assert rel_err(got.float().numpy(), want) <= TOL[dtype]
    one = SB.window_matvec(b[R * SB.row_bytes(kind, C):], kind, R, C, x[1].to(dev)).cpu()
    assert torch.equal(one, got[1])


@pytest.mark.parametrize("kind", ["Q2_0", "IQ4_XS", "IQ2_S"])
def test_a_tokens_bits_do_not_depend_on_its_window(kind, tables, dev):
    R, C = 96, 2048
    raw, _ = mats(kind, 1, R, C, 340, tables)
    x = torch.randn(8, C)
    b = torch.from_numpy(raw).to(dev)
    whole = SB.window_matvec(b, kind, R, C, x.to(dev)).cpu()
    for t in (0, 3, 7):
        assert torch.equal(SB.window_matvec(b, kind, R, C, x[t : t + 1].to(dev)).cpu()[0], whole[t])
        assert torch.equal(SB.window_matvec(b, kind, R, C, x[: t + 1].to(dev)).cpu()[t], whole[t])


def test_the_float32_matvec_at_its_benchmark_shape(tables, dev):
    """Q2_0 3072 x 2048 with a float32 vector, out float32: 1e-5 of the oracle, alone and as one of a stack of
    eight (the same bits)."""
    R, C, n = 3072, 2048, 8
    raw, w = mats("Q2_0", n, R, C, 350, tables)
    rng = np.random.default_rng(351)
    x, xv = act(rng, (n, 1, C), "float32")
    b = torch.from_numpy(raw).to(dev)
    got = SB.window_matvec(b[: R * SB.row_bytes("Q2_0", C)], "Q2_0", R, C, x[0].to(dev)).cpu()
    assert rel_err(got[0].numpy(), w[0].astype(np.float64) @ xv[0, 0].astype(np.float64)) <= 1e-5
    stacked = SB.stack_matvec(b, "Q2_0", (n, R, C), x.to(dev)).cpu()
    assert torch.equal(stacked[0], got)
    want = np.einsum("mrc,mtc->mtr", w.astype(np.float64), xv.astype(np.float64))
    assert rel_err(stacked.numpy(), want) <= 1e-5


def test_the_stream_refuses_what_it_does_not_take(tables, dev):
    """More than 8 tokens a matrix of an exact-weight kind, and activations too wide for LDS, are refused (the
    MFMA kinds take 16 tokens in bf16 / fp16)."""
    raw, _ = mats("IQ4_XS", 2, 16, 512, 360, tables)
    b = torch.from_numpy(raw).to(dev)
    with pytest.raises(Exception, match="tokens"):
        SB.stack_matvec(b, "IQ4_XS", (2, 16, 512), torch.zeros((2, 9, 512), dtype=torch.bfloat16).to(dev))
    wide = torch.from_numpy(mats("IQ4_NL", 1, 4, 4096, 361, tables)[0]).to(dev)
    with pytest.raises(Exception, match="LDS"):
        SB.stack_matvec(wide, "IQ4_NL", (1, 4, 4096), torch.zeros((1, 8, 4096)).to(dev))
    # one layer of them still multiplies, through the generic window kernel
    got = SB.window_matvec(wide, "IQ4_NL", 4, 4096, torch.ones((8, 4096)).to(dev))
    assert got.shape == (8, 4)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("share", [1, 3])
def test_expert_pairs_through_the_stream(kind, dtype, share, tables, dev):
    """switch_matvec's pairs (each its expert of the stack and its row of x, pairs sharing a row, a pair naming no
    expert): the oracle's products, zeros for the pair without an expert, the generic kernel's bits for the kinds
    whose runs the stream takes as it does."""
    E, R, C = 5, 96, 512
    raw, w = mats(kind, E, R, C, 380, tables)
    idx = np.array([4, 0, 2, 2, 7, 1, 0, 3, -1], dtype=np.int32)  # 7 and -1 name no expert
    rng = np.random.default_rng(381)
    x, xv = act(rng, (-(-len(idx) // share), C), dtype)
    b = torch.from_numpy(raw).to(dev)
    if kind in ("Q2_0", "IQ3_S") and dtype != "float32":
        pytest.skip("the MFMA kernels take these pairs")
    got = SB.switch_matvec(b, kind, (E, R, C), torch.from_numpy(idx).to(dev), x.to(dev), share).cpu()
    for p, e in enumerate(idx):
        if 0 <= e < E:
            want = w[e].astype(np.float64) @ xv[p // share].astype(np.float64)
            assert rel_err(got[p].float().numpy(), want) <= TOL[dtype]
        else:
            assert not got[p].any()
    if kind not in FACTORED:
        mat = R * SB.row_bytes(kind, C)
        ok = [p for p, e in enumerate(idx) if 0 <= e < E]
        sep = SB.matvec_separate([b[idx[p] * mat : (idx[p] + 1) * mat] for p in ok], kind, R, C,
                                 off16(torch.stack([x[p // share] for p in ok]).to(dev)), 1).cpu()
        assert torch.equal(got[ok], sep)


@pytest.mark.parametrize("kind", ["Q2_0", "IQ4_XS", "IQ2_XS"])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_pairs_bringing_their_own_buffers(kind, dtype, tables, dev):
    """matvec_separate (an expert buffer a pair, as the paged experts bring them): buffers starting anywhere in
    their allocation (5 bytes in), the oracle's products; the generic kernel's bits for a codebook kind."""
    R, C = 48, 768
    raw, w = mats(kind, 3, R, C, 420, tables)
    mat = R * SB.row_bytes(kind, C)
    big = torch.zeros(3 * mat + 64, dtype=torch.uint8)
    big[5 : 5 + 3 * mat] = torch.from_numpy(raw)
    big = big.to(dev)
    order = [2, 0, 2, 1]
    experts = [big[5 + e * mat : 5 + (e + 1) * mat] for e in order]
    rng = np.random.default_rng(421)
    x, xv = act(rng, (len(order), C), dtype)
    got = SB.matvec_separate(experts, kind, R, C, x.to(dev), 1).cpu()
    for p, e in enumerate(order):
        want = w[e].astype(np.float64) @ xv[p].astype(np.float64)
        assert rel_err(got[p].float().numpy(), want) <= TOL[dtype]
    if kind not in FACTORED:
        assert torch.equal(got, SB.matvec_separate(experts, kind, R, C, off16(x.to(dev)), 1).cpu())


@pytest.mark.parametrize("kind", ["Q2_0", "IQ2_S"])
def test_activations_off_16_bytes_take_the_generic_kernel(kind, tables, dev):
    """Activations that do not start on 16 bytes (a view one element in) are not the stream's: the window and the
    pairs go to the generic kernel, the stack is refused; the products are the same within the tolerance (the
    same bits for a codebook kind)."""
    E, R, C = 3, 64, 512
    raw, w = mats(kind, E, R, C, 390, tables)
    b = torch.from_numpy(raw).to(dev)
    rng = np.random.default_rng(391)
    xs, xv = act(rng, (1, 2 * C + 1), "float32")
    off = xs.to(dev)[0, 1 : 1 + 2 * C].reshape(2, C)  # 4 bytes past a 16-byte boundary
    ok = off.clone()
    assert off.data_ptr() % 16 and ok.data_ptr() % 16 == 0
    mat = R * SB.row_bytes(kind, C)
    got = SB.window_matvec(b[:mat], kind, R, C, off).cpu()
    ref = SB.window_matvec(b[:mat], kind, R, C, ok).cpu()
    want = xv[0, 1 : 1 + 2 * C].reshape(2, C).astype(np.float64) @ w[0].T.astype(np.float64)
    assert rel_err(got.numpy(), want) <= 1e-5 and rel_err(ref.numpy(), want) <= 1e-5
    idx = torch.tensor([2, 0], dtype=torch.int32).to(dev)
    pairs = SB.switch_matvec(b, kind, (E, R, C), idx, off, 1).cpu()
    assert rel_err(pairs[0].numpy(), w[2].astype(np.float64) @ xv[0, 1 : 1 + C].astype(np.float64)) <= 1e-5
    if kind not in FACTORED:
        assert torch.equal(got, ref)
        assert torch.equal(pairs, SB.switch_matvec(b, kind, (E, R, C), idx, ok, 1).cpu())
    with pytest.raises(Exception, match="aligned"):
        SB.stack_matvec(b[:mat], kind, (1, R, C), off[None])


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
def test_dequantize_by_the_stream(kind, dtype, tables, dev):
    """dequantize through the coalesced stream: the oracle's weights rounded once to the dtype, bit for bit, over
    items of several rows, a last item of fewer, and rows whose bytes are not whole 16-byte chunks."""
    cols = {"Q2_0": 2880, "IQ4_NL": 1120, "Q3_K": 2560}.get(kind, 1280)
    raw, w = mats(kind, 3, 37, cols, 400, tables)
    got = SB.dequantize(torch.from_numpy(raw).to(dev), kind, (3, 37, cols), TORCH[dtype]).cpu()
    want = torch.from_numpy(w).to(TORCH[dtype])
    assert got.shape == want.shape and torch.equal(got, want)
    # an output that does not start on 16 bytes takes the generic kernel: the same values
    flat = torch.empty(3 * 37 * cols + 1, dtype=TORCH[dtype], device=dev)
    lib_out = flat[1:].view(3, 37, cols)
    from strata_hip import _lib

    blocks = torch.from_numpy(raw).to(dev)
    _lib.call("sh_dequantize", SB._kind(kind), blocks.data_ptr(), SB._tabs(kind, lib_out.device), 3, 37, cols,
              lib_out.data_ptr(), _lib.dtype_code(TORCH[dtype]), _lib.stream_of(lib_out))
    assert torch.equal(lib_out.cpu(), want)


def test_dequantize_many_items_a_block(tables, dev):
    """A tensor of 9,000 rows: items of 5 rows, each block several items (the next item's loads in flight while
    one is decoded)."""
    raw, w = mats("Q2_0", 3, 3000, 2880, 410, tables)
    got = SB.dequantize(torch.from_numpy(raw).to(dev), "Q2_0", (3, 3000, 2880), torch.bfloat16).cpu()
    assert torch.equal(got, torch.from_numpy(w).to(torch.bfloat16))
