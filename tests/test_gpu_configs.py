"""The benchmark configurations at their full sizes on the GPU, each against the oracle: the Q2_0 3072 x 2048 matvec
with float32 activations (1e-5), paged attention at 32K and 128K positions for one and eight queries (float64
softmax head group by head group, 1e-2), the 2048-token IQ3_S prompt layer of 512 experts under Zipf(1.1) routing
(the tokens' pairs against the reference's composition from the rounded weights), and switch_glu's middle branch
(more pairs than the fused down takes, fewer than the tiles)."""

import numpy as np
import pytest
import torch

from conftest import rel_err
from oracle import blocks as OB
from oracle import moe as OM
from oracle import route as OR
from strata_hip import attention as SA
from strata_hip import blocks as SB
from strata_hip import fused as SF
from strata_hip import synth

pytestmark = pytest.mark.gpu


def test_the_q2_0_matvec_with_float32_activations(tables, dev):
    """3072 x 2048 Q2_0, x float32 (1, 2048): the window product and the one-expert switch product, 1e-5."""
    R, C = 3072, 2048
    rng = np.random.default_rng(1)
    raw = synth.random_blocks("Q2_0", R, C, rng)
    w = OB.dequantize(raw, "Q2_0", (1, R, C), tables)[0].astype(np.float64)
    x = rng.standard_normal((1, C)).astype(np.float32)
    want = x.astype(np.float64) @ w.T
    b = torch.from_numpy(raw).to(dev)
    got = SB.window_matvec(b, "Q2_0", R, C, torch.from_numpy(x).to(dev))
    assert got.dtype == torch.float32 and got.shape == (1, R)
    assert rel_err(got.cpu().numpy(), want) <= 1e-5
    lin = SB.BlockSwitchLinear(b, "Q2_0", (1, R, C))
    got = lin(torch.from_numpy(x).to(dev).reshape(1, 1, 1, C), torch.zeros((1, 1), dtype=torch.int32, device=dev))
    assert rel_err(got.reshape(1, R).cpu().numpy(), want) <= 1e-5


def paged_want(q, k, v, table, ctx, scale):
    """float64 softmax(q k^T scale) v over the page-gathered keys, query t seeing positions <= ctx - B + t; one KV
    head at a time (k, v: torch bf16 (pages, hkv, 16, D) on the GPU, gathered there, moved one head at a time)."""
    B, Hq, D = q.shape
    hkv = k.shape[1]
    group = Hq // hkv
    pos = torch.arange(ctx, device=k.device)
    phys = table.long()[pos // 16]
    out = np.zeros((B, Hq, D))
    for g in range(hkv):
        K = k[phys, g, pos % 16].cpu().double().numpy()
        V = v[phys, g, pos % 16].cpu().double().numpy()
        for t in range(B):
            rows = q[t, g * group:(g + 1) * group].cpu().double().numpy()
            seen = ctx - B + t + 1
            s = rows @ K[:seen].T * scale
            p = np.exp(s - s.max(axis=1, keepdims=True))
            out[t, g * group:(g + 1) * group] = (p / p.sum(axis=1, keepdims=True)) @ V[:seen]
    return out


@pytest.mark.parametrize("ctx, B", [(32768, 1), (32768, 8), (131072, 1), (131072, 8)])
def test_paged_attention_at_long_contexts(ctx, B, dev):
    """16 query heads, 2 KV heads of 256, pages of 16 in a shuffled order: the splits and their merge as the
    benchmark runs them (at 128K and eight queries, hundreds of splits a head)."""
    Hq, Hkv, D = 16, 2, 256
    n_pages = ctx // 16
    gen = torch.Generator(device=dev)
    gen.manual_seed(ctx + B)
    k = torch.randn((n_pages, Hkv, 16, D), generator=gen, device=dev).to(torch.bfloat16)
    v = torch.randn((n_pages, Hkv, 16, D), generator=gen, device=dev).to(torch.bfloat16)
    table = torch.randperm(n_pages, generator=gen, device=dev).to(torch.int32)
    q = torch.randn((B, Hq, D), generator=gen, device=dev).to(torch.bfloat16)
    torch.cuda.synchronize()
    got = SA.paged_decode_attention(q, k, v, table, ctx)
    want = paged_want(q, k, v, table, ctx, 1 / 16)
    assert got.shape == (B, Hq, D)
    assert rel_err(got.float().cpu().numpy(), want) <= 1e-2


def test_the_prompt_layer_at_its_benchmark_shape(tables, dev):
    """2048 tokens x top-10 of 512 IQ3_S experts (d 2048, ffn 512) under Zipf(1.1) popularity, made as the benchmark
    makes them (same generators and seeds): the fused two-pass prompt path; 8 tokens' 80 pairs against the
    reference's composition (blocks.py:566-576: float32 products of the weights rounded to bf16, h = swiglu rounded
    once to bf16, down rounded to bf16), and every pair against the pair-by-pair branch."""
    E, D, F, T, K = 512, 2048, 512, 2048, 10
    rng = np.random.default_rng(5)
    logits = synth.zipf_logits(rng, T, E).to(dev)
    x = torch.from_numpy(rng.standard_normal((T, D)).astype(np.float32)).to(torch.bfloat16)
    shapes = {"g": (E, F, D), "u": (E, F, D), "d": (E, D, F)}
    raw = {n: synth.random_blocks_gpu("IQ3_S", shapes[n][0] * shapes[n][1], shapes[n][2], seed, dev)
           for n, seed in (("g", 11), ("u", 12), ("d", 13))}
    lin = {n: SB.BlockSwitchLinear(raw[n], "IQ3_S", shapes[n]) for n in raw}
    idx = SF.top_k(logits, K)
    glu = SB.BlockSwitchGLU(lin["g"], lin["u"], lin["d"])
    got = glu(x.to(dev), idx).float().cpu().numpy()
    idx = idx.cpu().numpy()
    assert got.shape == (T, K, D)
    sample = np.random.default_rng(61).choice(T, 8, replace=False)
    rb = {n: OB.row_bytes("IQ3_S", shapes[n][2]) * shapes[n][1] for n in raw}
    xs = x.float().numpy().astype(np.float64)
    want = np.zeros((len(sample), K, D))
    for e in np.unique(idx[sample]):
        w = {n: OR.round_to(OB.dequantize(raw[n][e * rb[n]:(e + 1) * rb[n]].cpu().numpy(), "IQ3_S", shapes[n][1:],
                                          tables), "bfloat16").astype(np.float64) for n in raw}
        for i, t in enumerate(sample):
            for j in np.nonzero(idx[t] == e)[0]:
                g, u = w["g"] @ xs[t], w["u"] @ xs[t]
                h = OR.round_to(g / (1 + np.exp(-g)) * u, "bfloat16").astype(np.float64)
                want[i, j] = OR.round_to(w["d"] @ h, "bfloat16")
    assert np.isfinite(want).all()
    assert rel_err(got[sample], want) <= 1e-2
    old = SB.TILES_FROM
    SB.TILES_FROM = 1 << 62
    try:
        pairwise = glu(x.to(dev), torch.from_numpy(idx).to(dev)).float().cpu().numpy()
    finally:
        SB.TILES_FROM = old
    assert rel_err(got, pairwise) <= 2e-2


@pytest.mark.parametrize("kind", ["Q2_0", "IQ3_S"])
@pytest.mark.parametrize("tokens", [4, 20, 150])
def test_switch_glus_middle_branch(kind, tokens, tables, dev):
    """40 to 1,500 pairs: gate and up by the expert matvec, down by the matvec of swiglu(gate, up) rounded as the
    reference rounds (blocks.py:819-829), against the oracle's composition."""
    E, D, F, K = 32, 512, 256, 10
    rng = np.random.default_rng(tokens)
    raws = {n: synth.random_blocks(kind, E * r, c, rng) for n, r, c in (("g", F, D), ("u", F, D), ("d", D, F))}
    shapes = {"g": (E, F, D), "u": (E, F, D), "d": (E, D, F)}
    lin = {n: SB.BlockSwitchLinear(torch.from_numpy(raws[n]).to(dev), kind, shapes[n]) for n in raws}
    w = {n: OB.dequantize(raws[n], kind, shapes[n], tables) for n in raws}
    idx = np.stack([rng.choice(E, K, replace=False) for _ in range(tokens)])
    x = synth.bf16_normal(rng, (tokens, D))
    assert SB.MATVEC_GLU_UPTO < idx.size < SB.TILES_FROM
    got = SB.BlockSwitchGLU(lin["g"], lin["u"], lin["d"])(x.to(dev), torch.from_numpy(idx).to(dev))
    want = OM.expert_products(w["g"], w["u"], w["d"], idx, x.float().numpy(), "bfloat16")
    assert got.shape == (tokens, K, D)
    assert rel_err(got.float().cpu().numpy(), want) <= 1e-2
