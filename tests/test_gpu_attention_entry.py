"""The attention entry on the GPU (strata_mlx/attention.py:228-261): norm and rope of q and k against the oracle, the
window's keys and values appended to shuffled pages, the output gate applied in the merge, the cell-list form over
pages, and a whole layer's call (projections, cache append, attend, gate, o_proj) including a verify pass whose
rejected drafts are trimmed and overwritten."""

import math

import numpy as np
import pytest
import torch

from conftest import rel_err
from oracle import attention as OA
from oracle import route as OR
from strata_hip import attention as SA

pytestmark = pytest.mark.gpu
NAME = {torch.float16: "float16", torch.bfloat16: "bfloat16"}


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D, rot, stride_mul", [(256, 64, 2), (128, 128, 1), (256, 0, 1), (64, 64, 1), (192, 32, 1),
                                                (320, 320, 2), (384, 0, 1), (448, 64, 1), (512, 128, 1)])
def test_qk_rope_is_the_oracles(dtype, D, rot, stride_mul, dev):
    rng = np.random.default_rng(D + rot)
    S, H = 5, 6
    x = torch.from_numpy(rng.standard_normal((1, S, H * D * stride_mul)).astype(np.float32) * 2).to(dtype)
    w = torch.from_numpy(1 + 0.2 * rng.standard_normal(D).astype(np.float32)).to(dtype)
    th = rng.uniform(0, 6.3, (S, max(rot // 2, 1)))[:, :rot // 2]
    cos = torch.from_numpy(np.cos(np.concatenate([th, th], axis=1))).to(dtype)
    sin = torch.from_numpy(np.sin(np.concatenate([th, th], axis=1))).to(dtype)
    got = SA.qk_rope(x.to(dev), w.to(dev), 1e-6, cos.to(dev), sin.to(dev), H, D, D * stride_mul).float().cpu()
    assert got.shape == (1, H, S, D)
    want = OA.qk_rope(x.float().numpy()[0], w.float().numpy(), cos.float().numpy(), sin.float().numpy(), H, D,
                      D * stride_mul, 1e-6, NAME[dtype])
    ulp = np.abs(want) * (2.0 ** -9 if dtype == torch.bfloat16 else 2.0 ** -10) + 1e-6
    diff = np.abs(got.numpy()[0] - want)
    assert (diff <= 2 * ulp).all() and (diff == 0).mean() > 0.95  # only the float32 sum's order may move a bit
    tok_major = SA.qk_rope(x.to(dev), w.to(dev), 1e-6, cos.to(dev), sin.to(dev), H, D, D * stride_mul,
                           heads_first=False).cpu()
    assert torch.equal(tok_major.transpose(0, 1).float(), got[0])


def test_kv_append_writes_the_pages_the_table_names(dev):
    rng = np.random.default_rng(3)
    n_pages, G, D = 12, 2, 256
    table = torch.from_numpy(rng.permutation(n_pages).astype(np.int32)).to(dev)
    cache = SA.PagedKVCache(n_pages, G, D, torch.bfloat16, dev, page_table=table)
    k_all, v_all = [], []
    for S in (37, 1, 8, 5):  # crossing page boundaries, one at a time, a window
        k = torch.randn((S, G, D), device=dev).to(torch.bfloat16)
        v = torch.randn((S, G, D), device=dev).to(torch.bfloat16)
        cache.update_and_fetch(k, v)
        k_all.append(k)
        v_all.append(v)
    K, V = torch.cat(k_all), torch.cat(v_all)
    pos = torch.arange(cache.offset, device=dev)
    phys = table.long()[pos // 16]
    assert torch.equal(cache.k_pages[phys, :, pos % 16], K) and torch.equal(cache.v_pages[phys, :, pos % 16], V)
    untouched = torch.ones(n_pages * 16, dtype=torch.bool, device=dev)
    untouched[(phys * 16 + pos % 16)] = False
    assert (cache.k_pages.permute(0, 2, 1, 3).reshape(n_pages * 16, G, D)[untouched] == 0).all()
    assert cache.trim(6) == 6 and cache.offset == 45
    with pytest.raises(ValueError):
        cache.update_and_fetch(torch.zeros((200, G, D), device=dev, dtype=torch.bfloat16),
                               torch.zeros((200, G, D), device=dev, dtype=torch.bfloat16))


@pytest.mark.parametrize("B, ctx", [(1, 300), (4, 2000), (8, 4096)])
def test_gated_paged_attention(B, ctx, dev):
    rng = np.random.default_rng(B)
    Hq, Hkv, D = 16, 2, 256
    n_pages = -(-ctx // 16)
    k = torch.from_numpy(rng.standard_normal((n_pages, Hkv, 16, D)).astype(np.float32)).to(torch.float16)
    v = torch.from_numpy(rng.standard_normal((n_pages, Hkv, 16, D)).astype(np.float32)).to(torch.float16)
    table = rng.permutation(n_pages).astype(np.int32)
    q = torch.from_numpy(rng.standard_normal((B, Hq, D)).astype(np.float32)).to(torch.float16)
    proj = torch.from_numpy(rng.standard_normal((B, Hq, 2 * D)).astype(np.float32) * 2).to(torch.float16)
    gate = proj.to(dev)[..., D:]  # the q projection's second half a head: a strided view
    got = SA.paged_decode_attention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(table).to(dev), ctx,
                                    gate=gate).float().cpu().numpy()
    att = OA.paged_decode(q.float().numpy(), k.float().numpy(), v.float().numpy(), table, ctx, 1 / 16)
    want = OA.gate_out(att.astype(np.float32), proj.float().numpy()[..., D:], "float16")
    assert rel_err(got, want) <= 1e-2


def test_cells_over_pages(dev):
    """The indexer's cells read through a shuffled page table (attention.py:144-165 on a paged pool)."""
    rng = np.random.default_rng(9)
    S, H, G, D, L, n_pages = 3, 16, 2, 256, 260, 40
    kv_len = n_pages * 16
    k = torch.from_numpy(rng.standard_normal((n_pages, G, 16, D)).astype(np.float32)).to(torch.bfloat16)
    v = torch.from_numpy(rng.standard_normal((n_pages, G, 16, D)).astype(np.float32)).to(torch.bfloat16)
    table = rng.permutation(n_pages).astype(np.int32)
    q = torch.from_numpy(rng.standard_normal((S, H, D)).astype(np.float32)).to(torch.bfloat16)
    cells = rng.integers(0, kv_len, (S, L)).astype(np.int32)
    real = rng.random((S, L)) < 0.8
    real[:, 0] = True
    gate = torch.from_numpy(rng.standard_normal((S, H, D)).astype(np.float32)).to(torch.bfloat16)
    from strata_hip import _lib

    out = torch.empty((S, H, D), dtype=torch.bfloat16, device=dev)
    need = _lib.load().sh_cells_attn_workspace(S, H, G, D, L)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    qd, kd, vd, gd = q.to(dev), k.to(dev), v.to(dev), gate.to(dev)
    td = torch.from_numpy(table).to(dev)
    cd = torch.from_numpy(cells).to(dev)
    rd = torch.from_numpy(real.astype(np.uint8)).to(dev)
    _lib.call("sh_cells_attn_paged", qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), td.data_ptr(), n_pages,
              cd.data_ptr(), rd.data_ptr(), L, S, H, G, D, 1 / 16, 2, gd.data_ptr(), H * D, D, out.data_ptr(),
              ws.data_ptr(), need, _lib.stream_of(qd))
    pos = np.arange(kv_len)
    kf = k.float().numpy()[table[pos // 16], :, pos % 16].transpose(1, 0, 2)[None]  # (1, G, kv_len, D) in order
    vf = v.float().numpy()[table[pos // 16], :, pos % 16].transpose(1, 0, 2)[None]
    att = OA.gathered(q.float().numpy().transpose(1, 0, 2)[None], kf, vf, cells, real, 1 / 16).reshape(S, H, D)
    want = OA.gate_out(att.astype(np.float32), gate.float().numpy(), "bfloat16")
    assert rel_err(out.float().cpu().numpy(), want) <= 1e-2


class Linear:
    def __init__(self, w):
        self.weight = w

    def __call__(self, x):
        return (x.float() @ self.weight.float().T).to(x.dtype)


def rope_of(rot, base=10000.0):
    inv = 1.0 / base ** (np.arange(0, rot, 2) / rot)

    def rope(positions):
        ang = positions.double().cpu().numpy()[:, None] * inv[None]
        ang = np.concatenate([ang, ang], axis=1)
        return torch.from_numpy(np.cos(ang)).float().to(positions.device), torch.from_numpy(np.sin(ang)).float().to(
            positions.device)

    return rope


def layer_want(layer, x, cache_k, cache_v, offset, rope, dtype):
    """The layer in float64 from the same projections: qk_rope (oracle), history + new keys, causal attention, the
    gate, o_proj."""
    S = x.shape[1]
    H, G, D = layer.n_heads, layer.n_kv_heads, layer.head_dim
    cos, sin = rope(torch.arange(offset, offset + S))
    cos, sin = OR.round_to(cos.numpy(), NAME[dtype]), OR.round_to(sin.numpy(), NAME[dtype])
    proj = layer.q_proj(x).float().cpu().numpy()[0]
    q = OA.qk_rope(proj, layer.q_norm_weight.float().cpu().numpy(), cos, sin, H, D, 2 * D, layer.eps, NAME[dtype])
    kn = OA.qk_rope(layer.k_proj(x).float().cpu().numpy()[0], layer.k_norm_weight.float().cpu().numpy(), cos, sin, G,
                    D, D, layer.eps, NAME[dtype])
    vn = layer.v_proj(x).float().cpu().numpy()[0].reshape(S, G, D)
    K = np.concatenate([cache_k, kn.transpose(1, 0, 2)])  # (ctx, G, D)
    V = np.concatenate([cache_v, vn])
    ctx = K.shape[0]
    out = np.zeros((S, H, D))
    group = H // G
    for t in range(S):
        seen = ctx - S + t + 1
        for h in range(H):
            s = K[:seen, h // group].astype(np.float64) @ q[h, t].astype(np.float64) * layer.scale
            p = np.exp(s - s.max())
            out[t, h] = (p / p.sum()) @ V[:seen, h // group]
    gated = OA.gate_out(out.astype(np.float32), proj.reshape(S, H, 2 * D)[..., D:], NAME[dtype])
    return gated.reshape(S, H * D).astype(np.float64) @ layer.o_proj.weight.float().cpu().numpy().T.astype(np.float64)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_an_attention_layer_through_a_verify_pass(dtype, dev):
    """A layer of 16 query heads and 2 KV heads of 256, rope on 64 dims: a prompt's keys and values already cached,
    then a window of 4 (a verify pass), 3 drafts rejected and trimmed, then a window of 2 that overwrites them."""
    rng = np.random.default_rng(11)
    dm, H, G, D, rot = 512, 16, 2, 256, 64

    def lin(rows, cols, s):
        return Linear(torch.from_numpy(rng.standard_normal((rows, cols)).astype(np.float32) * s).to(dtype).to(dev))

    layer = SA.Attention(lin(H * 2 * D, dm, 0.05), lin(G * D, dm, 0.05), lin(G * D, dm, 0.05), lin(dm, H * D, 0.02),
                         torch.from_numpy(1 + 0.1 * rng.standard_normal(D).astype(np.float32)).to(dtype).to(dev),
                         torch.from_numpy(1 + 0.1 * rng.standard_normal(D).astype(np.float32)).to(dtype).to(dev),
                         H, G, D)
    n_pages = 80
    cache = SA.PagedKVCache(n_pages, G, D, dtype, dev,
                            page_table=torch.from_numpy(rng.permutation(n_pages).astype(np.int32)))
    prompt = 1000
    k0 = torch.from_numpy(rng.standard_normal((prompt, G, D)).astype(np.float32)).to(dtype).to(dev)
    v0 = torch.from_numpy(rng.standard_normal((prompt, G, D)).astype(np.float32)).to(dtype).to(dev)
    cache.update_and_fetch(k0, v0)
    rope = rope_of(rot)
    hist_k, hist_v = k0.float().cpu().numpy(), v0.float().cpu().numpy()
    for S, reject in ((4, 3), (2, 0)):
        x = torch.from_numpy(rng.standard_normal((1, S, dm)).astype(np.float32)).to(dtype).to(dev)
        offset = cache.offset
        got = layer(x, rope, None, cache)
        assert got.shape == (1, S, dm) and cache.offset == offset + S
        want = layer_want(layer, x, hist_k, hist_v, offset, rope, dtype)
        assert rel_err(got.float().cpu().numpy()[0], want) <= 1e-2
        # what the cache now holds for the window: the keys after norm and rope, the values as projected
        pos = torch.arange(offset, offset + S, device=dev)
        phys = cache.page_table.long()[pos // 16]
        kw = cache.k_pages[phys, :, pos % 16].float().cpu().numpy()
        vw = cache.v_pages[phys, :, pos % 16].float().cpu().numpy()
        keep = S - reject
        hist_k, hist_v = np.concatenate([hist_k, kw[:keep]]), np.concatenate([hist_v, vw[:keep]])
        assert cache.trim(reject) == reject
