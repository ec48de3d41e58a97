"""Decode attention on the GPU against the oracle's textbook SDPA over the gathered keys and values: paged
(context sizes around page and split edges, 1..8 queries, causal among the window) and the cell-list form of
`_gathered` (strata_mlx/attention.py:132-165). Outputs within 1e-2 of max|want| (bf16 / fp16, fp32 softmax)."""

import numpy as np
import pytest
import torch

from conftest import rel_err
from oracle import attention as OA
from strata_hip import attention as SA

pytestmark = pytest.mark.gpu


def pages(rng, n_pages, hkv, d, dtype):
    k = torch.from_numpy(rng.standard_normal((n_pages, hkv, 16, d)).astype(np.float32)).to(dtype)
    v = torch.from_numpy(rng.standard_normal((n_pages, hkv, 16, d)).astype(np.float32)).to(dtype)
    return k, v


@pytest.mark.parametrize("ctx", [1, 15, 16, 17, 100, 1000, 4096])
@pytest.mark.parametrize("B", [1, 3, 8])
def test_paged_attention_is_the_oracles(ctx, B, dev):
    if B > ctx:
        pytest.skip("more queries than positions")
    rng = np.random.default_rng(ctx * 10 + B)
    Hq, Hkv, D = 16, 2, 256
    n_log = -(-ctx // 16)
    n_pages = n_log + 3
    k, v = pages(rng, n_pages, Hkv, D, torch.bfloat16)
    table = rng.permutation(n_pages)[:n_log].astype(np.int32)  # shuffled physical pages, some unused
    q = torch.from_numpy(rng.standard_normal((B, Hq, D)).astype(np.float32)).to(torch.bfloat16)
    got = SA.paged_decode_attention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(table).to(dev), ctx)
    want = OA.paged_decode(q.float().numpy(), k.float().numpy(), v.float().numpy(), table, ctx, 1 / 16)
    assert got.shape == (B, Hq, D) and got.dtype == torch.bfloat16
    assert rel_err(got.float().cpu(), want) <= 1e-2


@pytest.mark.parametrize("B", [1, 2, 4, 5, 8])
def test_paged_attention_group_shapes(B, dev):
    """Query rows B * group = 8..64 fill one to four row tiles of 16; fp16 and head_dim 128 too."""
    rng = np.random.default_rng(100 + B)
    for Hq, Hkv, D, dtype in ((16, 2, 256, torch.float16), (8, 1, 128, torch.bfloat16), (32, 4, 128, torch.float16)):
        ctx = 300 + B
        n_pages = -(-ctx // 16)
        k, v = pages(rng, n_pages, Hkv, D, dtype)
        table = rng.permutation(n_pages).astype(np.int32)
        q = torch.from_numpy(rng.standard_normal((B, Hq, D)).astype(np.float32)).to(dtype)
        got = SA.paged_decode_attention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(table).to(dev), ctx,
                                        scale=0.07)
        want = OA.paged_decode(q.float().numpy(), k.float().numpy(), v.float().numpy(), table, ctx, 0.07)
        assert rel_err(got.float().cpu(), want) <= 1e-2, (Hq, Hkv, D, dtype)


def test_paged_attention_long_context(dev):
    """32K positions: many splits merged."""
    rng = np.random.default_rng(7)
    ctx, B, Hq, Hkv, D = 32768, 4, 16, 2, 256
    n_pages = ctx // 16
    k, v = pages(rng, n_pages, Hkv, D, torch.bfloat16)
    table = rng.permutation(n_pages).astype(np.int32)
    q = torch.from_numpy(rng.standard_normal((B, Hq, D)).astype(np.float32)).to(torch.bfloat16)
    got = SA.paged_decode_attention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(table).to(dev), ctx)
    want = OA.paged_decode(q.float().numpy(), k.float().numpy(), v.float().numpy(), table, ctx, 1 / 16)
    assert rel_err(got.float().cpu(), want) <= 1e-2


def test_sharp_scores_stay_finite(dev):
    """Large scores (scale 1): the running max must keep exp in range."""
    rng = np.random.default_rng(8)
    ctx, B, Hq, Hkv, D = 513, 2, 16, 2, 256
    n_pages = -(-ctx // 16)
    k, v = pages(rng, n_pages, Hkv, D, torch.bfloat16)
    table = np.arange(n_pages, dtype=np.int32)
    q = torch.from_numpy(rng.standard_normal((B, Hq, D)).astype(np.float32)).to(torch.bfloat16)
    got = SA.paged_decode_attention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(table).to(dev), ctx, scale=1.0)
    want = OA.paged_decode(q.float().numpy(), k.float().numpy(), v.float().numpy(), table, ctx, 1.0)
    assert torch.isfinite(got.float()).all()
    assert rel_err(got.float().cpu(), want) <= 1e-2


@pytest.mark.parametrize("S, L", [(1, 36), (3, 20), (4, 2052)])
def test_gathered_is_the_oracles(S, L, dev):
    rng = np.random.default_rng(S * 1000 + L)
    H, G, D, kv_len = 16, 2, 256, 3000
    q = torch.from_numpy(rng.standard_normal((1, H, S, D)).astype(np.float32)).to(torch.bfloat16)
    k = torch.from_numpy(rng.standard_normal((1, G, kv_len, D)).astype(np.float32)).to(torch.bfloat16)
    v = torch.from_numpy(rng.standard_normal((1, G, kv_len, D)).astype(np.float32)).to(torch.bfloat16)
    cells = rng.integers(0, kv_len, (S, L)).astype(np.int32)
    real = rng.random((S, L)) < 0.8
    real[:, 0] = True
    got = SA._gathered(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(cells).to(dev),
                       torch.from_numpy(real).to(dev), 1 / 16)
    want = OA.gathered(q.float().numpy(), k.float().numpy(), v.float().numpy(), cells, real, 1 / 16)
    assert got.shape == (1, S, H * D)
    assert rel_err(got.float().cpu(), want) <= 1e-2


def test_cells_lists_match_the_reference_rule(dev):
    """attention.py:132-141 on a small choice: chosen blocks' cells, then the query's own block up to itself."""
    top = torch.tensor([[0, 2], [1, 0]], device=dev)
    picked = torch.tensor([[True, False], [True, True]], device=dev)
    whole = torch.tensor([3, 3], device=dev)
    cells, real = SA._cells((top, picked, whole), 4, 2, 14)
    assert cells.cpu().tolist() == [[0, 1, 2, 3, 8, 9, 10, 11, 12, 13, 13, 13],
                                    [4, 5, 6, 7, 0, 1, 2, 3, 12, 13, 13, 13]]
    assert real.cpu().tolist() == [[True] * 4 + [False] * 4 + [True, False, False, False],
                                   [True] * 8 + [True, True, False, False]]
