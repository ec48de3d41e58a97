"""The oracle's attention, pinned without itself: torch's scaled_dot_product_attention in float64 on the CPU (an
independent implementation), a dense restatement that inverts the page table, and closed forms (equal keys give
the mean of the visible values; one dominant score picks its value). CPU only."""

import numpy as np
import pytest
import torch

from oracle import attention as OA


def test_sdpa_is_torchs(rng=np.random.default_rng(1)):
    q, k, v = rng.standard_normal((5, 32)), rng.standard_normal((40, 32)), rng.standard_normal((40, 32))
    mask = rng.random((5, 40)) < 0.7
    mask[:, 0] = True
    got = OA.sdpa(q, k, v, mask, 0.3)
    want = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q)[None], torch.from_numpy(k)[None], torch.from_numpy(v)[None],
        attn_mask=torch.from_numpy(mask)[None], scale=0.3)[0].numpy()
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("ctx, B", [(1, 1), (17, 3), (64, 8), (100, 5)])
def test_paged_decode_is_dense_causal_attention(ctx, B):
    rng = np.random.default_rng(ctx + B)
    Hq, Hkv, D = 8, 2, 16
    n_log = -(-ctx // 16)
    k, v = rng.standard_normal((n_log + 2, Hkv, 16, D)), rng.standard_normal((n_log + 2, Hkv, 16, D))
    table = rng.permutation(n_log + 2)[:n_log]
    q = rng.standard_normal((B, Hq, D))
    got = OA.paged_decode(q, k, v, table, ctx, 0.25)
    # dense K / V of each head by walking the table page by page, then one torch SDPA per head with a causal mask
    K = np.concatenate([k[table[p]] for p in range(n_log)], axis=1)[:, :ctx]  # (Hkv, ctx, D)
    V = np.concatenate([v[table[p]] for p in range(n_log)], axis=1)[:, :ctx]
    mask = np.arange(ctx)[None, :] <= (ctx - B + np.arange(B))[:, None]  # (B, ctx)
    group = Hq // Hkv
    for h in range(Hkv):
        qs = torch.from_numpy(q[:, h * group:(h + 1) * group]).transpose(0, 1)  # (group, B, D)
        want = torch.nn.functional.scaled_dot_product_attention(
            qs, torch.from_numpy(K[h])[None].expand(group, -1, -1), torch.from_numpy(V[h])[None].expand(group, -1, -1),
            attn_mask=torch.from_numpy(mask)[None], scale=0.25).transpose(0, 1).numpy()
        np.testing.assert_allclose(got[:, h * group:(h + 1) * group], want, rtol=1e-10, atol=1e-10)


def test_equal_keys_average_the_visible_values():
    rng = np.random.default_rng(3)
    ctx, B, D = 40, 4, 8
    k = np.ones((3, 1, 16, D))
    v = rng.standard_normal((3, 1, 16, D))
    table = np.array([2, 0, 1])
    q = rng.standard_normal((B, 2, D))
    got = OA.paged_decode(q, k, v, table, ctx, 1.0)
    V = np.concatenate([v[p, 0] for p in table])[:ctx]
    for t in range(B):
        np.testing.assert_allclose(got[t], np.broadcast_to(V[:ctx - B + t + 1].mean(0), (2, D)), rtol=1e-12)


def test_one_dominant_score_picks_its_value():
    rng = np.random.default_rng(4)
    D = 8
    k = rng.standard_normal((2, 1, 16, D)) * 0.01
    k[1, 0, 3] = 50.0  # position 19
    v = rng.standard_normal((2, 1, 16, D))
    q = np.ones((1, 1, D))
    got = OA.paged_decode(q, k, v, np.array([0, 1]), 32, 1.0)
    np.testing.assert_allclose(got[0, 0], v[1, 0, 3], rtol=1e-12)


def test_gathered_over_every_cell_is_dense_attention():
    rng = np.random.default_rng(5)
    H, G, S, D, kv = 4, 2, 3, 8, 20
    q = rng.standard_normal((1, H, S, D))
    k, v = rng.standard_normal((1, G, kv, D)), rng.standard_normal((1, G, kv, D))
    cells = np.tile(np.arange(kv), (S, 1))
    real = np.ones((S, kv), bool)
    real[1, 5:] = False
    got = OA.gathered(q, k, v, cells, real, 0.5)
    for s in range(S):
        for h in range(H):
            g = h // (H // G)
            m = real[s]
            sc = (k[0, g, m] @ q[0, h, s]) * 0.5
            p = np.exp(sc - sc.max())
            want = (p / p.sum()) @ v[0, g, m]
            np.testing.assert_allclose(got[0, s, h * D:(h + 1) * D], want, rtol=1e-12)
