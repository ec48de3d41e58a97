"""The hyper-connection read (strata_hip.hc.FusedResidual, strata_mlx/fused.py:281-323) on the GPU against the oracle
(oracle/hc.py), at the reference's own test shape in spirit (4 streams, a low rank) and at a model's width (4 x 2560,
rank 128): the reference's tolerances (2e-5 of the largest value in float32, 4e-3 in float16; 1e-2 in bfloat16),
the residual exact where nothing is written before, and a token's bits the same alone and in a window."""

import os

import numpy as np
import pytest
import torch

from oracle import hc as OH
from oracle.route import round_to
from strata_hip import hc as SH

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(os.environ.get("STRATA_HOSTRUN") != "1",
                                 reason="not yet run on a GPU: written while this repository's GPU runs were closed; "
                                        "the next GPU session runs it first (it runs on the host build)")]

TORCH = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}
TOL = {"float32": 2e-5, "float16": 4e-3, "bfloat16": 1e-2}


def weights(rng, hc, D, R, inject, wdt):
    HD = hc * D
    norm = (1 + 0.2 * rng.standard_normal(HD)).astype(np.float32)
    down = round_to(rng.standard_normal((R, HD)) / np.sqrt(HD), wdt)
    up = round_to(rng.standard_normal((HD, R)) / np.sqrt(R), wdt)
    inject_w = round_to(rng.standard_normal((hc, HD)) / np.sqrt(HD), wdt) if inject else None
    return norm, down, up, inject_w


def inputs(rng, T, hc, D, dtype):
    return (round_to(rng.standard_normal((T, hc * D)), dtype), round_to(rng.standard_normal((T, D)), dtype),
            round_to(2 * rng.random((T, hc)), dtype))


def on(a, dt, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(TORCH[dt]).to(dev)


@pytest.mark.parametrize("T, hc, D, R, inject", [(1, 4, 128, 32, True), (2, 4, 128, 32, False), (5, 4, 256, 64, True),
                                                  (8, 4, 2560, 128, True), (16, 2, 512, 64, True),
                                                  (3, 8, 64, 32, True), (20, 4, 128, 32, True)])
@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
def test_the_read_is_the_oracles(T, hc, D, R, inject, dtype, dev):
    rng = np.random.default_rng(T * 1000 + D + R)
    wdt = "float32" if dtype == "float32" else dtype
    norm, down, up, inject_w = weights(rng, hc, D, R, inject, wdt)
    before, out, inject_in = inputs(rng, T, hc, D, dtype)
    want = OH.fused_residual(before, out, inject_in, norm, down, up, inject_w, hc, 1e-6, dtype)
    fr = SH.FusedResidual.from_weights(torch.from_numpy(norm).to(dev), on(down, wdt, dev), on(up, wdt, dev),
                                       None if inject_w is None else on(inject_w, wdt, dev), hc)
    got = fr(on(before, dtype, dev)[None], on(out, dtype, dev)[None], on(inject_in, dtype, dev)[None])
    torch.cuda.synchronize()
    for g, w in zip(got, want):
        g = g[0].float().cpu().numpy()
        assert g.shape == w.shape
        assert np.abs(g - w).max() <= TOL[dtype] * np.abs(w).max()


@pytest.mark.parametrize("dtype", ["float32", "float16"])
def test_nothing_before_is_a_plain_read(dtype, dev):
    rng = np.random.default_rng(6)
    norm, down, up, inject_w = weights(rng, 4, 128, 32, True, dtype)
    before = round_to(rng.standard_normal((2, 512)), dtype)
    fr = SH.FusedResidual.from_weights(torch.from_numpy(norm).to(dev), on(down, dtype, dev), on(up, dtype, dev),
                                       on(inject_w, dtype, dev), 4)
    b = on(before, dtype, dev)[None]
    mixed, residual, inject = fr(b, torch.zeros((1, 2, 128), dtype=TORCH[dtype], device=dev),
                                 torch.zeros((1, 2, 4), dtype=TORCH[dtype], device=dev))
    assert torch.equal(residual, b)


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
def test_a_token_gets_the_same_bits_alone_and_in_a_window(dtype, dev):
    rng = np.random.default_rng(7)
    norm, down, up, inject_w = weights(rng, 4, 256, 64, True, dtype)
    before, out, inject_in = (on(a, dtype, dev)[None] for a in inputs(rng, 6, 4, 256, dtype))
    fr = SH.FusedResidual.from_weights(torch.from_numpy(norm).to(dev), on(down, dtype, dev), on(up, dtype, dev),
                                       on(inject_w, dtype, dev), 4)
    window = fr(before, out, inject_in)
    for t in range(6):
        alone = fr(before[:, t:t + 1], out[:, t:t + 1], inject_in[:, t:t + 1])
        assert all(torch.equal(a, w[:, t:t + 1]) for a, w in zip(alone, window))
