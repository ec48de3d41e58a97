"""A MoE layer read from a GGUF file (strata_hip/gguf.py, after strata_mlx/gguf.py and load.py:411-421) and the
paged experts of strata_mlx/paged.py:373-419, on the GPU against the oracle from the file's own bytes."""

import numpy as np
import pytest
import torch

from conftest import rel_err
from gguf_write import write
from oracle import blocks as OB
from oracle import moe as OM
from strata_hip import blocks as SB
from strata_hip import gguf as G
from strata_hip import paged as SP
from strata_hip import synth

pytestmark = pytest.mark.gpu
E, D, F, K = 64, 512, 256, 4


@pytest.fixture(scope="module")
def model_file(tmp_path_factory, tables):
    rng = np.random.default_rng(21)
    t = {}
    for part, (r, c) in (("gate", (F, D)), ("up", (F, D)), ("down", (D, F))):
        t[f"blk.0.ffn_{part}_exps.weight"] = ((E, r, c), "Q2_0", synth.random_blocks("Q2_0", E * r, c, rng, sigma=0.01))
        t[f"blk.0.ffn_{part}_shexp.weight"] = ((r, c), "Q2_0", synth.random_blocks("Q2_0", r, c, rng, sigma=0.01))
    router = (rng.standard_normal((E, D)) * 0.05).astype(np.float16)
    sgate = (rng.standard_normal(D) * 0.05).astype(np.float16)
    t["blk.0.ffn_gate_inp.weight"] = ((E, D), "F16", router.view(np.uint8))
    t["blk.0.ffn_gate_inp_shexp.weight"] = ((D,), "F16", sgate.view(np.uint8))
    path = str(tmp_path_factory.mktemp("model") / "moe.gguf")
    write(path, {"general.architecture": "qwen4exp", "qwen4exp.expert_used_count": K},
          [(n, s, k, raw) for n, (s, k, raw) in t.items()])
    w = {n: OB.dequantize(raw, k, s if len(s) == 3 else (1,) + s, tables) for n, (s, k, raw) in t.items()
         if k == "Q2_0"}
    return G.GGUF(path), w, router, sgate


@pytest.mark.parametrize("tokens", [3, 20])
def test_a_moe_layer_from_a_file(tokens, model_file, tables, dev):
    g, w, router, sgate = model_file
    block = G.moe_layer(g, 0, dev)
    rng = np.random.default_rng(tokens)
    x = torch.from_numpy(rng.standard_normal((1, tokens, D)).astype(np.float32)).to(torch.float16).to(dev)
    got = block(x)
    assert (block._fused_for(x) is not None) == (tokens <= 16)
    logits = (x.float() @ torch.from_numpy(router).float().to(dev).T)[0].cpu().numpy()
    p = "blk.0.ffn_{}_{}.weight"
    stacks = tuple(w[p.format(n, "exps")] for n in ("gate", "up", "down"))
    shared = tuple(w[p.format(n, "shexp")] for n in ("gate", "up", "down"))
    if tokens > 8:  # past a window the shared expert's block layers multiply weights unpacked to the type
        from oracle import route as OR

        shared = tuple(OR.round_to(m, "float16") for m in shared)
    want, _, _ = OM.moe_decode(logits, x.float().cpu().numpy()[0], K, stacks, shared, sgate.astype(np.float32),
                               "float16")
    assert rel_err(got.float().cpu().numpy()[0], want) <= 1e-2


@pytest.mark.parametrize("tokens", [3, 40])
def test_paged_experts(tokens, model_file, tables, dev):
    """A window of 12 pairs: each pair's expert read where it lies (`_separately`); of 160: stacks of the used
    experts. Against the layer's stacks held whole and the oracle."""
    g, w, _, _ = model_file
    names = [f"blk.0.ffn_{n}_exps.weight" for n in ("gate", "up", "down")]
    store = SP.ExpertStore(dev, budget=1 << 20)
    paged = SP.PagedSwitchGLU(0, store, *(g[n] for n in names))
    whole = SB.BlockSwitchGLU(*(SB.BlockSwitchLinear(torch.from_numpy(np.ascontiguousarray(g[n].data)).to(dev),
                                                     "Q2_0", g[n].shape) for n in names))
    rng = np.random.default_rng(tokens + 1)
    idx = np.stack([rng.choice(E, K, replace=False) for _ in range(tokens)])[None]
    x = torch.from_numpy(rng.standard_normal((1, tokens, D)).astype(np.float32)).to(torch.float16).to(dev)
    got = paged(x, torch.from_numpy(idx).to(dev))
    ref = whole(x, torch.from_numpy(idx).to(dev))
    assert got.shape == ref.shape == (1, tokens, K, D)
    want = OM.expert_products(*(w[n] for n in names), idx[0], x.float().cpu().numpy()[0], "float16")
    assert rel_err(got.float().cpu().numpy()[0], want) <= 1e-2
    assert rel_err(got.float().cpu().numpy(), ref.float().cpu().numpy()) <= 1e-2
    assert store.misses > 0 and (store.held <= store.budget or len(store.lru) == len(np.unique(idx)))
    again = paged(x, torch.from_numpy(idx).to(dev))
    assert torch.equal(again, got)
