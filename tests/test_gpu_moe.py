"""One MoE block's decode step (route, gate/up + SwiGLU, down + combine) on the GPU against the oracle: the choice of
experts bit for bit, the routing weights to float32 rounding, the output within 1e-2 of max|want| (bf16/fp16)."""

import numpy as np
import pytest
import torch

from conftest import rel_err
from oracle import blocks as OB
from oracle import moe as OM
from strata_hip import blocks as SB
from strata_hip import fused as SF
from strata_hip import synth

pytestmark = pytest.mark.gpu


def layer(kind, kind_down, E, D, F, seed, dev, tables, sigma=0.02):
    rng = np.random.default_rng(seed)

    def blocks(k, rows, cols):
        return synth.random_blocks(k, rows, cols, rng, sigma=sigma)

    raw = {"gate": blocks(kind, E * F, D), "up": blocks(kind, E * F, D), "down": blocks(kind_down, E * D, F),
           "sgate": blocks(kind, F, D), "sup": blocks(kind, F, D), "sdown": blocks(kind_down, D, F)}
    kinds = {"gate": kind, "up": kind, "down": kind_down, "sgate": kind, "sup": kind, "sdown": kind_down}
    shapes = {"gate": (E, F, D), "up": (E, F, D), "down": (E, D, F), "sgate": (1, F, D), "sup": (1, F, D),
              "sdown": (1, D, F)}
    lin = {n: SB.BlockSwitchLinear(torch.from_numpy(raw[n]).to(dev), kinds[n], shapes[n]) for n in raw}
    w = {n: OB.dequantize(raw[n], kinds[n], shapes[n], tables) for n in raw}
    return lin, w, rng


@pytest.mark.parametrize("kinds", [("Q2_0", "Q2_0"), ("IQ3_S", "IQ3_S"), ("IQ3_S", "Q2_0")])
@pytest.mark.parametrize("tokens", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_moe_decode_is_the_oracles_block(kinds, tokens, dtype, tables, dev):
    E, D, F, K = 64, 512, 256, 10
    # IQ3_S weights reach 465 times their block scale: with fp16 activations smaller scales keep the block's values
    # finite (the oracle, like the reference, overflows otherwise)
    sigma = 0.002 if dtype == torch.float16 else 0.02
    lin, w, rng = layer(*kinds, E, D, F, tokens, dev, tables, sigma)
    name = "bfloat16" if dtype == torch.bfloat16 else "float16"
    x = torch.from_numpy(rng.standard_normal((tokens, D)).astype(np.float32)).to(dtype)
    logits = torch.from_numpy(rng.standard_normal((tokens, E)).astype(np.float32)).to(dtype)
    if tokens >= 4:
        logits[1] = logits[0]  # two tokens with one choice: groups of several tokens
        logits[3] = logits[0]
    wg = torch.from_numpy(rng.standard_normal(D).astype(np.float32) * 0.05).to(dtype)
    moe = SF.MoEDecode(lin["gate"], lin["up"], lin["down"], lin["sgate"], lin["sup"], lin["sdown"], wg.to(dev), K)
    out, idx, wt = moe(logits.to(dev), x.to(dev), want_choice=True)
    want, want_idx, want_w = OM.moe_decode(logits.float().numpy(), x.float().numpy(), K,
                                           (w["gate"], w["up"], w["down"]), (w["sgate"], w["sup"], w["sdown"]),
                                           wg.float().numpy(), name)
    np.testing.assert_array_equal(idx.cpu().numpy(), want_idx)
    np.testing.assert_allclose(wt.cpu().numpy(), want_w, rtol=2e-6, atol=1e-7)
    assert np.isfinite(want).all()
    assert rel_err(out.float().cpu(), want) <= 1e-2


@pytest.mark.parametrize("tokens", [1, 8])
def test_float32_logits_route_exactly(tokens, tables, dev):
    """A real router gives float32 logits (strata_mlx/fused.py:357-390): the choice is made on them, unrounded."""
    E, D, F, K = 128, 256, 256, 10
    lin, w, rng = layer("Q2_0", "Q2_0", E, D, F, 7, dev, tables)
    x = torch.from_numpy(rng.standard_normal((tokens, D)).astype(np.float32)).to(torch.bfloat16)
    logits = torch.from_numpy(rng.standard_normal((tokens, E)).astype(np.float32))
    logits[:, 5] = logits[:, 9]  # exact ties go to the lower index
    wg = torch.from_numpy(rng.standard_normal(D).astype(np.float32) * 0.05).to(torch.bfloat16)
    moe = SF.MoEDecode(lin["gate"], lin["up"], lin["down"], lin["sgate"], lin["sup"], lin["sdown"], wg.to(dev), K)
    out, idx, wt = moe(logits.to(dev), x.to(dev), want_choice=True)
    want, want_idx, want_w = OM.moe_decode(logits.numpy(), x.float().numpy(), K, (w["gate"], w["up"], w["down"]),
                                           (w["sgate"], w["sup"], w["sdown"]), wg.float().numpy(), "bfloat16")
    np.testing.assert_array_equal(idx.cpu().numpy(), want_idx)
    assert rel_err(out.float().cpu(), want) <= 1e-2


@pytest.mark.parametrize("E", [256, 1024, 2048])
@pytest.mark.parametrize("tokens, logit_dtype", [(1, torch.bfloat16), (3, torch.float32), (9, torch.bfloat16)])
def test_many_experts_route_exactly(E, tokens, logit_dtype, tables, dev):
    """The route at 4, 16 and 32 keys a lane (256, 1024 and 2048 experts), with ties at the k-th value, through the
    whole step at narrow widths (d 64, ffn 64: one Q2_0 block a row)."""
    D, F, K = 64, 64, 12
    lin, w, rng = layer("Q2_0", "Q2_0", E, D, F, E + tokens, dev, tables)
    x = torch.from_numpy(rng.standard_normal((tokens, D)).astype(np.float32)).to(torch.bfloat16)
    logits = torch.from_numpy(rng.standard_normal((tokens, E)).astype(np.float32)).to(logit_dtype)
    top = torch.topk(logits.float(), K, dim=1).indices
    logits[:, E - 1] = logits[torch.arange(tokens), top[:, K - 1]]  # the last expert ties with the k-th choice
    if tokens > 1:  # a token whose k-th choice falls among signed zeros: equal, chosen by index
        logits[1] = -logits[1].abs() - 1
        logits[1, :K - 2] = 1
        logits[1, K - 2::3] = -0.0
        logits[1, K - 1::3] = 0.0
    wg = torch.from_numpy(rng.standard_normal(D).astype(np.float32) * 0.05).to(torch.bfloat16)
    moe = SF.MoEDecode(lin["gate"], lin["up"], lin["down"], lin["sgate"], lin["sup"], lin["sdown"], wg.to(dev), K)
    assert moe.takes(x)
    out, idx, wt = moe(logits.to(dev), x.to(dev), want_choice=True)
    want, want_idx, want_w = OM.moe_decode(logits.float().numpy(), x.float().numpy(), K,
                                           (w["gate"], w["up"], w["down"]), (w["sgate"], w["sup"], w["sdown"]),
                                           wg.float().numpy(), "bfloat16")
    np.testing.assert_array_equal(idx.cpu().numpy(), want_idx)
    np.testing.assert_allclose(wt.cpu().numpy(), want_w, rtol=2e-6, atol=1e-7)
    assert rel_err(out.float().cpu(), want) <= 1e-2


@pytest.mark.parametrize("kinds, D, F", [(("Q2_0", "Q2_0"), 320, 64), (("Q2_0", "Q2_0"), 576, 192),
                                         (("Q2_0", "Q2_0"), 128, 320), (("IQ3_S", "Q2_0"), 768, 192)])
@pytest.mark.parametrize("tokens", [1, 5])
def test_widths_of_any_whole_blocks(kinds, D, F, tokens, tables, dev):
    """Rows of a number of scale groups that four waves do not split evenly (5, 9 and 2 Q2_0 blocks of gate / up):
    every group counted once."""
    E, K = 64, 6
    lin, w, rng = layer(*kinds, E, D, F, D + F + tokens, dev, tables)
    x = torch.from_numpy(rng.standard_normal((tokens, D)).astype(np.float32)).to(torch.bfloat16)
    logits = torch.from_numpy(rng.standard_normal((tokens, E)).astype(np.float32)).to(torch.bfloat16)
    wg = torch.from_numpy(rng.standard_normal(D).astype(np.float32) * 0.05).to(torch.bfloat16)
    moe = SF.MoEDecode(lin["gate"], lin["up"], lin["down"], lin["sgate"], lin["sup"], lin["sdown"], wg.to(dev), K)
    assert moe.takes(x)
    out = moe(logits.to(dev), x.to(dev))
    want, _, _ = OM.moe_decode(logits.float().numpy(), x.float().numpy(), K, (w["gate"], w["up"], w["down"]),
                               (w["sgate"], w["sup"], w["sdown"]), wg.float().numpy(), "bfloat16")
    assert rel_err(out.float().cpu(), want) <= 1e-2


def test_repeated_calls_reuse_the_workspace(tables, dev):
    """The down kernel's row-tile counters return to zero: call after call gives the same bits."""
    E, D, F, K = 64, 512, 256, 8
    lin, w, rng = layer("Q2_0", "Q2_0", E, D, F, 3, dev, tables)
    wg = torch.zeros(D, dtype=torch.bfloat16, device=dev)
    moe = SF.MoEDecode(lin["gate"], lin["up"], lin["down"], lin["sgate"], lin["sup"], lin["sdown"], wg, K)
    x = torch.randn(4, D, device=dev).to(torch.bfloat16)
    logits = torch.randn(4, E, device=dev).to(torch.bfloat16)
    first = moe(logits, x)
    for _ in range(5):
        assert torch.equal(moe(logits, x), first)


@pytest.fixture(scope="module")
def c3_layers(tables, dev):
    """The benchmark's layer shape (512 experts, d 2048, ffn 512), blocks made on the GPU: Q2_0, IQ3_S, and IQ3_S
    gate/up with Q2_0 down. The oracle fetches the chosen experts' bytes back."""
    E, D, F = 512, 2048, 512
    out = {}
    for n_k, kinds in enumerate((("Q2_0", "Q2_0"), ("IQ3_S", "IQ3_S"), ("IQ3_S", "Q2_0"))):
        kd = {"gate": kinds[0], "up": kinds[0], "down": kinds[1], "sgate": kinds[0], "sup": kinds[0],
              "sdown": kinds[1]}
        rc = {"gate": (E * F, D), "up": (E * F, D), "down": (E * D, F), "sgate": (F, D), "sup": (F, D),
              "sdown": (D, F)}
        shapes = {"gate": (E, F, D), "up": (E, F, D), "down": (E, D, F), "sgate": (1, F, D), "sup": (1, F, D),
                  "sdown": (1, D, F)}
        # IQ3_S weights reach 465 times their block scale: its smaller scales keep float16 products finite
        raw = {n: synth.random_blocks_gpu(kd[n], *rc[n], 40 + 10 * n_k + i, dev,
                                          sigma=0.0005 if kd[n] == "IQ3_S" else 0.01)
               for i, n in enumerate(rc)}
        lin = {n: SB.BlockSwitchLinear(raw[n], kd[n], shapes[n]) for n in raw}
        shared = tuple(OB.dequantize(raw[n].cpu().numpy(), kd[n], shapes[n], tables) for n in ("sgate", "sup", "sdown"))

        def fetcher(name, rows, cols, kind, stacks=raw):
            per = rows * OB.row_bytes(kind, cols)
            return lambda e: stacks[name][e * per:(e + 1) * per].cpu().numpy()

        fetch = (fetcher("gate", F, D, kinds[0]), fetcher("up", F, D, kinds[0]), fetcher("down", D, F, kinds[1]))
        out[kinds] = (fetch, lin, shared)
    return out


@pytest.mark.parametrize("kinds, tokens, dtype", [
    (("Q2_0", "Q2_0"), 1, torch.bfloat16), (("Q2_0", "Q2_0"), 4, torch.bfloat16),
    (("Q2_0", "Q2_0"), 8, torch.bfloat16), (("Q2_0", "Q2_0"), 16, torch.bfloat16),
    (("Q2_0", "Q2_0"), 2, torch.float16), (("IQ3_S", "IQ3_S"), 1, torch.bfloat16),
    (("IQ3_S", "IQ3_S"), 8, torch.bfloat16), (("IQ3_S", "IQ3_S"), 3, torch.float16),
    (("IQ3_S", "Q2_0"), 5, torch.bfloat16)])
def test_the_benchmark_shape_is_the_oracles_block(kinds, tokens, dtype, c3_layers, tables, dev):
    """512 experts, d 2048: route, gate and up in one kernel, then down and the combine."""
    E, D, F, K = 512, 2048, 512, 10
    fetch, lin, shared = c3_layers[kinds]
    rng = np.random.default_rng(tokens + 100)
    name = "bfloat16" if dtype == torch.bfloat16 else "float16"
    x = torch.from_numpy(rng.standard_normal((tokens, D)).astype(np.float32)).to(dtype)
    logits = torch.from_numpy(rng.standard_normal((tokens, E)).astype(np.float32)).to(dtype)
    if tokens >= 4:
        logits[2] = logits[0]  # tokens sharing their whole choice
    wg = torch.from_numpy(rng.standard_normal(D).astype(np.float32) * 0.05).to(dtype)
    moe = SF.MoEDecode(lin["gate"], lin["up"], lin["down"], lin["sgate"], lin["sup"], lin["sdown"], wg.to(dev), K)
    out, idx, wt = moe(logits.to(dev), x.to(dev), want_choice=True)
    want, want_idx, want_w = OM.moe_decode_blocks(logits.float().numpy(), x.float().numpy(), K, fetch, kinds,
                                                  (E, D, F), shared, wg.float().numpy(), tables, name)
    np.testing.assert_array_equal(idx.cpu().numpy(), want_idx)
    np.testing.assert_allclose(wt.cpu().numpy(), want_w, rtol=2e-6, atol=1e-7)
    assert np.isfinite(want).all()
    assert rel_err(out.float().cpu(), want) <= 1e-2


def test_the_benchmark_shape_with_float32_logits(c3_layers, tables, dev):
    E, D, F, K = 512, 2048, 512, 10
    fetch, lin, shared = c3_layers[("Q2_0", "Q2_0")]
    rng = np.random.default_rng(7)
    x = torch.from_numpy(rng.standard_normal((8, D)).astype(np.float32)).to(torch.bfloat16)
    logits = torch.from_numpy(rng.standard_normal((8, E)).astype(np.float32))
    logits[:, 5] = logits[:, 9]  # exact ties go to the lower index
    wg = torch.from_numpy(rng.standard_normal(D).astype(np.float32) * 0.05).to(torch.bfloat16)
    moe = SF.MoEDecode(lin["gate"], lin["up"], lin["down"], lin["sgate"], lin["sup"], lin["sdown"], wg.to(dev), K)
    out, idx, wt = moe(logits.to(dev), x.to(dev), want_choice=True)
    want, want_idx, _ = OM.moe_decode_blocks(logits.numpy(), x.float().numpy(), K, fetch, ("Q2_0", "Q2_0"),
                                             (E, D, F), shared, wg.float().numpy(), tables, "bfloat16")
    np.testing.assert_array_equal(idx.cpu().numpy(), want_idx)
    assert rel_err(out.float().cpu(), want) <= 1e-2
    for _ in range(3):  # the workspace reused: the same bits
        assert torch.equal(moe(logits.to(dev), x.to(dev)), out)


@pytest.mark.parametrize("logit_dtype", [torch.bfloat16, torch.float32])
def test_the_benchmark_shape_chooses_among_ties_by_index(logit_dtype, c3_layers, tables, dev):
    """Logits on a coarse grid: the k-th value is shared by many experts, so the choice among them (the lower
    indices first) decides which experts run; tokens 0-15, one of them with every logit equal."""
    E, D, F, K = 512, 2048, 512, 10
    fetch, lin, shared = c3_layers[("Q2_0", "Q2_0")]
    rng = np.random.default_rng(11)
    x = torch.from_numpy(rng.standard_normal((16, D)).astype(np.float32)).to(torch.bfloat16)
    logits = torch.from_numpy(np.round(rng.standard_normal((16, E)) * 2).astype(np.float32) / 2).to(logit_dtype)
    logits[3] = 0.25  # all tied: experts 0..9
    wg = torch.from_numpy(rng.standard_normal(D).astype(np.float32) * 0.05).to(torch.bfloat16)
    moe = SF.MoEDecode(lin["gate"], lin["up"], lin["down"], lin["sgate"], lin["sup"], lin["sdown"], wg.to(dev), K)
    out, idx, wt = moe(logits.to(dev), x.to(dev), want_choice=True)
    want, want_idx, want_w = OM.moe_decode_blocks(logits.float().numpy(), x.float().numpy(), K, fetch,
                                                  ("Q2_0", "Q2_0"), (E, D, F), shared, wg.float().numpy(), tables,
                                                  "bfloat16")
    np.testing.assert_array_equal(idx[3].cpu().numpy(), np.arange(K))
    np.testing.assert_array_equal(idx.cpu().numpy(), want_idx)
    np.testing.assert_allclose(wt.cpu().numpy(), want_w, rtol=2e-6, atol=1e-7)
    assert rel_err(out.float().cpu(), want) <= 1e-2


@pytest.mark.parametrize("tokens, k, dtype", [(1, 10, torch.bfloat16), (2, 7, torch.bfloat16), (3, 5, torch.float16),
                                              (1, 15, torch.float16)])
def test_the_benchmark_shape_with_few_groups(tokens, k, dtype, c3_layers, tables, dev):
    """At most 16 groups (the shared expert and the tokens' experts): the tail takes a wave a group and combines
    in LDS; against the oracle as every other window."""
    E, D, F = 512, 2048, 512
    fetch, lin, shared = c3_layers[("Q2_0", "Q2_0")]
    rng = np.random.default_rng(tokens * 31 + k)
    name = "bfloat16" if dtype == torch.bfloat16 else "float16"
    x = torch.from_numpy(rng.standard_normal((tokens, D)).astype(np.float32)).to(dtype)
    logits = torch.from_numpy(rng.standard_normal((tokens, E)).astype(np.float32)).to(dtype)
    wg = torch.from_numpy(rng.standard_normal(D).astype(np.float32) * 0.05).to(dtype)
    moe = SF.MoEDecode(lin["gate"], lin["up"], lin["down"], lin["sgate"], lin["sup"], lin["sdown"], wg.to(dev), k)
    out, idx, wt = moe(logits.to(dev), x.to(dev), want_choice=True)
    want, want_idx, want_w = OM.moe_decode_blocks(logits.float().numpy(), x.float().numpy(), k, fetch,
                                                  ("Q2_0", "Q2_0"), (E, D, F), shared, wg.float().numpy(), tables,
                                                  name)
    np.testing.assert_array_equal(idx.cpu().numpy(), want_idx)
    np.testing.assert_allclose(wt.cpu().numpy(), want_w, rtol=2e-6, atol=1e-7)
    assert rel_err(out.float().cpu(), want) <= 1e-2
    for _ in range(2):
        assert torch.equal(moe(logits.to(dev), x.to(dev)), out)


@pytest.mark.parametrize("kinds", [("Q2_0", "Q2_0"), ("IQ3_S", "IQ3_S")])
@pytest.mark.parametrize("tokens", [2, 3, 4])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_the_tails_own_combine_gives_the_combine_kernels_bits(kinds, tokens, dtype, c3_layers, tables, dev):
    """Windows of 2-4 tokens combine in the down kernel (its last block of a row tile, after a release / acquire
    hand-off of the routed outputs between blocks); larger ones in a combine kernel after it. The same inputs both
    ways give the same bits, call after call."""
    from strata_hip import _lib

    E, D, F, K = 512, 2048, 512, 10
    fetch, lin, shared = c3_layers[kinds]
    rng = np.random.default_rng(tokens + 300)
    x = torch.from_numpy(rng.standard_normal((tokens, D)).astype(np.float32)).to(dtype).to(dev)
    logits = torch.from_numpy(rng.standard_normal((tokens, E)).astype(np.float32)).to(dtype).to(dev)
    wg = torch.from_numpy(rng.standard_normal(D).astype(np.float32) * 0.05).to(dtype).to(dev)
    moe = SF.MoEDecode(lin["gate"], lin["up"], lin["down"], lin["sgate"], lin["sup"], lin["sdown"], wg, K)
    lib = _lib.load()
    before = lib.sh_moe_set_tail_combine(16)
    try:
        in_tail = moe(logits, x)
        torch.cuda.synchronize()
        lib.sh_moe_set_tail_combine(0)
        separate = moe(logits, x)
        torch.cuda.synchronize()
        assert torch.equal(in_tail, separate)
        lib.sh_moe_set_tail_combine(16)
        for _ in range(2):
            assert torch.equal(moe(logits, x), in_tail)
    finally:
        lib.sh_moe_set_tail_combine(before)
    name = "bfloat16" if dtype == torch.bfloat16 else "float16"
    want, _, _ = OM.moe_decode_blocks(logits.float().cpu().numpy(), x.float().cpu().numpy(), K, fetch, kinds,
                                      (E, D, F), shared, wg.float().cpu().numpy(), tables, name)
    assert rel_err(in_tail.float().cpu(), want) <= 1e-2


@pytest.mark.skip(reason="the one-launch layer is switched off: it made an illegal memory access at 2 tokens "
                         "(Q2_0, float16); the cause (direct loads inside the wait-state window after "
                         "v_readfirstlane wrote their base) is fixed but not yet run on a GPU; "
                         "sh_moe_set_one_launch(1) is refused")
@pytest.mark.parametrize("kinds", [("Q2_0", "Q2_0"), ("IQ3_S", "IQ3_S"), ("IQ3_S", "Q2_0")])
@pytest.mark.parametrize("tokens", [1, 2, 4, 5, 8, 16])
def test_one_launch_gives_the_two_kernels_bits(kinds, tokens, c3_layers, tables, dev):
    """The common shape's step as one launch (gate / up and down blocks in one grid, down waiting on its group's
    count) against the front and tail kernels launched one after the other: the same bits, call after call (the
    counts the launch leaves behind are cleared for the next)."""
    from strata_hip import _lib

    E, D, F, K = 512, 2048, 512, 10
    fetch, lin, shared = c3_layers[kinds]
    rng = np.random.default_rng(tokens + 500)
    x = torch.from_numpy(rng.standard_normal((tokens, D)).astype(np.float32)).to(torch.bfloat16).to(dev)
    logits = torch.from_numpy(rng.standard_normal((tokens, E)).astype(np.float32)).to(dev)
    wg = torch.from_numpy(rng.standard_normal(D).astype(np.float32) * 0.05).to(torch.bfloat16).to(dev)
    moe = SF.MoEDecode(lin["gate"], lin["up"], lin["down"], lin["sgate"], lin["sup"], lin["sdown"], wg, K)
    lib = _lib.load()
    before = lib.sh_moe_set_one_launch(0)
    try:
        two, idx2, w2 = moe(logits, x, want_choice=True)
        torch.cuda.synchronize()
        lib.sh_moe_set_one_launch(1)
        for _ in range(3):
            one, idx1, w1 = moe(logits, x, want_choice=True)
            torch.cuda.synchronize()
            assert torch.equal(one, two) and torch.equal(idx1, idx2) and torch.equal(w1, w2)
    finally:
        lib.sh_moe_set_one_launch(before)
    want, _, _ = OM.moe_decode_blocks(logits.cpu().numpy(), x.float().cpu().numpy(), K, fetch, kinds, (E, D, F),
                                      shared, wg.float().cpu().numpy(), tables, "bfloat16")
    assert rel_err(one.float().cpu(), want) <= 1e-2


@pytest.mark.parametrize("kinds", [("Q2_0", "Q2_0"), ("IQ3_S", "Q2_0")])
def test_one_workspace_serves_every_token_count(kinds, c3_layers, tables, dev):
    """One zeroed workspace, sized for 16 tokens, passed to calls of 16, 2, 8, 1 and 5 tokens in turn: the launch's
    counters sit at the workspace's head whatever the shape, so each call starts from the zeros the one before
    left, and gives the bits of a call with a workspace of its own."""
    E, D, F, K = 512, 2048, 512, 10
    fetch, lin, shared = c3_layers[kinds]
    wg = (torch.randn(D, device=dev, generator=torch.Generator(device=dev).manual_seed(9)) * 0.05).to(torch.bfloat16)
    fresh = SF.MoEDecode(lin["gate"], lin["up"], lin["down"], lin["sgate"], lin["sup"], lin["sdown"], wg, K)
    shared_ws = SF.MoEDecode(lin["gate"], lin["up"], lin["down"], lin["sgate"], lin["sup"], lin["sdown"], wg, K)
    big = fresh.workspace(16, torch.bfloat16, dev).clone()
    shared_ws.workspace = lambda tokens, dtype, device: big
    rng = np.random.default_rng(77)
    for tokens in (16, 2, 8, 1, 5):
        x = torch.from_numpy(rng.standard_normal((tokens, D)).astype(np.float32)).to(torch.bfloat16).to(dev)
        logits = torch.from_numpy(rng.standard_normal((tokens, E)).astype(np.float32)).to(dev)
        want, want_idx, want_w = fresh(logits, x, want_choice=True)
        got, idx, w = shared_ws(logits, x, want_choice=True)
        torch.cuda.synchronize()
        assert torch.equal(got, want) and torch.equal(idx, want_idx) and torch.equal(w, want_w), tokens


@pytest.fixture(scope="module")
def model_width_layers(tables, dev):
    """Layers at the reference model's widths, built once (the oracle's weights of 64 experts take seconds)."""
    E, D, F = 64, 2560, 640
    # small scales: IQ3_S weights reach 465 times theirs, and float16 products must stay finite
    return {kinds: layer(*kinds, E, D, F, 50 + n, dev, tables, 0.002)
            for n, kinds in enumerate((("Q2_0", "Q2_0"), ("IQ3_S", "Q2_0")))}


@pytest.mark.parametrize("kinds", [("Q2_0", "Q2_0"), ("IQ3_S", "Q2_0")])
@pytest.mark.parametrize("tokens, dtype", [(1, torch.bfloat16), (3, torch.float16), (8, torch.bfloat16),
                                           (16, torch.bfloat16)])
def test_the_reference_models_widths(kinds, tokens, dtype, model_width_layers, tables, dev):
    """d_model 2560, d_ff 640 (the reference model's, bench/blocks_matvec.py:18): gate / up rows of 40 Q2_0 blocks or
    10 IQ3_S ones, down rows of 10 Q2_0 blocks (640 is no whole IQ3_S block): the fused step takes them (route,
    gate / up, down + combine) and gives the oracle's block."""
    E, D, F, K = 64, 2560, 640, 10
    lin, w, _ = model_width_layers[kinds]
    rng = np.random.default_rng(60 + tokens)
    name = "bfloat16" if dtype == torch.bfloat16 else "float16"
    x = torch.from_numpy(rng.standard_normal((tokens, D)).astype(np.float32)).to(dtype)
    logits = torch.from_numpy(rng.standard_normal((tokens, E)).astype(np.float32))
    wg = torch.from_numpy(rng.standard_normal(D).astype(np.float32) * 0.05).to(dtype)
    moe = SF.MoEDecode(lin["gate"], lin["up"], lin["down"], lin["sgate"], lin["sup"], lin["sdown"], wg.to(dev), K)
    assert moe.takes(x)
    out, idx, wt = moe(logits.to(dev), x.to(dev), want_choice=True)
    want, want_idx, want_w = OM.moe_decode(logits.numpy(), x.float().numpy(), K, (w["gate"], w["up"], w["down"]),
                                           (w["sgate"], w["sup"], w["sdown"]), wg.float().numpy(), name)
    np.testing.assert_array_equal(idx.cpu().numpy(), want_idx)
    np.testing.assert_allclose(wt.cpu().numpy(), want_w, rtol=2e-6, atol=1e-7)
    assert np.isfinite(want).all()
    assert rel_err(out.float().cpu(), want) <= 1e-2
