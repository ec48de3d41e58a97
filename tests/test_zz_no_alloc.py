"""sh_moe_decode_noalloc, the MoE decode step with the library's own scratch array for its workspace (no
allocation), against sh_moe_decode with a workspace the caller allocated: the same bits, output and choice, on two
calls in a row, the second with fewer tokens; on the two-kernel benchmark shape and on the three-kernel general
shape. Shapes whose workspace exceeds the array are refused before anything is launched."""

import numpy as np
import pytest
import torch

from strata_hip import _lib
from strata_hip import blocks as SB
from strata_hip import fused as SF
from strata_hip import synth

pytestmark = pytest.mark.gpu


def moe_layer(kinds, E, D, F, K, seed, dev):
    shapes = {"gate": (E, F, D), "up": (E, F, D), "down": (E, D, F), "sgate": (1, F, D), "sup": (1, F, D),
              "sdown": (1, D, F)}
    kd = {"gate": kinds[0], "up": kinds[0], "down": kinds[1], "sgate": kinds[0], "sup": kinds[0], "sdown": kinds[1]}
    lin = {n: SB.BlockSwitchLinear(synth.random_blocks_gpu(kd[n], s[0] * s[1], s[2], seed + i, dev, sigma=0.002),
                                   kd[n], s) for i, (n, s) in enumerate(shapes.items())}
    wg = (torch.randn(D, device=dev) * 0.05).to(torch.bfloat16)
    return SF.MoEDecode(lin["gate"], lin["up"], lin["down"], lin["sgate"], lin["sup"], lin["sdown"], wg, K)


@pytest.mark.parametrize("kinds, E, D, F", [(("Q2_0", "Q2_0"), 512, 2048, 512), (("IQ3_S", "IQ3_S"), 512, 2048, 512),
                                            (("Q2_0", "IQ3_S"), 64, 512, 256)])
def test_noalloc_decode_gives_the_workspace_decodes_bits(kinds, E, D, F, tables, dev):
    K = 10
    moe = moe_layer(kinds, E, D, F, K, 70, dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(71)
    for tokens in (8, 2):  # the second call smaller than the first: nothing left over may matter
        x = torch.randn((tokens, D), generator=gen, device=dev).to(torch.bfloat16)
        logits = torch.randn((tokens, E), generator=gen, device=dev)
        want, want_idx, want_w = moe(logits, x, want_choice=True)
        out = torch.empty_like(x)
        idx = torch.empty((tokens, K), dtype=torch.int32, device=dev)
        w = torch.empty((tokens, K), dtype=torch.float32, device=dev)
        moe.decode_into(logits, x, out, idx, w)
        torch.cuda.synchronize()
        assert torch.equal(out, want) and torch.equal(idx, want_idx) and torch.equal(w, want_w)
        assert torch.isfinite(out.float()).all()


def test_noalloc_decode_refuses_what_its_array_cannot_hold(dev):
    lib = _lib.load()
    assert lib.sh_moe_scratch_bytes() == 8 << 20
    dummy = torch.zeros(16, dtype=torch.uint8, device=dev)
    p = dummy.data_ptr()
    # 16 tokens x 16 experts at d_model 8192: about 9 MB of workspace
    need = lib.sh_moe_workspace(16, 16, 8192, 512, 2)
    assert need > lib.sh_moe_scratch_bytes()
    st = lib.sh_moe_decode_noalloc(0, 0, p, p, p, 64, p, p, p, p, None, p, 0, p, 2, 16, 16, 8192, 512, p, None, None,
                                   None)
    assert st == -6 and b"scratch" in lib.sh_last_error()
