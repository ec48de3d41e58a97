"""Host-side logic of the drop-in (no GPU): the branch rules that must answer as the reference's do, and the block
swap install_routers performs (strata_mlx/fused.py:500-507)."""

import torch

from strata_hip import blocks as SB
from strata_hip import fused as SF


def test_what_fits_in_tiles():
    """tests/test_blocks.py:208-211, and rows of 64-column Q2_0 blocks that end inside a chunk of 256."""
    assert SB.tileable("Q2_0", 640, 2560) and SB.tileable("IQ3_S", 640, 2560) and SB.tileable("IQ4_NL", 2560, 640)
    assert not SB.tileable("IQ3_S", 2560, 640)  # its blocks are 256 weights: a row of 640 does not end on one
    assert not SB.tileable("Q2_0", 2, 2560)  # rows by the 64
    assert SB.tileable("Q2_0", 2560, 640) and SB.tileable("Q2_0", 128, 192)
    assert not SB.tileable("Q2_0", 128, 96)  # columns by the 64


class Linear(torch.nn.Module):
    def __init__(self, rows, cols):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.zeros(rows, cols, dtype=torch.float16), requires_grad=False)

    def forward(self, x):
        return x @ self.weight.T


class Block(torch.nn.Module):
    """A MoE block with the attributes of mlx-lm's SparseMoeBlock."""

    def __init__(self):
        super().__init__()
        self.gate = Linear(8, 16)
        self.switch_mlp = None
        self.shared_expert = None
        self.shared_expert_gate = Linear(1, 16)
        self.top_k = 2

    def forward(self, x):
        raise AssertionError("the block's own call")


class Layer:
    def __init__(self, mlp):
        self.mlp = mlp


def test_install_routers_swaps_the_blocks_class_in_place():
    blocks = [Block(), Block()]
    layers = [Layer(b) for b in blocks] + [Layer(None), Layer(torch.nn.Identity())]
    gate = blocks[0].gate
    SF.install_routers(layers)
    for b, layer in zip(blocks, layers):
        assert layer.mlp is b  # the same object: its parameters stay where they are
        assert isinstance(b, SF._RoutedCall) and isinstance(b, Block)
        assert isinstance(b.gate, SF.WindowLinear)
    assert blocks[0].gate.linear is gate and blocks[0].gate.weight is gate.weight
    assert type(blocks[0]) is type(blocks[1])  # one subclass a block class
    assert not isinstance(layers[3].mlp, SF._RoutedCall)
    SF.install_routers(layers)  # twice: nothing more happens
    assert isinstance(blocks[0].gate.linear, Linear)


def test_window_linear_answers_like_the_references():
    lin = Linear(8, 16)
    wl = SF.WindowLinear(lin)
    assert wl.takes(torch.zeros(1, 8, 16, dtype=torch.float16))
    assert not wl.takes(torch.zeros(1, 9, 16, dtype=torch.float16))  # more than a window: the layer itself
    x = torch.ones(1, 9, 16, dtype=torch.float16)
    lin.weight.data.fill_(0.5)
    assert torch.equal(wl(x), lin(x))  # (on the CPU the layer's own product)


def test_block_buffers_too_small_are_refused_before_any_launch():
    """The C ABI takes bare pointers: the Python layer checks that every byte a kernel reads lies in the tensor it
    passes (a short buffer would be read past its end on the GPU)."""
    import pytest

    E, R, C = 4, 64, 512
    whole = torch.zeros(E * R * SB.row_bytes("Q2_0", C), dtype=torch.uint8)
    short = whole[:-18]  # one Q2_0 block short
    x = torch.zeros((8, C), dtype=torch.bfloat16)
    idx = torch.zeros(8, dtype=torch.int32)
    with pytest.raises(ValueError, match="bytes for"):
        SB.switch_matvec(short, "Q2_0", (E, R, C), idx, x, 1)
    with pytest.raises(ValueError, match="bytes for"):
        SB.window_matvec(short[: R * SB.row_bytes("Q2_0", C) - 18], "Q2_0", R, C, x)
    with pytest.raises(ValueError, match="bytes for"):
        SB.tile_matmul(short, "Q2_0", (E, R, C), torch.zeros((16, C), dtype=torch.bfloat16),
                       torch.zeros(1, dtype=torch.int32))
    with pytest.raises(ValueError, match="bytes for"):
        SB.stack_matvec(short, "Q2_0", (E, R, C), torch.zeros((E, 1, C), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="bytes for"):
        SB.BlockSwitchLinear(short, "Q2_0", (E, R, C))
