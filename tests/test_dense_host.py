"""The dense layers' host-side rules (strata_hip.dense, strata_mlx/dense.py) on the CPU, as the reference's own tests
state them: which tensors stay blocks, which shapes the scaled kernel takes, and the float weights a prompt makes —
kept for the prompt's next pieces and let go by release(), or made for each piece when a layer does not keep them.
Nothing here launches a kernel: the float weights are made by a stand-in."""

import numpy as np
import pytest
import torch

from strata_hip import dense as SD
from strata_hip import gguf as G


def scaled(rows=8, cols=256):
    rng = np.random.default_rng(rows + cols)
    codes = torch.from_numpy(rng.integers(-32, 32, (rows, cols)).astype(np.int8))
    scales = torch.from_numpy(rng.integers(-128, 128, (rows, cols // 16)).astype(np.int8))
    d = torch.from_numpy((rng.random((rows, cols // 256)) * 0.01).astype(np.float16))
    return SD.ScaledLinear(codes, scales, d)


def with_made_floats(lin, made):
    """The layer's float weights worked out on the CPU (code * scale * d, as the kernel does), counting each time."""
    def floats(dtype):
        made.append(dtype)
        s = lin.scales.float().repeat_interleave(16, dim=1) * lin.d.float().repeat_interleave(lin.d_step, dim=1)
        return (lin.codes.float() * s).to(dtype)
    lin.floats = floats
    return lin


def test_floats_made_for_a_prompt_are_kept_until_release():
    SD.release()
    made = []
    lin = with_made_floats(scaled(), made)
    x = torch.randn(SD.MAX_TOKENS + 2, 256)
    first = lin(x)
    held = lin._floats
    assert held is not None and lin in SD._holding and len(made) == 1
    assert torch.equal(lin(x), first) and lin._floats is held and len(made) == 1  # the next piece: not made again
    SD.release()
    assert lin._floats is None and not SD._holding
    assert torch.equal(lin(x), first) and len(made) == 2
    SD.release()


def test_floats_not_kept_are_made_for_each_piece_and_let_go():
    SD.release()
    made_k, made_n = [], []
    kept, fresh = with_made_floats(scaled(), made_k), with_made_floats(scaled(), made_n)
    fresh.keep = False
    x = torch.randn(SD.MAX_TOKENS + 2, 256)
    assert torch.equal(fresh(x), kept(x))
    assert torch.equal(fresh(x), kept(x))
    assert fresh._floats is None and fresh not in SD._holding and len(made_n) == 2 and len(made_k) == 1
    SD.release()


def test_which_shapes_the_scaled_kernel_takes():
    assert SD.fits(8, 256) and SD.fits(4, 512) and not SD.fits(6, 256) and not SD.fits(8, 320)
    with pytest.raises(ValueError):
        scaled(rows=6)


def tensor(name, shape, kind):
    per_block, block_bytes = {v[0]: (v[1], v[2]) for v in G.TYPES.values()}[kind]
    n = int(np.prod(shape)) // per_block * block_bytes
    return G.Tensor(name, shape, kind, np.zeros(n, dtype=np.uint8))


def test_a_file_tensor_becomes_the_layer_the_reference_makes():
    dev = torch.device("cpu")
    assert isinstance(G.dense(tensor("q3k", (8, 512), "Q3_K"), dev), SD.BlockLinear)
    assert isinstance(G.dense(tensor("q6k", (8, 512), "Q6_K"), dev), SD.ScaledLinear)
    odd = G.dense(tensor("odd", (6, 512), "Q6_K"), dev)  # six rows: not groups of four
    assert isinstance(odd, SD.FloatLinear) and tuple(odd.weight.shape) == (6, 512)
    assert isinstance(G.dense(tensor("f16", (8, 64), "F16"), dev), SD.FloatLinear)


def test_what_stays_blocks():
    assert SD.as_blocks((4, 512), "Q3_K") and SD.as_blocks((4, 512), "IQ4_XS")
    assert not SD.as_blocks((2, 4, 512), "Q3_K")  # not a layer
    assert not SD.as_blocks((4, 320), "Q3_K")  # rows that do not end on a block
    assert not SD.as_blocks((4, 512), "Q4_K")  # a type not asked for as blocks
    assert not SD.as_blocks((4, 512), "Q3_K", kinds=("IQ4_XS",))
