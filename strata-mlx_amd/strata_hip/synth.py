"""Seeded synthetic inputs of the path's workloads: GGUF blocks with valid scales, activations, router logits,
paged KV caches. Random bytes for codes and indices; every fp16 scale written as a finite value (as the
reference's own tests do, tests/test_gguf.py:17-30, tests/test_blocks.py:75-95)."""

import numpy as np
import torch

from .blocks import BLOCK

# where each block keeps its fp16 scales (IQ1_M spreads its scale over four words: _put_iq1m_scale)
SCALE_BYTES = {"Q2_0": [0], "IQ4_NL": [0], "IQ4_XS": [0], "Q3_K": [108], "IQ3_S": [0], "IQ3_XXS": [0],
               "IQ2_S": [0], "IQ2_XS": [0], "IQ2_XXS": [0], "IQ1_M": []}


def _scales(rng, n: int, dist: str, sigma: float) -> np.ndarray:
    if dist == "halfnormal":
        return np.abs(rng.normal(0.0, sigma, n)).astype("<f2")
    if dist == "uniform":
        return rng.uniform(-2.5 * sigma, 2.5 * sigma, n).astype("<f2")
    raise ValueError(dist)


def random_blocks(kind: str, rows: int, cols: int, rng: np.random.Generator, dist: str = "halfnormal",
                  sigma: float = 0.02) -> np.ndarray:
    """uint8 bytes of a (rows, cols) `kind` tensor (rows may cover a whole stack of experts)."""
    per_block, block_bytes = BLOCK[kind]
    if cols % per_block:
        raise ValueError(f"{kind}: rows of {cols} weights do not end on a block of {per_block}")
    n = rows * cols // per_block
    b = rng.integers(0, 256, (n, block_bytes), dtype=np.uint8)
    for at in SCALE_BYTES[kind]:
        b[:, at:at + 2] = _scales(rng, n, dist, sigma).view(np.uint8).reshape(n, 2)
    if kind == "IQ1_M":
        d = _scales(rng, n, dist, sigma).view("<u2")
        words = b[:, 48:56].copy().view("<u2")
        for i in range(4):
            words[:, i] = (words[:, i] & 0x0FFF) | (((d >> (4 * i)) & 15) << 12)
        b[:, 48:56] = words.view(np.uint8)
    return b.reshape(-1)


def random_blocks_gpu(kind: str, rows: int, cols: int, seed: int, device, sigma: float = 0.02) -> torch.Tensor:
    """The same kind of tensor generated on the GPU (for stacks of many GB): random bytes, then the scale
    bytes of every block overwritten with fp16 |N(0, sigma)|."""
    per_block, block_bytes = BLOCK[kind]
    n = rows * cols // per_block
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    b = torch.randint(0, 256, (n, block_bytes), dtype=torch.uint8, device=device, generator=g)
    d = (torch.randn(n, device=device, generator=g) * sigma).abs().to(torch.float16)
    if kind == "IQ1_M":
        du = d.view(torch.int16).to(torch.int32) & 0xFFFF
        words = b[:, 48:56].contiguous().view(torch.int16).to(torch.int32) & 0xFFFF
        for i in range(4):
            words[:, i] = (words[:, i] & 0x0FFF) | (((du >> (4 * i)) & 15) << 12)
        b[:, 48:56] = words.to(torch.int16).view(torch.uint8).reshape(n, 8)
    else:
        for at in SCALE_BYTES[kind]:
            b[:, at:at + 2] = d.view(torch.uint8).reshape(n, 2)
    return b.reshape(-1)


def bf16_normal(rng: np.random.Generator, shape, scale: float = 1.0) -> torch.Tensor:
    """N(0, scale) values rounded to bfloat16 (CPU tensor)."""
    return torch.from_numpy(rng.standard_normal(shape).astype(np.float32) * scale).to(torch.bfloat16)


def zipf_logits(rng: np.random.Generator, tokens: int, experts: int, s: float = 1.1) -> torch.Tensor:
    """Router logits whose top-k sample experts with Zipf(s) popularity over a seeded permutation:
    log p_e + Gumbel noise (Gumbel-top-k samples without replacement in proportion to p)."""
    rank = rng.permutation(experts) + 1
    logp = -s * np.log(rank)
    gumbel = -np.log(-np.log(rng.uniform(1e-12, 1.0, (tokens, experts))))
    return torch.from_numpy((logp[None, :] + gumbel).astype(np.float32)).to(torch.bfloat16)
