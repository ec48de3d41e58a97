"""Dense layers kept as the file's blocks — strata_mlx/dense.py's interface over the HIP kernels.

  * BlockLinear (dense.py:197-228): a linear layer held as the file's blocks, called like `nn.Linear`. A window of
    up to MAX_TOKENS tokens multiplies on the blocks (window_matvec: the streaming MFMA matvec for Q2_0 / IQ3_S,
    exact float32 weights for the other kinds); a chunk of a prompt unpacks the weights to the activations' type
    (sh_dequantize) and multiplies them as a plain GEMM (torch.matmul, hipBLASLt), as the reference unpacks them
    and multiplies with MLX's matmul.
  * ScaledLinear (dense.py:109-167): a Q6_K layer held as int8 codes, int8 scales of 16 weights and float16 d of
    256, called like `nn.Linear`; `q6k_parts` splits the file's blocks into those three (gguf.py:150-164).
  * BlockEmbedding (dense.py:231-244): an embedding held as the file's blocks, a token's row unpacked when it comes.
"""

import numpy as np
import torch

from . import _lib
from .blocks import BLOCK, _kind, _on_gpu, _tabs, _u8, dequantize, row_bytes, window_matvec

MAX_TOKENS = 8  # dense.py:33: more than a window is a chunk of a prompt, multiplied as floats
AS_BLOCKS = ("Q3_K", "IQ4_XS")  # dense.py:189

_holding = []  # dense.py:85: the layers holding their weights as floats as well, since a prompt was read


def release():
    """Let go of the float weights made for chunks of prompts (dense.py:88-94); nothing calls this by itself."""
    for layer in _holding:
        layer._floats = None
    _holding.clear()


def as_blocks(shape: tuple, kind: str, kinds: tuple = AS_BLOCKS) -> bool:
    """Whether a dense tensor of `shape` and `kind` can stay blocks (dense.py:193-195)."""
    return kind in kinds and len(shape) == 2 and shape[1] % BLOCK[kind][0] == 0


class BlockLinear:
    """A linear layer held as the file's blocks; called like `nn.Linear` (strata_mlx/dense.py:197-228).

    `blocks` are the rows in the order of the layer's outputs. `inputs`, if given, is where in the file's row each
    input is: the blocks cannot be reordered inside, so the activations are, before they multiply."""

    def __init__(self, blocks: torch.Tensor, kind: str, shape: tuple, inputs=None):
        _kind(kind)
        self.blocks, self.kind = _u8(blocks), kind
        self.output_dims, self.input_dims = shape
        if blocks.numel() < self.output_dims * row_bytes(kind, self.input_dims):
            raise ValueError(f"blocks: {blocks.numel()} bytes for a {kind} layer of {tuple(shape)}")
        self.to_file = None
        if inputs is not None:
            order = np.argsort(np.asarray(inputs)).astype(np.int64)
            self.to_file = torch.from_numpy(order).to(blocks.device)

    @property
    def nbytes(self) -> int:
        return self.blocks.numel()

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        rows, cols = self.output_dims, self.input_dims
        lead = x.shape[:-1]
        tokens = int(np.prod(lead)) if len(lead) else 1
        x = x.reshape(tokens, cols)
        if self.to_file is not None:
            x = x.index_select(1, self.to_file)
        if tokens <= MAX_TOKENS:
            out = window_matvec(self.blocks, self.kind, rows, cols, x)
        else:
            out = x @ dequantize(self.blocks, self.kind, (rows, cols), x.dtype).T
        return out.reshape(*lead, rows)


class FloatLinear:
    """A float16 / bfloat16 weight (rows, cols) called like `nn.Linear`: x @ W^T in x's type (torch.matmul, a plain
    GEMM on hipBLASLt; sums in float32). What a float tensor of the file becomes (load.py:243-252)."""

    def __init__(self, weight: torch.Tensor):
        self.weight = weight
        self.output_dims, self.input_dims = weight.shape

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        return x @ self.weight.to(x.dtype).T


class BlockEmbedding:
    """An embedding held as the file's blocks; a token's row is unpacked when the token comes
    (strata_mlx/dense.py:231-244)."""

    def __init__(self, blocks: torch.Tensor, kind: str, shape: tuple, dtype: torch.dtype):
        self.num_embeddings, self.dims = shape
        self.kind, self.dtype = kind, dtype
        self.rows = _u8(blocks).reshape(self.num_embeddings, row_bytes(kind, self.dims))

    @property
    def nbytes(self) -> int:
        return self.rows.numel()

    def __call__(self, ids: torch.Tensor) -> torch.Tensor:
        taken = self.rows.index_select(0, ids.reshape(-1).long()).contiguous()
        return dequantize(taken.reshape(-1), self.kind, (ids.numel(), 1, self.dims), self.dtype).reshape(
            *ids.shape, self.dims)


def q6k_parts(blocks: np.ndarray, rows: int, cols: int):
    """A Q6_K tensor (rows, cols) of 210-byte blocks as its three parts (strata_mlx/gguf.py:150-164): a weight is
    code * scale * d. codes int8 (rows, cols), the six bits less 32; scales int8 (rows, cols / 16); d float16
    (rows, cols / 256). Each half of a block holds four runs of 32: low nibbles in ql (two runs a byte run),
    high bit pairs in qh."""
    b = np.asarray(blocks, np.uint8).reshape(-1, 210)
    ql, qh = b[:, :128].reshape(-1, 2, 64), b[:, 128:192].reshape(-1, 2, 32)
    hi = np.stack([(qh >> s) & 3 for s in (0, 2, 4, 6)], axis=2)
    lo = np.stack([ql[..., :32] & 15, ql[..., 32:] & 15, ql[..., :32] >> 4, ql[..., 32:] >> 4], axis=2)
    codes = ((lo | (hi << 4)).astype(np.int16) - 32).astype(np.int8)
    return (codes.reshape(rows, cols), np.ascontiguousarray(b[:, 192:208]).view(np.int8).reshape(rows, cols // 16),
            np.ascontiguousarray(b[:, 208:210]).view("<f2").reshape(rows, cols // 256))


def fits(rows: int, cols: int) -> bool:
    """Whether the scaled kernel takes a layer of this shape (dense.py:97-99): rows by 4, columns by 256."""
    return rows % 4 == 0 and cols % 256 == 0


class ScaledLinear:
    """A linear layer held as int8 codes, int8 scales of 16 weights and float16 d (strata_mlx/dense.py:109-167):
    w = code * scale * d, called like `nn.Linear`. Up to MAX_TOKENS tokens the product reads the three parts
    (sh_scaled_matvec, float32 sums); a chunk of a prompt multiplies the weights made as floats (sh_scaled_floats,
    each worked out in float32 and rounded once), kept for the next chunks unless `keep` is False."""

    def __init__(self, codes: torch.Tensor, scales: torch.Tensor, d: torch.Tensor):
        if codes.dtype != torch.int8 or scales.dtype != torch.int8 or d.dtype != torch.float16:
            raise ValueError("ScaledLinear: int8 codes, int8 scales, float16 d")
        self.codes, self.scales, self.d = codes.contiguous(), scales.contiguous(), d.contiguous()
        self.output_dims, self.input_dims = codes.shape
        if scales.shape != (self.output_dims, self.input_dims // 16) or d.shape[0] != self.output_dims:
            raise ValueError(f"ScaledLinear: scales {tuple(scales.shape)} / d {tuple(d.shape)} for {tuple(codes.shape)}")
        self.d_step = self.input_dims // d.shape[1]
        if self.d_step % 16 or self.input_dims % self.d_step:
            raise ValueError(f"ScaledLinear: a d to {self.d_step} weights")
        self._floats = None
        self.keep = True
        if not fits(*codes.shape):
            raise ValueError(f"a layer of {tuple(codes.shape)} does not fit the kernel")

    @classmethod
    def from_blocks(cls, blocks: np.ndarray, rows: int, cols: int, device) -> "ScaledLinear":
        codes, scales, d = q6k_parts(blocks, rows, cols)
        return cls(*(torch.from_numpy(np.ascontiguousarray(a)).to(device) for a in (codes, scales, d)))

    @property
    def nbytes(self) -> int:
        return self.codes.numel() + self.scales.numel() + 2 * self.d.numel()

    def floats(self, dtype: torch.dtype) -> torch.Tensor:
        """The weights (out, in), each worked out in float32 and rounded once to `dtype` (dense.py:120-135)."""
        _on_gpu(self.codes)
        out = torch.empty((self.output_dims, self.input_dims), dtype=dtype, device=self.codes.device)
        _lib.call("sh_scaled_floats", self.codes.data_ptr(), self.scales.data_ptr(), self.d.data_ptr(),
                  self.output_dims, self.input_dims, self.d_step, out.data_ptr(), _lib.dtype_code(dtype),
                  _lib.stream_of(self.codes))
        return out

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        rows, cols = self.output_dims, self.input_dims
        lead = x.shape[:-1]
        tokens = int(np.prod(lead)) if len(lead) else 1
        if tokens > MAX_TOKENS:
            if not self.keep:
                return x @ self.floats(x.dtype).T
            if self._floats is None or self._floats.dtype != x.dtype:
                self._floats = self.floats(x.dtype)
                if self not in _holding:
                    _holding.append(self)
            return x @ self._floats.T
        xs = x.reshape(tokens, cols).contiguous()
        _on_gpu(self.codes, xs)
        out = torch.empty((tokens, rows), dtype=x.dtype, device=x.device)
        _lib.call("sh_scaled_matvec", self.codes.data_ptr(), self.scales.data_ptr(), self.d.data_ptr(), rows, cols,
                  self.d_step, xs.data_ptr(), _lib.dtype_code(xs.dtype), tokens, out.data_ptr(), _lib.stream_of(xs))
        return out.reshape(*lead, rows)
