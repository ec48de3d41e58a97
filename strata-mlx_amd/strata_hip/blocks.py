"""Experts computed on the GGUF file's own blocks — strata_mlx/blocks.py's interface over HIP kernels for MI355X.

Same names, argument order and return conventions as the reference module (strata_mlx/blocks.py), on torch
tensors that live on the GPU: blocks are uint8 tensors holding a tensor's bytes as the file has them, activations
are float32, float16 or bfloat16. Functions the reference answers with None ("not taken here, fall back") keep
that contract.

What runs where (csrc/):
    dequantize, generic products      blocks.hip   every type, exact float32 weights, float32 sums
    switch / separate / window / glu  expert.hip   MFMA decode path for bf16/fp16 activations of the fast kinds
    table of sums (Q2_0)              blocks.hip   the reference's lookup_* functions, for parity of interface
    tiles_of, tile_matmul             route.hip, tiles.hip
"""

import numpy as np
import torch

from . import _lib
from . import tables as _tables

# type -> (weights per block, bytes per block): strata_mlx/blocks.py:36-38
BLOCK = {"IQ4_NL": (32, 18), "IQ4_XS": (256, 136), "IQ3_S": (256, 110), "IQ3_XXS": (256, 98),
         "IQ2_S": (256, 82), "IQ2_XS": (256, 74), "IQ2_XXS": (256, 66), "IQ1_M": (256, 56), "Q2_0": (64, 18),
         "Q3_K": (256, 110)}
KIND = {"Q2_0": 0, "IQ4_NL": 1, "IQ4_XS": 2, "IQ3_S": 3, "IQ3_XXS": 4, "IQ2_S": 5, "IQ2_XS": 6, "IQ2_XXS": 7,
        "IQ1_M": 8, "Q3_K": 9}

MAX_SEPARATE = 29  # strata_mlx/blocks.py:328 — kept as the interface's limit of buffers a call
TILES_FROM = 1600  # (token, expert) pairs from which a prompt goes through the tiles (blocks.py:460)
TOKENS_TILE, ROWS_TILE, COLS_TILE = 16, 64, 64  # blocks.py:462 (what `tileable` accepts)
# The reference's Q2_0 table of sums is its answer to an arithmetic-bound Apple kernel; on MI355X the MFMA decode
# path is faster, so switch_glu does not route through it (the lookup_* functions remain, same interface).
LOOKUP_FROM = 1 << 62
GLU_IN_DOWN = True
BLOCK_GLU = True
MATVEC_GLU_UPTO = 30  # pairs (blocks.py:779)


def _kind(kind: str) -> int:
    try:
        return KIND[kind]
    except KeyError:
        raise ValueError(f"{kind}: not a block type ({', '.join(sorted(KIND))})") from None


def _check_cols(kind: str, cols: int):
    per_block = BLOCK[kind][0]
    if cols % per_block:
        raise ValueError(f"{kind}: rows of {cols} weights do not end on a block of {per_block}")


def row_bytes(kind: str, cols: int) -> int:
    _check_cols(kind, cols)
    return cols // BLOCK[kind][0] * BLOCK[kind][1]


def _tabs(kind: str, device) -> int | None:
    if not _tables.NEEDS[kind]:
        return None
    return _tables.device_blob(device).data_ptr()


def _on_gpu(*ts):
    dev = ts[0].device
    for t in ts:
        if t.device != dev:
            raise ValueError(f"tensors on {t.device} and {dev}")
    _lib.stream_of(ts[0])
    return dev


def _check_stack(blocks: torch.Tensor, kind: str, n: int, rows: int, cols: int, what: str) -> None:
    """The bytes a kernel reads for n (rows, cols) matrices of `kind` are all in `blocks` (the C ABI cannot know)."""
    if blocks.numel() < n * rows * row_bytes(kind, cols):
        raise ValueError(f"{what}: {blocks.numel()} bytes for {n} x ({rows}, {cols}) {kind} weights")


def _u8(blocks: torch.Tensor) -> torch.Tensor:
    if blocks.dtype != torch.uint8 or not blocks.is_contiguous():
        raise ValueError("blocks: a contiguous uint8 tensor of the file's bytes expected")
    return blocks


def _idx32(indices: torch.Tensor) -> torch.Tensor:
    return indices.reshape(-1).to(torch.int32).contiguous()


def dequantize(blocks: torch.Tensor, kind: str, shape: tuple, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """The weights of `blocks` (uint8, a tensor of `shape` as the file holds it) as floats
    (strata_mlx/blocks.py:397-404)."""
    *lead, rows, cols = shape
    n = int(np.prod(lead)) if lead else 1
    _check_cols(kind, cols)
    blocks = _u8(blocks)
    if blocks.numel() < n * rows * row_bytes(kind, cols):
        raise ValueError(f"blocks: {blocks.numel()} bytes for a {kind} tensor of {tuple(shape)}")
    _on_gpu(blocks)
    out = torch.empty(tuple(shape), dtype=dtype, device=blocks.device)
    _lib.call("sh_dequantize", _kind(kind), blocks.data_ptr(), _tabs(kind, blocks.device), n, rows, cols,
              out.data_ptr(), _lib.dtype_code(dtype), _lib.stream_of(blocks))
    return out


def switch_matvec(blocks: torch.Tensor, kind: str, shape: tuple, idx: torch.Tensor, x: torch.Tensor,
                  share: int) -> torch.Tensor:
    """out[pair] = W[idx[pair]] . x[pair // share] for a stack of `shape` (experts, rows, cols); (pairs, rows)
    in x's type. The kernel behind BlockSwitchLinear (strata_mlx/blocks.py:196-220, 420-436)."""
    experts, rows, cols = shape
    _check_cols(kind, cols)
    _check_stack(blocks, kind, experts, rows, cols, "switch_matvec")
    idx = _idx32(idx)
    pairs = idx.numel()
    x = x.reshape(-1, cols).contiguous()
    if x.shape[0] * share < pairs:
        raise ValueError(f"{pairs} pairs at {share} a row need {-(-pairs // share)} rows of x, not {x.shape[0]}")
    _on_gpu(blocks, idx, x)
    out = torch.empty((pairs, rows), dtype=x.dtype, device=x.device)
    if pairs == 0:
        return out
    k, dt = _kind(kind), _lib.dtype_code(x.dtype)
    ws_bytes = _lib.load().sh_switch_workspace(k, rows, cols, pairs, dt)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    _lib.call("sh_switch_matvec", k, _u8(blocks).data_ptr(), _tabs(kind, x.device), experts, rows, cols,
              idx.data_ptr(), pairs, x.data_ptr(), dt, share, out.data_ptr(), ws.data_ptr(), ws_bytes,
              _lib.stream_of(x))
    return out


def matvec_separate(experts: list, kind: str, rows: int, cols: int, x: torch.Tensor, share: int) -> torch.Tensor:
    """out[pair] = W[pair] . x, every pair bringing its expert's blocks as a tensor of its own. x (pairs / share,
    cols). Returns (pairs, rows) (strata_mlx/blocks.py:331-346)."""
    n = len(experts)
    _check_cols(kind, cols)
    x = x.reshape(-1, cols).contiguous()
    _on_gpu(x, *experts)
    for e in experts:
        if _u8(e).numel() < rows * row_bytes(kind, cols):
            raise ValueError(f"an expert of {e.numel()} bytes for {rows} rows of {cols} {kind} weights")
    out = torch.empty((n, rows), dtype=x.dtype, device=x.device)
    if n == 0:
        return out
    ptrs = torch.tensor([e.data_ptr() for e in experts], dtype=torch.int64).to(x.device)
    _lib.call("sh_matvec_separate", _kind(kind), ptrs.data_ptr(), _tabs(kind, x.device), rows, cols, n,
              x.data_ptr(), _lib.dtype_code(x.dtype), share, out.data_ptr(), _lib.stream_of(x))
    return out


def stack_takes(kind: str, cols: int, dtype: torch.dtype) -> bool:
    """Whether stack_matvec (the MFMA path) takes matrices of `kind` with rows of `cols` and `dtype` activations."""
    return kind in ("Q2_0", "IQ3_S") and cols % 256 == 0 and dtype in (torch.bfloat16, torch.float16)


def stack_matvec(blocks: torch.Tensor, kind: str, shape: tuple, x: torch.Tensor) -> torch.Tensor:
    """out[m, t] = W_m . x[m, t] for a stack of `shape` (matrices, rows, cols) and x (matrices, tokens, cols): the
    window matvec (strata_mlx/blocks.py:351-394) over many matrices in one launch, streaming their blocks. Returns
    (matrices, tokens, rows) in x's type. Q2_0 / IQ3_S with bf16 / fp16 activations (rows of whole 256s) take the
    MFMA kernels, up to 16 tokens; every other kind, and float32 activations, the exact-weight kernel (float32
    sums, the generic window kernel's bits), up to 8 tokens."""
    n, rows, cols = shape
    _check_cols(kind, cols)
    x = x.reshape(n, -1, cols).contiguous()
    tokens = x.shape[1]
    if blocks.numel() < n * rows * row_bytes(kind, cols):
        raise ValueError(f"blocks: {blocks.numel()} bytes for a {kind} stack of {tuple(shape)}")
    _on_gpu(blocks, x)
    out = torch.empty((n, tokens, rows), dtype=x.dtype, device=x.device)
    k, dt = _kind(kind), _lib.dtype_code(x.dtype)
    ws_bytes = _lib.load().sh_stack_workspace(k, n, rows, cols, tokens, dt)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    _lib.call("sh_stack_matvec", k, _u8(blocks).data_ptr(), _tabs(kind, x.device), n, rows, cols, x.data_ptr(), dt,
              tokens, out.data_ptr(), ws.data_ptr(), ws_bytes, _lib.stream_of(x))
    return out


def _stack_plans(blocks: torch.Tensor, kind: str, rows: int, cols: int, x: torch.Tensor) -> bool:
    """Whether the streaming stack kernel has a plan for this one layer (its waves' column splits and LDS ring hold
    the row); wider rows take the generic window kernel."""
    _on_gpu(blocks, x)
    return bool(_lib.load().sh_stack_takes(_kind(kind), _u8(blocks).data_ptr(), _tabs(kind, x.device), 1, rows, cols,
                                           x.data_ptr(), _lib.dtype_code(x.dtype), x.shape[0]))


def window_matvec(blocks: torch.Tensor, kind: str, rows: int, cols: int, x: torch.Tensor,
                  per_row: int | None = None) -> torch.Tensor:
    """out[t] = W . x[t] for one layer `blocks` of (rows, cols) and x (tokens, cols). Returns (tokens, rows)
    (strata_mlx/blocks.py:384-394). `per_row` is accepted for the interface; the library chooses its lanes. A token's
    bits do not depend on the window it is in, on either path."""
    _check_cols(kind, cols)
    _check_stack(blocks, kind, 1, rows, cols, "window_matvec")
    x = x.reshape(-1, cols).contiguous()
    tokens = x.shape[0]
    if stack_takes(kind, cols, x.dtype) and 0 < tokens <= 16 and _stack_plans(blocks, kind, rows, cols, x):
        return stack_matvec(blocks, kind, (1, rows, cols), x[None])[0]
    _on_gpu(blocks, x)
    out = torch.empty((tokens, rows), dtype=x.dtype, device=x.device)
    for a in range(0, tokens, 8):
        b = min(tokens, a + 8)
        _lib.call("sh_window_matvec", _kind(kind), _u8(blocks).data_ptr(), _tabs(kind, x.device), rows, cols,
                  x[a:b].data_ptr(), _lib.dtype_code(x.dtype), b - a, out[a:b].data_ptr(), _lib.stream_of(x))
    return out


class BlockSwitchLinear:
    """A stack of linear layers kept as the file's blocks; called like mlx-lm's `QuantizedSwitchLinear`
    (strata_mlx/blocks.py:407-440)."""

    unpack_from = 5000

    def __init__(self, blocks: torch.Tensor, kind: str, shape: tuple, per_row: int | None = None):
        _kind(kind)
        self.blocks, self.kind = _u8(blocks), kind
        self.num_experts, self.output_dims, self.input_dims = shape
        if blocks.numel() < self.num_experts * self.output_dims * row_bytes(kind, self.input_dims):
            raise ValueError(f"blocks: {blocks.numel()} bytes for a {kind} stack of {tuple(shape)}")
        self.per_row = per_row

    @property
    def shape(self):
        return (self.num_experts, self.output_dims, self.input_dims)

    def __call__(self, x: torch.Tensor, indices: torch.Tensor, sorted_indices: bool = False) -> torch.Tensor:
        """x (..., 1, in): one row to each index or to each run of the last axis of `indices`."""
        batch, k = tuple(x.shape[:-2]), (indices.shape[-1] if indices.dim() else 1)
        ishape = tuple(indices.shape)
        if batch == ishape:
            share = 1
        elif batch == (*ishape[:-1], 1):
            share = k
        else:
            x, share = torch.broadcast_to(x, (*ishape, 1, self.input_dims)), 1
        pairs = indices.numel()
        if pairs >= self.unpack_from:
            return self._as_floats(x, indices)
        out = switch_matvec(self.blocks, self.kind, self.shape, indices, x, share)
        return out.reshape(*ishape, 1, self.output_dims)

    def _as_floats(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        """Many pairs of a shape the tiles of switch_glu did not take. The reference unpacks the stack to x's type
        and multiplies with gather_mm (strata_mlx/blocks.py:438-440): the same roundings here, the pairs laid out
        in tiles of one expert and multiplied by the grouped GEMM (weights rounded to x's type, float32 sums, the
        result in x's type). Shapes the tiles do not take go through the expert matvec."""
        ishape = tuple(indices.shape)
        xs = torch.broadcast_to(x, (*ishape, 1, self.input_dims)).reshape(-1, self.input_dims)
        flat = indices.reshape(-1)
        if tileable(self.kind, self.output_dims, self.input_dims):
            te, token, where = tiles_of(flat[:, None], self.num_experts)
            out = tile_matmul(self.blocks, self.kind, self.shape, xs[token.long()], te)[where.long()].to(x.dtype)
        else:
            out = torch.cat([switch_matvec(self.blocks, self.kind, self.shape, flat[a:a + 65535], xs[a:a + 65535], 1)
                             for a in range(0, flat.numel(), 65535)])
        return out.reshape(*ishape, 1, self.output_dims)


def _glu_shapes(lin, idx, gate, up):
    idx = _idx32(idx)
    pairs = idx.numel()
    if gate.shape != up.shape or gate.reshape(-1, lin.input_dims).shape[0] != pairs:
        raise ValueError(f"gate {tuple(gate.shape)} / up {tuple(up.shape)} for {pairs} pairs of {lin.input_dims}")
    return idx, pairs, gate.reshape(pairs, -1).contiguous(), up.reshape(pairs, -1).contiguous()


def matvec_glu(lin, idx: torch.Tensor, gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor | None:
    """`lin(swiglu(gate, up), idx)` for a BlockSwitchLinear, one pair to each row of gate and up, (pairs, out); None
    where the inner activations do not fit a block's LDS (strata_mlx/blocks.py:782-798)."""
    if lin.input_dims * gate.element_size() > 65536:
        return None
    idx, pairs, gate, up = _glu_shapes(lin, idx, gate, up)
    _on_gpu(lin.blocks, idx, gate, up)
    out = torch.empty((pairs, lin.output_dims), dtype=gate.dtype, device=gate.device)
    if pairs:
        _lib.call("sh_matvec_glu", _kind(lin.kind), lin.blocks.data_ptr(), _tabs(lin.kind, gate.device),
                  lin.num_experts, lin.output_dims, lin.input_dims, idx.data_ptr(), pairs, gate.data_ptr(),
                  up.data_ptr(), _lib.dtype_code(gate.dtype), out.data_ptr(), _lib.stream_of(gate))
    return out


# ---- Q2_0 table of sums (strata_mlx/blocks.py:579-771)

def lookable(lin, dtype: torch.dtype) -> bool:
    return lin.kind == "Q2_0" and dtype == torch.float16


def lookup_table(x: torch.Tensor) -> torch.Tensor:
    """x (n, cols) -> (n, cols / 2, 16): for every two inputs, the sums two Q2_0 weights can make of them."""
    n, cols = x.shape
    x = x.contiguous()
    _on_gpu(x)
    table = torch.empty((n, cols // 2, 16), dtype=x.dtype, device=x.device)
    _lib.call("sh_lookup_table", x.data_ptr(), _lib.dtype_code(x.dtype), n, cols, table.data_ptr(), _lib.stream_of(x))
    return table


def lookup_table_glu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """The table of silu(gate) * up, both (n, cols)."""
    n, cols = gate.shape
    gate, up = gate.contiguous(), up.contiguous()
    _on_gpu(gate, up)
    table = torch.empty((n, cols // 2, 16), dtype=gate.dtype, device=gate.device)
    _lib.call("sh_lookup_table_glu", gate.data_ptr(), up.data_ptr(), _lib.dtype_code(gate.dtype), n, cols,
              table.data_ptr(), _lib.stream_of(gate))
    return table


def lookup_matvec(lin, idx: torch.Tensor, table: torch.Tensor, share: int) -> torch.Tensor:
    """out[pair] = W[idx[pair]] . x[pair / share], x given as its `lookup_table`. Returns (pairs, rows)."""
    if lin.kind != "Q2_0":
        raise ValueError(f"lookup_matvec: {lin.kind} experts (Q2_0 only)")
    idx = _idx32(idx)
    pairs = idx.numel()
    table = table.contiguous()
    _on_gpu(lin.blocks, idx, table)
    out = torch.empty((pairs, lin.output_dims), dtype=table.dtype, device=table.device)
    if pairs:
        _lib.call("sh_lookup_matvec", lin.blocks.data_ptr(), lin.num_experts, lin.output_dims, lin.input_dims,
                  idx.data_ptr(), pairs, table.data_ptr(), _lib.dtype_code(table.dtype), share, out.data_ptr(),
                  _lib.stream_of(table))
    return out


def lookup_down_glu(lin, idx: torch.Tensor, gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor | None:
    """`lookup_matvec(lin, idx, lookup_table_glu(gate, up), 1)` in one kernel, or None where the table would not fit
    a block's LDS."""
    if lin.kind != "Q2_0" or lin.input_dims // 2 * 16 * gate.element_size() > 65536:
        return None
    idx, pairs, gate, up = _glu_shapes(lin, idx, gate, up)
    _on_gpu(lin.blocks, idx, gate, up)
    out = torch.empty((pairs, lin.output_dims), dtype=gate.dtype, device=gate.device)
    if pairs:
        _lib.call("sh_lookup_down_glu", lin.blocks.data_ptr(), lin.num_experts, lin.output_dims, lin.input_dims,
                  idx.data_ptr(), pairs, gate.data_ptr(), up.data_ptr(), _lib.dtype_code(gate.dtype),
                  out.data_ptr(), _lib.stream_of(gate))
    return out


def _lookup_glu(x, indices, up, gate, down):
    k = indices.shape[-1]
    idx = indices.reshape(-1)
    table = lookup_table(x.reshape(-1, x.shape[-1]))
    g, u = lookup_matvec(gate, idx, table, k), lookup_matvec(up, idx, table, k)
    out = lookup_down_glu(down, idx, g, u) if GLU_IN_DOWN else None
    if out is None:
        out = lookup_matvec(down, idx, lookup_table_glu(g, u), 1)
    return out.reshape(*indices.shape, down.output_dims)


# ---- prompts: pairs in tiles of one expert, under MFMA (tiles.hip)

def tileable(kind: str, rows: int, cols: int) -> bool:
    """Whether `tile_matmul` takes a stack of such layers: the reference's rule (strata_mlx/blocks.py:511-513:
    rows % 64, cols % 64, whole blocks). The kernels take columns in chunks of 256, the last one partial where the
    row ends earlier. Q2_0 and IQ3_S stream their rows through LDS chunk by chunk; the other kinds keep a row group
    of 64 rows in LDS beside the chunk buffers and their codebooks, so their rows must fit there too: IQ4_NL up to
    2,240 weights, IQ4_XS up to 2,304 (at 2,560 the reference tiles them and this answers False: those prompts take
    the expert matvec, with exact weights instead of weights rounded to the activations' type)."""
    if rows % ROWS_TILE or cols % COLS_TILE or cols % BLOCK[kind][0]:
        return False
    if kind in STREAMED:
        return True
    rb = row_bytes(kind, cols)
    room = 160 * 1024 - 2 * 64 * 256 * 2 - (0 if kind == "Q3_K" else 16512)
    return 64 * rb <= room


STREAMED = ("Q2_0", "IQ3_S")  # kinds with the fused gate / up / SwiGLU and down products of the prompt path


def tiles_of(indices: torch.Tensor, experts: int) -> tuple:
    """The pairs of `indices` (..., k) in tiles of TOKENS_TILE, each tile one expert's
    (strata_mlx/blocks.py:539-563): (expert of each tile or `experts`, token of each slot, slot of each pair),
    int32, computed on the GPU in a number of tiles that depends only on the number of pairs."""
    k = indices.shape[-1] if indices.dim() else 1
    flat = _idx32(indices)
    pairs = flat.numel()
    _on_gpu(flat)
    lib = _lib.load()
    most = lib.sh_tiles_most(pairs, experts)
    tile_expert = torch.empty(most, dtype=torch.int32, device=flat.device)
    token = torch.empty(most * TOKENS_TILE, dtype=torch.int32, device=flat.device)
    where = torch.empty(pairs, dtype=torch.int32, device=flat.device)
    ws_bytes = lib.sh_tiles_workspace(experts)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=flat.device)
    _lib.call("sh_tiles_of", flat.data_ptr(), pairs, k, experts, tile_expert.data_ptr(), token.data_ptr(),
              where.data_ptr(), ws.data_ptr(), ws_bytes, _lib.stream_of(flat))
    return tile_expert, token, where


def tile_matmul(blocks: torch.Tensor, kind: str, shape: tuple, a: torch.Tensor, tile_expert: torch.Tensor) -> torch.Tensor:
    """out[p] = W[expert of p's tile] . a[p] for a stack of `shape` (experts, rows, cols); a (P, cols) float16,
    bfloat16 or float32, P a multiple of TOKENS_TILE; the weights rounded to a's type, float32 sums. Rows of a
    tile naming no expert are left as they were (strata_mlx/blocks.py:516-536). Returns (P, rows) float32.
    float32 activations take the weights exactly: each slot is then the expert matvec of its tile's expert
    (switch_matvec's kernels), tiles naming no expert computed against expert 0 (their rows are unspecified)."""
    if a.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError(f"tile_matmul: activations of {a.dtype} (float16, bfloat16 or float32)")
    experts, rows, cols = shape
    if not tileable(kind, rows, cols):
        raise ValueError(f"tile_matmul: {kind} ({rows}, {cols}) is not tileable")
    _check_stack(blocks, kind, experts, rows, cols, "tile_matmul")
    a = a.contiguous()
    p = a.shape[0]
    if p % TOKENS_TILE or a.shape[1] != cols:
        raise ValueError(f"tile_matmul: a {tuple(a.shape)} for rows of {cols}, in tiles of {TOKENS_TILE}")
    te = tile_expert.to(torch.int32).contiguous()
    if te.numel() * TOKENS_TILE != p:
        raise ValueError(f"tile_matmul: {te.numel()} tiles for {p} rows")
    if a.dtype == torch.float32:
        slot_expert = te.repeat_interleave(TOKENS_TILE)
        slot_expert = torch.where((slot_expert >= 0) & (slot_expert < experts), slot_expert,
                                  torch.zeros_like(slot_expert))
        return switch_matvec(blocks, kind, shape, slot_expert, a, 1)
    _on_gpu(blocks, a, te)
    out = torch.empty((p, rows), dtype=torch.float32, device=a.device)
    _lib.call("sh_tile_matmul", _kind(kind), _u8(blocks).data_ptr(), _tabs(kind, a.device), experts, rows, cols,
              a.data_ptr(), _lib.dtype_code(a.dtype), p, te.data_ptr(), out.data_ptr(), _lib.stream_of(a))
    return out


def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """mlx-lm's swiglu as the reference rounds it (sigmoid rounded to the type, then two products in it)."""
    if gate.dtype == torch.float32:
        return torch.nn.functional.silu(gate) * up
    sig = torch.sigmoid(gate.float()).to(gate.dtype)
    return (gate * sig) * up


def tile_glu(gate, up, x: torch.Tensor, token: torch.Tensor, tile_expert: torch.Tensor) -> torch.Tensor:
    """silu(gate . x[token[s]]) * (up . x[token[s]]) for every slot s of the tiles, the weights rounded to x's type,
    float32 sums, the result rounded to x's type: `_tiled_glu`'s first two products and its swiglu
    (strata_mlx/blocks.py:570-574) in one pass over gate's and up's rows. x (tokens, cols) float16 / bfloat16;
    token (16 * tiles,) int32 from tiles_of. Rows of tiles naming no expert are left as they were."""
    experts, rows, cols = gate.num_experts, gate.output_dims, gate.input_dims
    if gate.kind != up.kind or (up.num_experts, up.output_dims, up.input_dims) != (experts, rows, cols):
        raise ValueError("tile_glu: gate and up of one shape and kind expected")
    x = x.contiguous()
    tok = token.to(torch.int32).contiguous()
    te = tile_expert.to(torch.int32).contiguous()
    slots = tok.numel()
    if slots != TOKENS_TILE * te.numel() or x.dim() != 2 or x.shape[1] != cols:
        raise ValueError(f"tile_glu: {te.numel()} tiles, {slots} slots, x {tuple(x.shape)} for rows of {cols}")
    _on_gpu(gate.blocks, up.blocks, x, tok, te)
    h = torch.empty((slots, rows), dtype=x.dtype, device=x.device)
    _lib.call("sh_tile_glu", _kind(gate.kind), _u8(gate.blocks).data_ptr(), _u8(up.blocks).data_ptr(),
              _tabs(gate.kind, x.device), experts, rows, cols, x.data_ptr(), _lib.dtype_code(x.dtype), x.shape[0],
              tok.data_ptr(), slots, te.data_ptr(), h.data_ptr(), _lib.stream_of(x))
    return h


def tile_down(down, h: torch.Tensor, tile_expert: torch.Tensor, where: torch.Tensor) -> torch.Tensor:
    """down . h[where[p]] for every pair p, the weights rounded to h's type, float32 sums, the result rounded to
    h's type: `_tiled_glu`'s last product, its un-permutation and its cast (strata_mlx/blocks.py:575) in one pass.
    h (16 * tiles, cols) from tile_glu; where (pairs,) from tiles_of. Returns (pairs, rows)."""
    experts, rows, cols = down.num_experts, down.output_dims, down.input_dims
    h = h.contiguous()
    te = tile_expert.to(torch.int32).contiguous()
    slots, pairs = h.shape[0], where.numel()
    if slots != TOKENS_TILE * te.numel() or h.shape[1] != cols:
        raise ValueError(f"tile_down: h {tuple(h.shape)} for {te.numel()} tiles of rows of {cols}")
    _on_gpu(down.blocks, h, te, where)
    pair = torch.full((slots,), -1, dtype=torch.int32, device=h.device)  # the pair of each slot, -1 for none
    pair[where.long()] = torch.arange(pairs, dtype=torch.int32, device=h.device)
    out = torch.empty((pairs, rows), dtype=h.dtype, device=h.device)
    _lib.call("sh_tile_down", _kind(down.kind), _u8(down.blocks).data_ptr(), _tabs(down.kind, h.device), experts,
              rows, cols, h.data_ptr(), _lib.dtype_code(h.dtype), slots, te.data_ptr(), pair.data_ptr(), pairs,
              out.data_ptr(), _lib.stream_of(h))
    return out


def _tiled_glu(x, indices, up, gate, down):
    """The three products of a prompt's pairs through the tiles (strata_mlx/blocks.py:566-576):
    h = swiglu(gate . a, up . a) rounded to x's type, out = (down . h)[where] rounded to x's type. Q2_0 and IQ3_S
    in two fused passes (tile_glu, tile_down); other kinds through tile_matmul as the reference composes it."""
    tiles, token, where = tiles_of(indices, gate.num_experts)
    x2 = x.reshape(-1, x.shape[-1])
    if (gate.kind == up.kind == down.kind and gate.kind in STREAMED and x.dtype in (torch.float16, torch.bfloat16)
            and gate.output_dims % 32 == 0):
        out = tile_down(down, tile_glu(gate, up, x2, token, tiles), tiles, where)
        return out.reshape(*indices.shape, down.output_dims)
    a = x2[token.long()]

    def product(lin, a):
        return tile_matmul(lin.blocks, lin.kind, lin.shape, a, tiles)

    h = swiglu(product(gate, a), product(up, a)).to(x.dtype)
    out = product(down, h)[where.long()].to(x.dtype)
    return out.reshape(*indices.shape, down.output_dims)


def switch_glu(x: torch.Tensor, indices: torch.Tensor, up, gate, down) -> torch.Tensor:
    """down(silu(gate(x)) * up(x)) through each token's experts: x (..., in), indices (..., experts per token)
    (strata_mlx/blocks.py:801-829). The branches: a prompt's many pairs through the tiles; otherwise gate and up
    by the expert matvec (one row of x to each token's k pairs) and down taking silu(gate) * up itself."""
    if (indices.numel() >= TILES_FROM and x.dtype in (torch.float16, torch.bfloat16, torch.float32)
            and all(tileable(lin.kind, lin.output_dims, lin.input_dims) for lin in (up, gate, down))):
        return _tiled_glu(x, indices, up, gate, down)
    if indices.numel() >= LOOKUP_FROM and all(lookable(lin, x.dtype) for lin in (up, gate, down)):
        return _lookup_glu(x, indices, up, gate, down)
    x5 = x.unsqueeze(-2).unsqueeze(-3)
    g, u = gate(x5, indices), up(x5, indices)
    flat = indices.reshape(-1)
    out = None
    if BLOCK_GLU and flat.numel() <= MATVEC_GLU_UPTO:
        out = matvec_glu(down, flat, g.reshape(flat.numel(), -1), u.reshape(flat.numel(), -1))
    if out is not None:
        return out.reshape(*indices.shape, down.output_dims)
    return down(swiglu(g, u), indices).squeeze(-2)


class BlockSwitchGLU:
    """A layer's routed experts, called like mlx-lm's `SwitchGLU` (strata_mlx/blocks.py:832-839)."""

    def __init__(self, gate: BlockSwitchLinear, up: BlockSwitchLinear, down: BlockSwitchLinear):
        self.gate_proj, self.up_proj, self.down_proj = gate, up, down

    def __call__(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        return switch_glu(x, indices, self.up_proj, self.gate_proj, self.down_proj)
