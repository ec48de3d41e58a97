"""Decode attention over a paged KV cache or over each query's cell list — strata_mlx/attention.py's `_gathered`
and `_cells` (attention.py:132-165) over the HIP kernels of csrc/attention.hip.

`_gathered(q, k, v, cells, real, scale, cache)` keeps the reference's arguments and result: q (1, heads, S, d),
k / v (1, kv heads, kv_len, d), cells / real (S, L) -> (1, S, heads * d). `paged_decode_attention` is the same
attention over a page table with pages of 16 positions, the causal mask among the window's queries built in.
"""

import math

import torch

from . import _lib

PAGE = 16  # positions a page


def _check_half(*ts):
    dt = ts[0].dtype
    if dt not in (torch.bfloat16, torch.float16):
        raise ValueError(f"attention in {dt}: bfloat16 or float16 expected")
    for t in ts[1:]:
        if t.dtype != dt:
            raise ValueError(f"q, k and v differ in dtype: {[t.dtype for t in ts]}")
    return dt


def paged_decode_attention(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor, page_table: torch.Tensor,
                           ctx_len: int, scale: float | None = None) -> torch.Tensor:
    """q (B, Hq, D) the window's B queries, the last B positions of a context of ctx_len; k_pages / v_pages
    (n_pages, Hkv, 16, D); page_table (>= ceil(ctx_len / 16),) int32 physical page of each 16 positions.
    Query t sees positions 0 .. ctx_len - B + t. Returns (B, Hq, D) in q's dtype; scale defaults to D ** -0.5."""
    dt = _check_half(q, k_pages, v_pages)
    B, Hq, D = q.shape
    n_pages, Hkv, P, D2 = k_pages.shape
    if P != PAGE or D2 != D or v_pages.shape != k_pages.shape:
        raise ValueError(f"pages {tuple(k_pages.shape)} / {tuple(v_pages.shape)} for q {tuple(q.shape)}")
    if page_table.dtype != torch.int32 or page_table.numel() < -(-ctx_len // PAGE):
        raise ValueError(f"page_table of {page_table.numel()} {page_table.dtype} for {ctx_len} positions")
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    q, k_pages, v_pages, page_table = (t.contiguous() for t in (q, k_pages, v_pages, page_table))
    out = torch.empty((B, Hq, D), dtype=dt, device=q.device)
    lib = _lib.load()
    need = lib.sh_paged_attn_workspace(B, Hq, Hkv, D, ctx_len)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    _lib.call("sh_paged_attn", q.data_ptr(), k_pages.data_ptr(), v_pages.data_ptr(), page_table.data_ptr(), n_pages,
              ctx_len, B, Hq, Hkv, D, scale, _lib.dtype_code(dt), out.data_ptr(), ws.data_ptr(), ws.numel(),
              _lib.stream_of(q))
    return out


def _gathered(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cells: torch.Tensor, real: torch.Tensor,
              scale: float, cache=None) -> torch.Tensor:
    """attention.py:144-165: q (1, heads, S, d) attending to its own cells of k, v (1, kv heads, kv_len, d)
    -> (1, S, heads * d). cells (S, L) integer cell ids, real (S, L) which of them count. `cache` is accepted for
    the reference's signature (its quantized-cache hook) and must be None here."""
    if cache is not None:
        raise ValueError("_gathered: a quantized KV cache is not taken")
    dt = _check_half(q, k, v)
    _, H, S, D = q.shape
    _, G, kv_len, D2 = k.shape
    L = cells.shape[1]
    if D2 != D or v.shape != k.shape or cells.shape != (S, L) or real.shape != (S, L):
        raise ValueError(f"_gathered: q {tuple(q.shape)}, k {tuple(k.shape)}, cells {tuple(cells.shape)}")
    qs = q[0].transpose(0, 1).contiguous()  # (S, H, D)
    kk, vv = k[0].contiguous(), v[0].contiguous()
    cl = cells.to(torch.int32).contiguous()
    rl = real.to(torch.uint8).contiguous()
    out = torch.empty((S, H, D), dtype=dt, device=q.device)
    lib = _lib.load()
    need = lib.sh_cells_attn_workspace(S, H, G, D, L)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    _lib.call("sh_cells_attn", qs.data_ptr(), kk.data_ptr(), vv.data_ptr(), kv_len, cl.data_ptr(), rl.data_ptr(), L,
              S, H, G, D, float(scale), _lib.dtype_code(dt), out.data_ptr(), ws.data_ptr(), ws.numel(),
              _lib.stream_of(qs))
    return out.reshape(1, S, H * D)


def _cells(chosen, ratio: int, S: int, kv_len: int):
    """attention.py:132-141: the cells of each query as a list (S, L) and which entries are real (S, L), from the
    indexer's choice (top (S, k) block ids, picked (S, k) bool, whole (S,) whole blocks before each query). Index
    arithmetic on the tensors' device."""
    top, picked, whole = chosen
    within = torch.arange(ratio, device=top.device)
    chosen_cells = (top[..., None] * ratio + within).reshape(S, -1)
    chosen_real = picked.repeat_interleave(ratio, dim=-1)
    own = (whole * ratio)[:, None] + within
    own_real = own <= torch.arange(kv_len - S, kv_len, device=top.device)[:, None]
    return (torch.cat([chosen_cells, torch.clamp(own, max=kv_len - 1)], dim=-1),
            torch.cat([chosen_real, own_real], dim=-1))
