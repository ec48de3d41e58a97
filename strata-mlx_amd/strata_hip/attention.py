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
                           ctx_len: int, scale: float | None = None, gate: torch.Tensor | None = None) -> torch.Tensor:
    """q (B, Hq, D) the window's B queries, the last B positions of a context of ctx_len; k_pages / v_pages
    (n_pages, Hkv, 16, D); page_table (>= ceil(ctx_len / 16),) int32 physical page of each 16 positions.
    Query t sees positions 0 .. ctx_len - B + t. Returns (B, Hq, D) in q's dtype; scale defaults to D ** -0.5.
    `gate` (B, Hq, D), a view whose last axis is contiguous, makes the output out * sigmoid(gate) (attention.py:261),
    applied as the splits merge."""
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
    if gate is None:
        _lib.call("sh_paged_attn", q.data_ptr(), k_pages.data_ptr(), v_pages.data_ptr(), page_table.data_ptr(),
                  n_pages, ctx_len, B, Hq, Hkv, D, scale, _lib.dtype_code(dt), out.data_ptr(), ws.data_ptr(),
                  ws.numel(), _lib.stream_of(q))
        return out
    ts, hs = _gate_strides(gate, (B, Hq, D), dt)
    _lib.call("sh_paged_attn_gated", q.data_ptr(), k_pages.data_ptr(), v_pages.data_ptr(), page_table.data_ptr(),
              n_pages, ctx_len, B, Hq, Hkv, D, scale, _lib.dtype_code(dt), gate.data_ptr(), ts, hs, out.data_ptr(),
              ws.data_ptr(), ws.numel(), _lib.stream_of(q))
    return out


def _gate_strides(gate: torch.Tensor, shape: tuple, dtype) -> tuple:
    if tuple(gate.shape) != tuple(shape) or gate.dtype != dtype or gate.stride(-1) != 1:
        raise ValueError(f"gate {tuple(gate.shape)} {gate.dtype} (stride {gate.stride()}) for {shape} {dtype}")
    return gate.stride(0), gate.stride(1)


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


# ---- the attention entry (attention.py:228-261): norm and rope, the paged cache, the gated output

QK_ROPE_UPTO = 16  # attention.py:207: windows the reference's fused norm-and-rope kernel takes (one kernel here for all)


def qk_rope(x: torch.Tensor, weight: torch.Tensor, eps: float, cos: torch.Tensor, sin: torch.Tensor, heads: int,
            head_dim: int, stride: int, heads_first: bool = True) -> torch.Tensor:
    """attention.py:216-222: x (1, S, heads * stride), each head's head_dim values first; each head's rms norm with
    `weight` and `eps`, then rope on the first rot dims (cos / sin (S, rot) in x's type), every step rounded to x's
    type. Returns (1, heads, S, head_dim), or (S, heads, head_dim) with heads_first False (the paged kernels' order)."""
    S = x.numel() // (heads * stride)
    xs = x.reshape(S, heads * stride).contiguous()
    rot = cos.shape[-1]
    c = cos.reshape(S, rot).to(x.dtype).contiguous()
    s = sin.reshape(S, rot).to(x.dtype).contiguous()
    w = weight.to(x.dtype).contiguous()
    _on_dev(xs, c, s, w)
    shape = (heads, S, head_dim) if heads_first else (S, heads, head_dim)
    out = torch.empty(shape, dtype=x.dtype, device=x.device)
    _lib.call("sh_qk_rope", xs.data_ptr(), _lib.dtype_code(x.dtype), S, heads, head_dim, stride, w.data_ptr(),
              float(eps), c.data_ptr(), s.data_ptr(), rot, out.data_ptr(), int(heads_first), _lib.stream_of(xs))
    return out[None] if heads_first else out


def _on_dev(*ts):
    for t in ts:
        if t.device != ts[0].device:
            raise ValueError(f"tensors on {t.device} and {ts[0].device}")
    _lib.stream_of(ts[0])


class PagedKVCache:
    """A layer's keys and values in pages of PAGE positions — the cache `Attention.__call__` appends to and reads
    (mlx-lm's `_AttnCache` at attention.py:251; `trim` as the engine trims rejected drafts, engine.py:710-749).

    k_pages / v_pages (n_pages, n_kv_heads, 16, head_dim); page_table int32 (n_pages,): the physical page of each
    logical page (any order: pages need not be contiguous). `offset` positions are held."""

    def __init__(self, n_pages: int, n_kv_heads: int, head_dim: int, dtype=torch.float16, device="cuda",
                 page_table: torch.Tensor | None = None):
        self.k_pages = torch.zeros((n_pages, n_kv_heads, PAGE, head_dim), dtype=dtype, device=device)
        self.v_pages = torch.zeros_like(self.k_pages)
        self.page_table = (torch.arange(n_pages, dtype=torch.int32, device=device) if page_table is None
                           else page_table.to(torch.int32).to(device).contiguous())
        self.offset = 0

    @property
    def capacity(self) -> int:
        return self.page_table.numel() * PAGE

    def update_and_fetch(self, k: torch.Tensor, v: torch.Tensor):
        """Append a window's keys and values, (S, n_kv_heads, head_dim) each, at the current offset; returns the
        pools (what the paged attention reads with the new offset)."""
        S, hkv, D = k.shape
        if v.shape != k.shape or hkv != self.k_pages.shape[1] or D != self.k_pages.shape[3]:
            raise ValueError(f"keys {tuple(k.shape)} / values {tuple(v.shape)} for pages {tuple(self.k_pages.shape)}")
        if self.offset + S > self.capacity:
            raise ValueError(f"{self.offset} + {S} positions in a cache of {self.capacity}")
        k, v = k.to(self.k_pages.dtype).contiguous(), v.to(self.k_pages.dtype).contiguous()
        _lib.call("sh_kv_append", k.data_ptr(), v.data_ptr(), S, hkv, D, _lib.dtype_code(k.dtype),
                  self.k_pages.data_ptr(), self.v_pages.data_ptr(), self.page_table.data_ptr(),
                  self.page_table.numel(), self.k_pages.shape[0], self.offset, _lib.stream_of(k))
        self.offset += S
        return self.k_pages, self.v_pages

    def trim(self, n: int) -> int:
        """Drop the last n positions (drafts a verify pass rejected); returns how many were dropped."""
        n = min(self.offset, n)
        self.offset -= n
        return n

    def is_trimmable(self) -> bool:
        return True


class Attention:
    """A decode layer's attention (strata_mlx/attention.py:228-261, `Attention.__call__`) over a paged cache.

    The module's own parts: q_proj (its output per head: head_dim of query, then head_dim of output gate), k_proj,
    v_proj, o_proj (anything called like `nn.Linear`: BlockLinear, ScaledLinear, ...), the q / k norm weights and
    eps, the head counts and scale. A call: the queries' and keys' norm and rope (qk_rope), the window's keys and
    values appended to the cache, paged attention with the causal mask among the window's queries and the output
    gate applied as its splits merge, then o_proj. `chosen` (the indexer's choice, attention.py:88-115: top blocks,
    which are picked, whole blocks a query) makes each query attend to its gathered cells instead (attention.py:255-
    256; `_cells` and `_gathered`), read through the page table."""

    def __init__(self, q_proj, k_proj, v_proj, o_proj, q_norm_weight, k_norm_weight, n_heads: int, n_kv_heads: int,
                 head_dim: int, scale: float | None = None, eps: float = 1e-6, compress_ratio: int = 4):
        self.q_proj, self.k_proj, self.v_proj, self.o_proj = q_proj, k_proj, v_proj, o_proj
        self.q_norm_weight, self.k_norm_weight = q_norm_weight, k_norm_weight
        self.n_heads, self.n_kv_heads, self.head_dim = n_heads, n_kv_heads, head_dim
        self.scale = head_dim ** -0.5 if scale is None else scale
        self.eps = eps
        self.compress_ratio = compress_ratio

    def __call__(self, x: torch.Tensor, rope, mask=None, cache: PagedKVCache | None = None, idx_cache=None,
                 chosen=None) -> torch.Tensor:
        """x (1, S, d_model); rope(positions) -> (cos, sin), each (S, rot) (or with leading axes of one);
        `mask` is the model's causal mask, built in here (accepted for the reference's signature)."""
        B, S, _ = x.shape
        if B != 1 or not isinstance(cache, PagedKVCache):
            raise ValueError("one conversation, with a paged cache")
        H, G, D = self.n_heads, self.n_kv_heads, self.head_dim
        offset = cache.offset
        cos, sin = rope(torch.arange(offset, offset + S, device=x.device))
        rot = cos.shape[-1]
        cos, sin = cos.reshape(S, rot), sin.reshape(S, rot)
        proj = self.q_proj(x).reshape(S, H, 2 * D)
        q = qk_rope(proj, self.q_norm_weight, self.eps, cos, sin, H, D, 2 * D, heads_first=False)
        k = qk_rope(self.k_proj(x), self.k_norm_weight, self.eps, cos, sin, G, D, D, heads_first=False)
        v = self.v_proj(x).reshape(S, G, D)
        cache.update_and_fetch(k, v)
        kv_len = cache.offset
        gate = proj[..., D:]
        if chosen is None:
            out = paged_decode_attention(q, cache.k_pages, cache.v_pages, cache.page_table, kv_len, self.scale, gate)
        else:
            out = self._gathered_gated(q, cache, chosen, S, kv_len, gate)
        return self.o_proj(out.reshape(1, S, H * D))

    def _gathered_gated(self, q, cache, chosen, S, kv_len, gate):
        """attention.py:255-256 over the paged pool: each query's cells (`_cells`), read through the page table, the
        output gate applied as the splits merge."""
        H, G, D = self.n_heads, self.n_kv_heads, self.head_dim
        cells, real = _cells(chosen, self.compress_ratio, S, kv_len)
        cl = cells.to(torch.int32).contiguous()
        rl = real.to(torch.uint8).contiguous()
        L = cl.shape[1]
        out = torch.empty((S, H, D), dtype=q.dtype, device=q.device)
        lib = _lib.load()
        need = lib.sh_cells_attn_workspace(S, H, G, D, L)
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
        ts, hs = _gate_strides(gate, (S, H, D), q.dtype)
        _lib.call("sh_cells_attn_paged", q.data_ptr(), cache.k_pages.data_ptr(), cache.v_pages.data_ptr(),
                  cache.page_table.data_ptr(), cache.page_table.numel(), cl.data_ptr(), rl.data_ptr(), L, S, H, G, D,
                  float(self.scale), _lib.dtype_code(q.dtype), gate.data_ptr(), ts, hs, out.data_ptr(), ws.data_ptr(),
                  ws.numel(), _lib.stream_of(q))
        return out
