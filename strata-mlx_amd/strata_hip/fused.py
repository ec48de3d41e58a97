"""The router's choice and the MoE block's end — strata_mlx/fused.py's interface (router product, top_k,
moe_combine, the routed MoE block) over HIP kernels (csrc/route.hip)."""

import torch

from . import _lib
from . import tables as _tables

ROUTER_TOPK = True   # fused.py:420
ROUTER_AS_IS = True  # fused.py:421
COMBINE_UPTO = 65535  # tokens a combine call takes (the reference stops at 16, what it checked against MLX)


class WindowLinear(torch.nn.Module):
    """A float16 / bfloat16 linear layer without bias whose products come back in float32, reading its weights as
    they are for a window of up to 8 tokens (strata_mlx/fused.py:357-390). `linear` is the model's layer (anything
    with a `weight` (rows, cols) tensor); longer inputs, or weights of other types, go through the layer itself as
    in the reference (`self.linear(x)`), or, for a layer that cannot be called, a float32 product."""

    upto = 8

    def __init__(self, linear):
        super().__init__()
        self.linear = linear
        self.rows, self.cols = linear.weight.shape

    @property
    def weight(self) -> torch.Tensor:
        return self.linear.weight

    def takes(self, x: torch.Tensor) -> bool:
        return x.numel() // self.cols <= self.upto and self.weight.dtype in (torch.float16, torch.bfloat16)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        tokens = x.numel() // self.cols
        if not self.takes(x):
            if callable(self.linear):
                return self.linear(x)
            return (x.reshape(-1, self.cols).float() @ self.weight.float().T).reshape(*x.shape[:-1], self.rows)
        xs = x.reshape(tokens, self.cols).contiguous()
        w = self.weight.contiguous()
        out = torch.empty((tokens, self.rows), dtype=torch.float32, device=x.device)
        _lib.call("sh_router_matvec", w.data_ptr(), _lib.dtype_code(w.dtype), self.rows, self.cols, xs.data_ptr(),
                  _lib.dtype_code(xs.dtype), tokens, out.data_ptr(), _lib.stream_of(xs))
        return out.reshape(*x.shape[:-1], self.rows)


def top_k(logits: torch.Tensor, k: int, weights: bool = False):
    """The indices of the k largest logits (..., N), largest first, ties to the lower index — the order
    `argpartition(-logits, k - 1)[..., :k]` gives (strata_mlx/fused.py:424-436). int32. With weights=True also
    the softmax of the chosen logits in float32 (fused.py:491), as a second result."""
    n = logits.shape[-1]
    flat = logits.reshape(-1, n).contiguous()
    rows = flat.shape[0]
    idx = torch.empty((rows, k), dtype=torch.int32, device=logits.device)
    w = torch.empty((rows, k), dtype=torch.float32, device=logits.device) if weights else None
    if rows:
        _lib.call("sh_top_k", flat.data_ptr(), _lib.dtype_code(flat.dtype), rows, n, k, idx.data_ptr(), _lib.ptr(w),
                  _lib.stream_of(flat))
    idx = idx.reshape(*logits.shape[:-1], k)
    return (idx, w.reshape(*logits.shape[:-1], k)) if weights else idx


def moe_combine(y: torch.Tensor, w: torch.Tensor, g: torch.Tensor, s: torch.Tensor) -> torch.Tensor | None:
    """y (..., K, D), w (..., K) float32, g (..., 1), s (..., D) -> (..., D): sum_k y_k w_k rounded to the
    activations' type, plus sigmoid(g) * s, in the reference's order and roundings (strata_mlx/fused.py:448-481).
    None where not taken (w not float32, or more tokens than COMBINE_UPTO)."""
    *lead, k, d = y.shape
    rows = y.numel() // (k * d) if k * d else 0
    if rows > COMBINE_UPTO or w.dtype != torch.float32:
        return None
    yc = y.reshape(rows, k, d).contiguous()
    wc = w.reshape(rows, k).contiguous()
    gc = g.reshape(rows).to(y.dtype).contiguous()
    sc = s.reshape(rows, d).to(y.dtype).contiguous()
    out = torch.empty((rows, d), dtype=y.dtype, device=y.device)
    if rows:
        _lib.call("sh_moe_combine", yc.data_ptr(), wc.data_ptr(), gc.data_ptr(), sc.data_ptr(), _lib.dtype_code(y.dtype),
                  rows, k, d, out.data_ptr(), _lib.stream_of(yc))
    return out.reshape(*lead, d)


class SwiGLUExpert:
    """The shared expert as mlx-lm's MLP computes it: down(swiglu(gate(x), up(x))), each projection a layer of the
    file's blocks (a BlockLinear, or anything called like `nn.Linear`)."""

    def __init__(self, gate_proj, up_proj, down_proj):
        self.gate_proj, self.up_proj, self.down_proj = gate_proj, up_proj, down_proj

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        from .blocks import swiglu

        return self.down_proj(swiglu(self.gate_proj(x), self.up_proj(x)))


FUSED = True  # windows the two-kernel decode takes go there (MoEDecode); False: always the composition


class _RoutedCall:
    """The MoE block's call with the router's choice made by `top_k` and its end by `moe_combine`
    (strata_mlx/fused.py:484-497, `_Routed.__call__`), over the block's own attributes: gate, switch_mlp,
    shared_expert, shared_expert_gate, top_k. A window the fused decode takes (routed experts as the file's Q2_0 /
    IQ3_S blocks, the shared expert's projections too, a window of up to 16 tokens) runs as the router's product
    and the two kernels of MoEDecode; any other as the reference composes it."""

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        gate = self.gate
        as_is = ROUTER_AS_IS and isinstance(gate, WindowLinear) and gate.takes(x)
        logits = gate(x if as_is else x.float())
        fused = self._fused_for(x)
        if fused is not None:
            return fused(logits, x)
        idx, w = top_k(logits, self.top_k, weights=True)
        y = self.switch_mlp(x, idx)
        g, s = self.shared_expert_gate(x), self.shared_expert(x)
        out = moe_combine(y, w, g, s) if COMBINE_UPTO else None
        if out is None:
            out = (y.float() * w[..., None]).sum(dim=-2).to(x.dtype) + torch.sigmoid(g.float()).to(x.dtype) * s
        return out

    def _fused_for(self, x: torch.Tensor):
        """The block's MoEDecode if it takes this window, else None (built once a block and activation type)."""
        from .blocks import BlockSwitchGLU

        if not FUSED or not isinstance(self.switch_mlp, BlockSwitchGLU):
            return None
        cache = self.__dict__.setdefault("_moe_decode", {})
        key = (x.dtype, x.device)
        if key not in cache:
            cache[key] = None
            sm, se = self.switch_mlp, self.shared_expert
            parts = [getattr(se, n, None) for n in ("gate_proj", "up_proj", "down_proj")]
            wg = getattr(self.shared_expert_gate, "weight", None)
            if (all(hasattr(p, "blocks") and hasattr(p, "kind") for p in parts) and isinstance(wg, torch.Tensor)
                    and wg.numel() == sm.gate_proj.input_dims and wg.dtype == x.dtype):
                try:
                    cache[key] = MoEDecode(sm.gate_proj, sm.up_proj, sm.down_proj, *parts, wg.reshape(-1), self.top_k)
                except ValueError:
                    cache[key] = None
        moe = cache[key]
        return moe if moe is not None and moe.takes(x) else None


class _Routed(_RoutedCall):
    """The MoE block as an object of its own (the reference swaps the class of mlx-lm's SparseMoeBlock instead:
    `install_routers` does that here for blocks of any class)."""

    def __init__(self, gate, switch_mlp, shared_expert, shared_expert_gate, top_k: int):
        self.gate, self.switch_mlp = gate, switch_mlp
        self.shared_expert, self.shared_expert_gate = shared_expert, shared_expert_gate
        self.top_k = top_k


Routed = _Routed
_routed_classes = {}


def install_routers(layers) -> None:
    """Make the routers of `layers` products of this kind (WindowLinear), and their blocks' call `_Routed`'s
    (strata_mlx/fused.py:500-507). A layer's `mlp` is taken when it has the MoE block's attributes; its class is
    swapped for a subclass whose call is the routed one, so its parameters stay where they are."""
    for layer in layers:
        mlp = getattr(layer, "mlp", None)
        if mlp is None or not all(hasattr(mlp, a) for a in ("gate", "switch_mlp", "shared_expert",
                                                               "shared_expert_gate", "top_k")):
            continue
        if isinstance(getattr(mlp.gate, "weight", None), torch.Tensor) and not isinstance(mlp.gate, WindowLinear):
            mlp.gate = WindowLinear(mlp.gate)
        cls = type(mlp)
        if not issubclass(cls, _RoutedCall):
            if cls not in _routed_classes:
                body = {"forward": _RoutedCall.__call__} if issubclass(cls, torch.nn.Module) else {}
                _routed_classes[cls] = type(f"Routed{cls.__name__}", (_RoutedCall, cls), body)
            mlp.__class__ = _routed_classes[cls]


class MoEDecode:
    """One MoE block's decode step for up to 16 tokens in three HIP kernels (csrc/moe.hip): route (top-k, weights,
    the shared expert's gate), gate/up with SwiGLU, down with the combine — what `Routed.__call__` computes
    (strata_mlx/fused.py:484-497) with the routed experts through switch_glu's bf16 branch (blocks.py:819-829).

    gate / up / down: BlockSwitchLinear stacks (Q2_0 or IQ3_S); shared_*: BlockSwitchLinear of one expert;
    shared_gate_w: the shared expert gate's weight (d_model,) in the activation type; k: experts a token."""

    MAX_TOKENS = 16

    def __init__(self, gate, up, down, shared_gate, shared_up, shared_down, shared_gate_w: torch.Tensor, k: int):
        from .blocks import KIND

        self.gate, self.up, self.down = gate, up, down
        self.shared = (shared_gate, shared_up, shared_down)
        self.shared_gate_w = shared_gate_w.contiguous()
        self.k = k
        self.experts, self.d_ff, self.d_model = gate.num_experts, gate.output_dims, gate.input_dims
        if up.kind != gate.kind or any(s.kind != l.kind for s, l in zip(self.shared, (gate, up, down))):
            raise ValueError("gate and up (and the shared expert's) must be of one kind")
        self.kinds = (KIND[gate.kind], KIND[down.kind])
        self._ws = {}

    def takes(self, x: torch.Tensor) -> bool:
        tokens = x.numel() // self.d_model
        v = self.experts // 64
        return (0 < tokens <= self.MAX_TOKENS and tokens * self.k <= 160 and x.dtype in (torch.float16, torch.bfloat16)
                and self.gate.kind in ("Q2_0", "IQ3_S") and self.down.kind in ("Q2_0", "IQ3_S")
                and self.experts % 64 == 0 and 1 <= v <= 32 and v & (v - 1) == 0
                and self.d_model % (256 if self.gate.kind == "IQ3_S" else 64) == 0 and self.d_model <= 8192
                and self.d_ff % (256 if self.down.kind == "IQ3_S" else 64) == 0)

    def workspace(self, tokens: int, dtype: torch.dtype, device) -> torch.Tensor:
        key = (tokens, dtype, str(device))
        if key not in self._ws:
            n = _lib.load().sh_moe_workspace(tokens, self.k, self.d_model, self.d_ff, _lib.dtype_code(dtype))
            self._ws[key] = torch.zeros(n, dtype=torch.uint8, device=device)
        return self._ws[key]

    def decode_into(self, logits: torch.Tensor, x: torch.Tensor, out: torch.Tensor, idx: torch.Tensor | None = None,
                    w: torch.Tensor | None = None) -> torch.Tensor:
        """The decode step into the caller's `out` (and optional idx int32 / w float32 of the choice) with nothing
        allocated: the library's own scratch array stands in for the workspace (sh_moe_decode_noalloc). For code
        under graph capture or loops that must not allocate; calls on one GPU must not overlap. Inputs and outputs
        contiguous."""
        tokens = x.numel() // self.d_model
        if not self.takes(x):
            raise ValueError(f"MoEDecode: {tokens} tokens of {x.dtype} (at most {self.MAX_TOKENS}, bf16/fp16)")
        for t in (logits, x, out) + tuple(a for a in (idx, w) if a is not None):
            if not t.is_contiguous():
                raise ValueError("decode_into: contiguous tensors expected")
        if out.numel() != x.numel() or out.dtype != x.dtype:
            raise ValueError(f"decode_into: out of {tuple(out.shape)} {out.dtype} for x of {tuple(x.shape)} {x.dtype}")
        needs = self.gate.kind == "IQ3_S" or self.down.kind == "IQ3_S"
        tabs = _tables.device_blob(x.device).data_ptr() if needs else None
        sg, su, sd = self.shared
        _lib.call("sh_moe_decode_noalloc", self.kinds[0], self.kinds[1], self.gate.blocks.data_ptr(),
                  self.up.blocks.data_ptr(), self.down.blocks.data_ptr(), self.experts, sg.blocks.data_ptr(),
                  su.blocks.data_ptr(), sd.blocks.data_ptr(), self.shared_gate_w.data_ptr(), tabs, logits.data_ptr(),
                  _lib.dtype_code(logits.dtype), x.data_ptr(), _lib.dtype_code(x.dtype), tokens, self.k, self.d_model,
                  self.d_ff, out.data_ptr(), _lib.ptr(idx), _lib.ptr(w), _lib.stream_of(x))
        return out

    def __call__(self, logits: torch.Tensor, x: torch.Tensor, want_choice: bool = False, phase: int | None = None,
                 out: torch.Tensor | None = None):
        """logits (..., experts) float32 or x's type; x (..., d_model). Returns (..., d_model) in x's type, and the
        choice (idx int32, weights float32) when want_choice. `phase` (0 route, 1 gate/up, 2 down) launches one of
        the three kernels alone, into `out` for phase 2 (for timing them one by one, in order)."""
        lead = x.shape[:-1]
        xs = x.reshape(-1, self.d_model).contiguous()
        ls = logits.reshape(-1, self.experts).contiguous()
        tokens = xs.shape[0]
        if not self.takes(xs):
            raise ValueError(f"MoEDecode: {tokens} tokens of {xs.dtype} (at most {self.MAX_TOKENS}, bf16/fp16)")
        if ls.dtype not in (torch.float32, xs.dtype):
            raise ValueError(f"MoEDecode: logits of {ls.dtype} with activations of {xs.dtype}")
        ws = self.workspace(tokens, xs.dtype, xs.device)
        out = torch.empty_like(xs) if out is None else out
        idx = torch.empty((tokens, self.k), dtype=torch.int32, device=xs.device) if want_choice else None
        w = torch.empty((tokens, self.k), dtype=torch.float32, device=xs.device) if want_choice else None
        needs = self.gate.kind == "IQ3_S" or self.down.kind == "IQ3_S"
        tabs = _tables.device_blob(xs.device).data_ptr() if needs else None
        sg, su, sd = self.shared
        if phase is not None:
            _lib.call("sh_moe_decode_phase", phase, self.kinds[0], self.kinds[1], self.gate.blocks.data_ptr(),
                      self.up.blocks.data_ptr(), self.down.blocks.data_ptr(), self.experts, sg.blocks.data_ptr(),
                      su.blocks.data_ptr(), sd.blocks.data_ptr(), self.shared_gate_w.data_ptr(), tabs, ls.data_ptr(),
                      _lib.dtype_code(ls.dtype), xs.data_ptr(), _lib.dtype_code(xs.dtype), tokens, self.k,
                      self.d_model, self.d_ff, out.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(xs))
            return out
        _lib.call("sh_moe_decode", self.kinds[0], self.kinds[1], self.gate.blocks.data_ptr(), self.up.blocks.data_ptr(),
                  self.down.blocks.data_ptr(), self.experts, sg.blocks.data_ptr(), su.blocks.data_ptr(),
                  sd.blocks.data_ptr(), self.shared_gate_w.data_ptr(), tabs, ls.data_ptr(), _lib.dtype_code(ls.dtype),
                  xs.data_ptr(), _lib.dtype_code(xs.dtype), tokens, self.k, self.d_model, self.d_ff, out.data_ptr(),
                  _lib.ptr(idx), _lib.ptr(w), ws.data_ptr(), ws.numel(), _lib.stream_of(xs))
        out = out.reshape(*lead, self.d_model)
        return (out, idx, w) if want_choice else out
