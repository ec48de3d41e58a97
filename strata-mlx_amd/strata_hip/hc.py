"""The hyper-connection read between two blocks over the HIP kernels — strata_mlx/fused.py:281-323 (FusedResidual),
its kernels at 46-131.

A decode layer's blocks read the HC residual streams through a hyper-connection and write back into them; the
write of the block before is folded into the read: the residual is `before + out * inject`. `FusedResidual(gr)` takes
the model's module (`hc_norm.weight`, `input_mix_weight_down.weight`, `input_mix_weight_up.weight`,
`block_inject_weight` or None, `hc`) as the reference does; `FusedResidual.from_weights` takes the tensors.
`__call__(before (1, T, HC D), out (1, T, D), inject_in (1, T, HC))` returns (the block's input (1, T, D), the
residual (1, T, HC D), inject for the block's output (1, T, HC), or inject_in without inject rows). A window of up
to 16 tokens is one call of the kernels; a longer one (a prompt) goes 16 tokens at a time, which gives the same
bits since every token's sums are its own.
"""

import torch

from . import _lib

MAX_TOKENS = 16  # tokens a call of the kernels


def _weight(t):
    w = getattr(t, "weight", t)
    return w if isinstance(w, torch.Tensor) else torch.as_tensor(w)


class FusedResidual:
    """A `GatedResidual` of the model, with the write that precedes it (strata_mlx/fused.py:281-323)."""

    def __init__(self, gr, eps: float = 1e-6):
        inject = getattr(gr, "block_inject_weight", None)
        self._setup(_weight(gr.hc_norm), _weight(gr.input_mix_weight_down), _weight(gr.input_mix_weight_up),
                    None if inject is None else _weight(inject), gr.hc, eps)

    @classmethod
    def from_weights(cls, norm, down, up, inject_w, hc: int, eps: float = 1e-6) -> "FusedResidual":
        self = cls.__new__(cls)
        self._setup(norm, down, up, inject_w, hc, eps)
        return self

    def _setup(self, norm, down, up, inject_w, hc, eps):
        self.rank, self.wide = down.shape
        if up.shape != (self.wide, self.rank) or norm.numel() != self.wide or self.wide % hc:
            raise ValueError(f"hyper-connection weights: norm {tuple(norm.shape)}, down {tuple(down.shape)}, "
                             f"up {tuple(up.shape)} for {hc} streams")
        if inject_w is not None and tuple(inject_w.shape) != (hc, self.wide):
            raise ValueError(f"inject weights {tuple(inject_w.shape)} for {hc} streams of {self.wide // hc}")
        self.hc, self.eps, self.d = hc, eps, self.wide // hc
        self.norm = norm.reshape(-1).float().contiguous()  # the kernels take the norm weights as float32
        self.down, self.up = down.contiguous(), up.to(down.dtype).contiguous()
        self.inject_w = None if inject_w is None else inject_w.to(down.dtype).contiguous()
        self._ws = {}

    def _workspace(self, tokens: int, device) -> torch.Tensor:
        key = (tokens, str(device))
        if key not in self._ws:
            n = _lib.load().sh_hc_workspace(tokens, self.hc, self.d, self.rank, self.hc if self.inject_w is not None
                                            else 0)
            self._ws[key] = torch.empty(n, dtype=torch.uint8, device=device)
        return self._ws[key]

    def __call__(self, before: torch.Tensor, out: torch.Tensor, inject_in: torch.Tensor):
        T, dtype = before.shape[-2], before.dtype
        if before.shape[-1] != self.wide or out.shape[-1] != self.d or inject_in.shape[-1] != self.hc:
            raise ValueError(f"FusedResidual: before {tuple(before.shape)}, out {tuple(out.shape)}, inject "
                             f"{tuple(inject_in.shape)} for {self.hc} streams of {self.d}")
        b = before.reshape(T, self.wide).contiguous()
        o = out.reshape(T, self.d).to(dtype).contiguous()
        i = inject_in.reshape(T, self.hc).to(dtype).contiguous()
        for w in (self.norm, self.down, self.up, self.inject_w):
            if w is not None and w.device != b.device:
                raise ValueError(f"FusedResidual: weights on {w.device}, activations on {b.device}")
        n_inject = self.hc if self.inject_w is not None else 0
        residual = torch.empty_like(b)
        mixed = torch.empty((T, self.d), dtype=dtype, device=b.device)
        inject = torch.empty((T, self.hc), dtype=dtype, device=b.device) if n_inject else None
        lib_dt, w_dt = _lib.dtype_code(dtype), _lib.dtype_code(self.down.dtype)
        for t0 in range(0, T, MAX_TOKENS):
            n = min(MAX_TOKENS, T - t0)
            ws = self._workspace(n, b.device)
            _lib.call("sh_hc_residual", b[t0:].data_ptr(), o[t0:].data_ptr(), i[t0:].data_ptr(), lib_dt,
                      self.norm.data_ptr(), self.down.data_ptr(), self.up.data_ptr(),
                      self.inject_w.data_ptr() if n_inject else None, w_dt, n, self.hc, self.d, self.rank, n_inject,
                      self.eps, residual[t0:].data_ptr(), mixed[t0:].data_ptr(),
                      inject[t0:].data_ptr() if n_inject else None, ws.data_ptr(), ws.numel(), _lib.stream_of(b))
        lead = before.shape[:-2]
        return (mixed.reshape(*lead, T, self.d), residual.reshape(*lead, T, self.wide),
                inject.reshape(*lead, T, self.hc) if n_inject else inject_in)
