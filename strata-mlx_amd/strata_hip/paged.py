"""Experts kept outside the GPU's memory and brought in as layers need them — strata_mlx/paged.py's PagedSwitchGLU
(paged.py:373-419) over the HIP kernels.

On MI355X a model's experts fit in HBM whole (288 GB), so this path is for a GPU shared with other work or a model
larger than its memory: each (layer, expert) is copied from the file's mapped bytes into a device buffer of its own
when a window first asks for it and kept in an LRU of a byte budget. A window of few pairs multiplies each pair's
expert where it lies (matvec_separate, the reference's `_separately`); more pairs build stacks of the used experts
(or take the whole layer) and go through switch_glu.
"""

from collections import OrderedDict

import numpy as np
import torch

from .blocks import BLOCK, MAX_SEPARATE, BlockSwitchLinear, matvec_separate, row_bytes, swiglu, switch_glu

SEPARATE_UPTO = 80  # paged.py:39: pairs a window multiplies expert by expert
WHOLE_FROM = 384  # paged.py:36: experts of a layer in one call from which its stacks are read whole
KEEP_UPTO = 640  # paged.py:37: pairs in one call up to which what was read stays (answers, not prompts)


class ExpertStore:
    """Device copies of experts, an LRU of `budget` bytes over (layer, expert). `layers[layer]` holds the layer's
    (up, gate, down) tensors: objects with `data` (the file's bytes, uint8, experts-major), `shape` (experts, rows,
    cols) and `type` (a block kind), such as gguf.Tensor."""

    def __init__(self, device, budget: int = 8 << 30):
        self.device, self.budget = device, budget
        self.layers = {}
        self.lru = OrderedDict()  # (layer, expert) -> (tensors, bytes)
        self.held = 0
        self.hits = self.misses = self.bytes_read = 0

    def _read(self, t, e: int) -> torch.Tensor:
        per = t.shape[1] * row_bytes(t.type, t.shape[2])
        raw = np.ascontiguousarray(np.asarray(t.data, np.uint8).reshape(-1)[e * per:(e + 1) * per])
        return torch.from_numpy(raw).to(self.device)

    def get(self, layer: int, tensors: tuple, experts: list, keep: bool = True) -> list:
        """Each expert's (up, gate, down) blocks on the device, in the order of `experts`."""
        missing = [e for e in experts if (layer, e) not in self.lru]
        self.hits += len(experts) - len(missing)
        self.misses += len(missing)
        got = {}
        for e in missing:
            got[e] = tuple(self._read(t, e) for t in tensors)
            size = sum(a.numel() for a in got[e])
            self.bytes_read += size
            if keep:
                self.lru[(layer, e)] = (got[e], size)
                self.held += size
        out = []
        for e in experts:
            if e in got:
                out.append(got[e])
            else:
                self.lru.move_to_end((layer, e))
                out.append(self.lru[(layer, e)][0])
        while self.held > self.budget and len(self.lru) > len(experts):  # what this call uses stays
            _, (_, size) = self.lru.popitem(last=False)
            self.held -= size
        return out

    def whole(self, tensors: tuple, layer: int) -> list:
        """The layer's three stacks on the device (not kept)."""
        return [torch.from_numpy(np.ascontiguousarray(np.asarray(t.data, np.uint8).reshape(-1))).to(self.device)
                for t in tensors]


class PagedSwitchGLU:
    """A layer's routed experts, called like mlx-lm's `SwitchGLU`, their weights in an `ExpertStore`
    (strata_mlx/paged.py:373-401)."""

    def __init__(self, layer: int, store: ExpertStore, gate, up, down):
        for t in (gate, up, down):
            if t.type not in BLOCK:
                raise ValueError(f"{getattr(t, 'name', t.type)}: {t.type} experts are not supported")
        self.layer, self.store, self.tensors = layer, store, (up, gate, down)
        store.layers[layer] = self.tensors

    def _linear(self, blocks: torch.Tensor, t, experts: int) -> BlockSwitchLinear:
        lin = BlockSwitchLinear(blocks, t.type, (experts, *t.shape[1:]))
        lin.unpack_from = 1 << 62  # a paged layer is never unpacked whole to floats
        return lin

    def __call__(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        idx = indices.cpu().numpy()  # the layer waits here for its router (paged.py:389)
        used, local = np.unique(idx, return_inverse=True)
        if idx.size <= SEPARATE_UPTO:
            return self._separately(x, idx, used)
        if len(used) >= WHOLE_FROM:
            stacks, n = self.store.whole(self.tensors, self.layer), self.tensors[0].shape[0]
        else:
            each = self.store.get(self.layer, self.tensors, used.tolist(), keep=idx.size <= KEEP_UPTO)
            stacks, n = [torch.cat(col) if len(col) > 1 else col[0] for col in zip(*each)], len(used)
            indices = torch.from_numpy(local.reshape(idx.shape).astype(np.int32)).to(x.device)
        up, gate, down = (self._linear(b, t, n) for b, t in zip(stacks, self.tensors))
        return switch_glu(x, indices, up, gate, down)

    def _separately(self, x: torch.Tensor, idx: np.ndarray, used: np.ndarray) -> torch.Tensor:
        """A few tokens: no stack is built, the kernels read each pair's expert where it lies
        (paged.py:403-419): gate and up of every pair by matvec_separate (one row of x to each token's k pairs),
        swiglu, down by matvec_separate (a row to each pair)."""
        k = idx.shape[-1]
        by = dict(zip(used.tolist(), self.store.get(self.layer, self.tensors, used.tolist())))
        pairs = [by[e] for e in idx.reshape(-1).tolist()]
        (_, hidden, wide), kinds = self.tensors[0].shape, [t.type for t in self.tensors]
        x = x.reshape(-1, wide)
        tokens = max(1, MAX_SEPARATE // k)  # tokens a call binds (the reference's limit of buffers a kernel)
        out = []
        for t in range(0, x.shape[0], tokens):
            ups, gates, downs = zip(*pairs[t * k:(t + tokens) * k])
            xs = x[t:t + tokens]
            h = swiglu(matvec_separate(list(gates), kinds[1], hidden, wide, xs, k),
                       matvec_separate(list(ups), kinds[0], hidden, wide, xs, k))
            out.append(matvec_separate(list(downs), kinds[2], wide, hidden, h, 1))
        out = torch.cat(out) if len(out) > 1 else out[0]
        return out.reshape(*idx.shape, wide)
