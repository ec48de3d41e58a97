"""GGUF files: the tensor table and metadata of a model's shards, each tensor's bytes as a view into the mapped file
(strata_mlx/gguf.py:25-132), and the MoE layer built from them on the GPU (the expert part of strata_mlx/load.py:
259-263, 411-421). Nothing is converted: expert stacks and block-typed dense tensors go to the device as the file
holds them and the kernels decode them there; float tensors and Q6_K come back as float32 (gguf.py:135-164).

The format (ggml's GGUF, versions 2 and 3, little-endian): magic "GGUF", uint32 version, uint64 tensor count,
uint64 metadata count; metadata as (string key, uint32 type, value); tensor infos as (string name, uint32 dims,
uint64 dims fastest first, uint32 type, uint64 offset into the data section); the data section starts at the next
multiple of `general.alignment` (32 by default). Strings are uint64 length + UTF-8 bytes.
"""

import mmap
import re
import struct
from dataclasses import dataclass

import numpy as np

# type id -> (name, weights per block, bytes per block): strata_mlx/gguf.py:25-33
TYPES = {
    0: ("F32", 1, 4), 1: ("F16", 1, 2), 30: ("BF16", 1, 2),
    2: ("Q4_0", 32, 18), 6: ("Q5_0", 32, 22), 8: ("Q8_0", 32, 34),
    11: ("Q3_K", 256, 110), 12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210),
    20: ("IQ4_NL", 32, 18), 23: ("IQ4_XS", 256, 136), 42: ("Q2_0", 64, 18),
    16: ("IQ2_XXS", 256, 66), 17: ("IQ2_XS", 256, 74), 18: ("IQ3_XXS", 256, 98), 21: ("IQ3_S", 256, 110),
    22: ("IQ2_S", 256, 82), 29: ("IQ1_M", 256, 56),
}
TYPE_ID = {v[0]: k for k, v in TYPES.items()}
# metadata value types: uint8, int8, uint16, int16, uint32, int32, float32, bool, (8 string), (9 array), uint64,
# int64, float64
_SCALAR = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}


@dataclass
class Tensor:
    name: str
    shape: tuple  # numpy order: the last axis is the one a row runs along
    type: str
    data: np.ndarray  # the raw bytes (uint8), a view into the file
    path: str = ""
    offset: int = 0  # where in the file the bytes start

    @property
    def quantized(self) -> bool:
        return self.type not in ("F32", "F16", "BF16")


class GGUF:
    """One GGUF file, mapped read-only: `meta` (key -> value) and `tensors` (name -> Tensor)."""

    def __init__(self, path: str):
        self.path = path
        self._f = open(path, "rb")
        self._map = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        buf = self._map
        pos = [4]

        def rd(fmt):
            out = struct.unpack_from("<" + fmt, buf, pos[0])
            pos[0] += struct.calcsize("<" + fmt)
            return out if len(out) > 1 else out[0]

        def string():
            n = rd("Q")
            s = bytes(buf[pos[0]:pos[0] + n]).decode("utf-8", "replace")
            pos[0] += n
            return s

        def value(t):
            if t == 8:
                return string()
            if t == 9:
                et, n = rd("IQ")
                return [value(et) for _ in range(n)]
            if t not in _SCALAR:
                raise ValueError(f"{path}: metadata value type {t}")
            return rd(_SCALAR[t])

        if bytes(buf[:4]) != b"GGUF":
            raise ValueError(f"{path} is not a GGUF file")
        self.version, n_tensors, n_kv = rd("IQQ")
        if self.version not in (2, 3):
            raise ValueError(f"{path}: GGUF version {self.version}")
        self.meta = {}
        for _ in range(n_kv):
            key = string()
            self.meta[key] = value(rd("I"))
        infos = []
        for _ in range(n_tensors):
            name = string()
            n_dims = rd("I")
            dims = struct.unpack_from(f"<{n_dims}Q", buf, pos[0])
            pos[0] += 8 * n_dims
            type_id, offset = rd("IQ")
            infos.append((name, tuple(reversed(dims)), type_id, offset))
        align = self.meta.get("general.alignment", 32)
        start = (pos[0] + align - 1) // align * align
        raw = np.frombuffer(buf, dtype=np.uint8)
        self.tensors = {}
        for name, shape, type_id, offset in infos:
            if type_id not in TYPES:
                raise ValueError(f"{name}: GGUF tensor type {type_id} is not supported")
            kind, per_block, block_bytes = TYPES[type_id]
            n = int(np.prod(shape))
            if shape and shape[-1] % per_block:
                raise ValueError(f"{name}: rows of {shape[-1]} weights do not end on a block of {per_block}")
            n_bytes = n // per_block * block_bytes
            if start + offset + n_bytes > len(raw):
                raise ValueError(f"{name}: {n_bytes} bytes at {start + offset} past the end of {path}")
            self.tensors[name] = Tensor(name, shape, kind, raw[start + offset:start + offset + n_bytes], path,
                                        start + offset)

    def __getitem__(self, name: str) -> Tensor:
        return self.tensors[name]

    def __contains__(self, name: str) -> bool:
        return name in self.tensors


_SPLIT = re.compile(r"-(\d{5})-of-(\d{5})\.gguf$")


def shards(path: str) -> list:
    """A model's files: the one named and, where its name says it is one of several, the others beside it
    (strata_mlx/gguf.py:125-132)."""
    m = _SPLIT.search(path)
    count = int(m.group(2)) if m else 1
    return [GGUF(path)] + [GGUF(_SPLIT.sub(f"-{i:05d}-of-{m.group(2)}.gguf", path)) for i in range(2, count + 1)]


def to_float(t: Tensor) -> np.ndarray:
    """A float tensor, or a Q6_K one, as float32 (strata_mlx/gguf.py:135-147)."""
    if t.type == "F32":
        return t.data.view("<f4").reshape(t.shape)
    if t.type == "F16":
        return t.data.view("<f2").astype(np.float32).reshape(t.shape)
    if t.type == "BF16":
        return (t.data.view("<u2").astype(np.uint32) << 16).view(np.float32).reshape(t.shape)
    if t.type == "Q6_K":
        from .dense import q6k_parts

        rows = int(np.prod(t.shape[:-1]))
        codes, scales, d = q6k_parts(t.data, rows, t.shape[-1])
        s = np.repeat(scales.astype(np.float32), 16, axis=1) * np.repeat(d.astype(np.float32), 256, axis=1)
        return (codes.astype(np.float32) * s).reshape(t.shape)
    raise ValueError(f"{t.name}: {t.type} stays blocks (the kernels decode it)")


# ---- a MoE layer from a file's tensors, on the GPU (strata_mlx/load.py:259-263, 411-421)

def _device_bytes(t: Tensor, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(t.data)).to(device)


def experts(t: Tensor, device):
    """A stack of experts (experts, rows, cols), kept as the file's blocks (load.py:259-263)."""
    from .blocks import BLOCK, BlockSwitchLinear

    if t.type not in BLOCK:
        raise ValueError(f"{t.name}: {t.type} experts are not supported")
    return BlockSwitchLinear(_device_bytes(t, device), t.type, t.shape)


def dense(t: Tensor, device, dtype=None):
    """A dense layer (rows, cols) called like nn.Linear (load.py:235-252): block kinds stay blocks (BlockLinear),
    Q6_K its three parts (ScaledLinear), float tensors a weight of `dtype` (FloatLinear)."""
    import torch

    from .blocks import BLOCK
    from .dense import BlockLinear, FloatLinear, ScaledLinear, fits

    if t.type in BLOCK:
        return BlockLinear(_device_bytes(t, device), t.type, t.shape)
    if t.type == "Q6_K" and fits(*t.shape):
        return ScaledLinear.from_blocks(t.data, t.shape[0], t.shape[1], device)
    return FloatLinear(torch.from_numpy(np.ascontiguousarray(to_float(t))).to(dtype or torch.float16).to(device))


def moe_layer(files, layer: int, device, dtype=None):
    """Layer `layer`'s MoE block from a model's files (a GGUF or a list of shards): the router (ffn_gate_inp) as a
    WindowLinear, the routed experts (ffn_{gate,up,down}_exps) as a BlockSwitchGLU, the shared expert
    (ffn_{gate,up,down}_shexp) and its gate (ffn_gate_inp_shexp), joined by _Routed (load.py:411-421)."""
    import torch

    from .blocks import BlockSwitchGLU
    from .dense import FloatLinear
    from .fused import SwiGLUExpert, WindowLinear, _Routed

    dtype = dtype or torch.float16
    files = files if isinstance(files, (list, tuple)) else [files]
    found = {}
    for f in files:
        found.update(f.tensors)

    def take(name):
        key = f"blk.{layer}.{name}"
        if key not in found:
            raise KeyError(f"{key}: not in the model's files")
        return found[key]

    router = FloatLinear(torch.from_numpy(np.ascontiguousarray(to_float(take("ffn_gate_inp.weight")))).to(dtype)
                         .to(device))
    gate_w = torch.from_numpy(np.ascontiguousarray(to_float(take("ffn_gate_inp_shexp.weight")))).to(dtype).to(device)
    routed = BlockSwitchGLU(*(experts(take(f"ffn_{p}_exps.weight"), device) for p in ("gate", "up", "down")))
    shared = SwiGLUExpert(*(dense(take(f"ffn_{p}_shexp.weight"), device, dtype) for p in ("gate", "up", "down")))
    k = None
    for f in files:
        for key, v in f.meta.items():
            if key.endswith(".expert_used_count"):
                k = int(v)
    if k is None:
        raise KeyError("expert_used_count: not in the model's metadata")
    return _Routed(WindowLinear(router), routed, shared, FloatLinear(gate_w.reshape(1, -1)), k)
