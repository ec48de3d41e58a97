"""The codebooks the block types read, as one blob of device memory.

strata-mlx takes ggml's grids from gguf-py at run time (strata_mlx/blocks.py:272-289): iq3s 512x4, iq3xxs 256x4,
iq2s 1024x8, iq2xs 512x8, iq2xxs 256x8, iq1 2048x8 (stored +1), ksigns 128 and the IQ4 values (gguf.py:34). The
kernels here take the same tables as data, in the fixed layout below (offsets shared with csrc/common.h).

Real tables: `use(load_npz(path))` with an .npz holding the arrays under the names of LAYOUT. Synthetic tables
(`synthetic(seed)`) obey what the real ones do: IQ3_S values odd in 1..15 (strata_mlx/gguf.py:11, 263), IQ3_XXS
values from {4, 12, ..., 62}, IQ2 values from {8, 25, 43}, IQ1 values in {0, 1, 2}, distinct entries, and ksigns
as seven sign bits completed to even parity.
"""

import hashlib

import numpy as np
import torch

KVALUES_IQ4NL = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], dtype=np.int8)

# name -> (byte offset, shape, dtype); must match csrc/common.h TAB_*
LAYOUT = {
    "kvalues": (0, (16,), np.int8),
    "ksigns": (16, (128,), np.uint8),
    "iq3s_grid": (144, (512, 4), np.uint8),
    "iq3xxs_grid": (2192, (256, 4), np.uint8),
    "iq2s_grid": (3216, (1024, 8), np.uint8),
    "iq2xs_grid": (11408, (512, 8), np.uint8),
    "iq2xxs_grid": (15504, (256, 8), np.uint8),
    "iq1_grid": (17552, (2048, 8), np.uint8),
}
IQ3S_SIGNED = 33936  # derived, uint8 [8192][4]: entry (index | signs << 9) -> 16 +- value (expert.hip)
BYTES = 66704

# which tables each block type reads
NEEDS = {"Q2_0": (), "Q3_K": (), "IQ4_NL": ("kvalues",), "IQ4_XS": ("kvalues",), "IQ3_S": ("iq3s_grid",),
         "IQ3_XXS": ("iq3xxs_grid", "ksigns"), "IQ2_S": ("iq2s_grid",), "IQ2_XS": ("iq2xs_grid", "ksigns"),
         "IQ2_XXS": ("iq2xxs_grid", "ksigns"), "IQ1_M": ("iq1_grid",)}


def even_parity_signs() -> np.ndarray:
    """ksigns: 7 stored sign bits k and an eighth that makes the count of set bits even."""
    k = np.arange(128)
    parity = np.array([bin(v).count("1") & 1 for v in k])
    return (k | (parity << 7)).astype(np.uint8)


def _distinct(rng, n: int, width: int, values) -> np.ndarray:
    values = np.asarray(values, dtype=np.uint8)
    seen, rows = set(), []
    while len(rows) < n:
        row = values[rng.integers(0, len(values), width)]
        key = row.tobytes()
        if key not in seen:
            seen.add(key)
            rows.append(row)
    return np.stack(rows)


def synthetic(seed: int = 0) -> dict:
    """Codebooks of the real tables' shapes and value sets, seeded."""
    rng = np.random.default_rng(seed)
    return {
        "kvalues": KVALUES_IQ4NL.copy(),
        "ksigns": even_parity_signs(),
        "iq3s_grid": _distinct(rng, 512, 4, range(1, 16, 2)),
        "iq3xxs_grid": _distinct(rng, 256, 4, [4, 12, 20, 28, 36, 44, 52, 62]),
        "iq2s_grid": _distinct(rng, 1024, 8, [8, 25, 43]),
        "iq2xs_grid": _distinct(rng, 512, 8, [8, 25, 43]),
        "iq2xxs_grid": _distinct(rng, 256, 8, [8, 25, 43]),
        "iq1_grid": _distinct(rng, 2048, 8, [0, 1, 2]),
    }


def iq3s_signed(grid: np.ndarray) -> np.ndarray:
    """The IQ3_S grid with every sign pattern applied: entry (index | signs << 9) holds, for each of the four
    values, 16 + value or 16 - value (sign bit j of the nibble set), as uint8 (8192, 4)."""
    g = np.asarray(grid, dtype=np.int16).reshape(512, 4)
    e = np.arange(8192)
    signs = (e[:, None] >> (9 + np.arange(4))) & 1
    return (16 + np.where(signs == 1, -g[e & 511], g[e & 511])).astype(np.uint8)


def blob(tables: dict) -> np.ndarray:
    """The tables in the library's layout, uint8 (BYTES,), with the derived tables appended."""
    out = np.zeros(BYTES, dtype=np.uint8)
    for name, (at, shape, dt) in LAYOUT.items():
        a = np.ascontiguousarray(np.asarray(tables[name]).astype(dt).reshape(shape))
        out[at:at + a.nbytes] = a.view(np.uint8).reshape(-1)
    out[IQ3S_SIGNED:IQ3S_SIGNED + 8192 * 4] = iq3s_signed(tables["iq3s_grid"]).reshape(-1)
    return out


def load_npz(path: str) -> dict:
    with np.load(path, allow_pickle=False) as f:
        return {name: f[name] for name in LAYOUT}


def digest(tables: dict) -> str:
    return hashlib.sha256(blob(tables).tobytes()).hexdigest()


_current = None
_on_device = {}


def use(tables: dict) -> None:
    """Make `tables` the codebooks every later call reads."""
    global _current
    _current = {k: np.asarray(v) for k, v in tables.items()}
    _on_device.clear()


def current() -> dict:
    if _current is None:
        raise RuntimeError("no codebooks: call strata_hip.tables.use(...) with real or synthetic tables first")
    return _current


def device_blob(device) -> torch.Tensor:
    """The current tables as a uint8 tensor on `device` (uploaded once per device)."""
    device = torch.device(device)
    key = (device.type, device.index)
    if key not in _on_device:
        _on_device[key] = torch.from_numpy(blob(current())).to(device)
    return _on_device[key]
