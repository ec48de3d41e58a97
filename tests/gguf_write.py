"""A GGUF writer for the tests (test infrastructure), written from ggml's published format description (docs/gguf.md
of ggml: header, key/value metadata, tensor infos with dimensions fastest first, the data section aligned to
`general.alignment`), independently of the reader it checks."""

import struct

import numpy as np

VALUE_TYPE = {int: 5, float: 6, bool: 7, str: 8}  # int32, float32, bool, string
TYPE_ID = {"F32": 0, "F16": 1, "BF16": 30, "Q6_K": 14, "Q3_K": 11, "IQ4_NL": 20, "IQ4_XS": 23, "Q2_0": 42,
           "IQ2_XXS": 16, "IQ2_XS": 17, "IQ3_XXS": 18, "IQ3_S": 21, "IQ2_S": 22, "IQ1_M": 29}


def _string(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(v) -> bytes:
    if isinstance(v, bool):
        return struct.pack("<I?", 7, v)
    if isinstance(v, int):
        return struct.pack("<Ii", 5, v) if -2 ** 31 <= v < 2 ** 31 else struct.pack("<Iq", 11, v)
    if isinstance(v, float):
        return struct.pack("<If", 6, v)
    if isinstance(v, str):
        return struct.pack("<I", 8) + _string(v)
    if isinstance(v, (list, tuple)):
        if all(isinstance(e, int) and not isinstance(e, bool) for e in v):
            return struct.pack("<IIQ", 9, 5, len(v)) + b"".join(struct.pack("<i", e) for e in v)
        return struct.pack("<IIQ", 9, 8, len(v)) + b"".join(_string(e) for e in v)
    raise TypeError(type(v))


def write(path: str, meta: dict, tensors: list, alignment: int = 32, version: int = 3):
    """tensors: (name, shape in numpy order, type name, raw bytes uint8)."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta) + (alignment != 32))
    kv = b"".join(_string(k) + _value(v) for k, v in meta.items())
    if alignment != 32:
        kv += _string("general.alignment") + struct.pack("<II", 4, alignment)
    infos, data, offset = b"", b"", 0
    for name, shape, kind, raw in tensors:
        dims = tuple(reversed(shape))
        infos += _string(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
        infos += struct.pack("<IQ", TYPE_ID[kind], offset)
        blob = np.asarray(raw, np.uint8).tobytes()
        pad = (-len(blob)) % alignment
        data += blob + b"\0" * pad
        offset += len(blob) + pad
    body = head + kv + infos
    body += b"\0" * ((-len(body)) % alignment)
    with open(path, "wb") as f:
        f.write(body + data)
