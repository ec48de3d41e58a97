"""The library's C ABI over its host build (tests/hostrun: the kernels compiled for the CPU, each workgroup's threads
run as fibers): the CPU tests call the entry points with numpy buffers, exactly as the GPU tests call them with
device tensors, and compare the kernels' results with the oracle. Test infrastructure only."""

import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "hostrun"))

import build as _build  # noqa: E402  (tests/hostrun/build.py)

_libs = {}

DTYPE = {"float32": 0, "float16": 1, "bfloat16": 2}


class HostError(RuntimeError):
    pass


def load(asan: bool | None = None) -> ctypes.CDLL:
    """The host build (built first if the sources changed), with the package's prototypes. With HOSTRUN_ASAN=1 in
    the environment the AddressSanitizer build (the process must preload the sanitizer's runtime); with HOSTRUN_COV=1 the
    line-coverage build."""
    if asan is None:
        asan = os.environ.get("HOSTRUN_ASAN") == "1"
    cov = os.environ.get("HOSTRUN_COV") == "1"
    if asan not in _libs:
        from strata_hip import _lib as L

        lib = ctypes.CDLL(_build.build(asan=asan, verbose=False, cov=cov))
        for name, args in L.PROTOTYPES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                continue
            fn.argtypes = args
            fn.restype = L._RESTYPE.get(name, ctypes.c_int)
        _libs[asan] = lib
    return _libs[asan]


def call(name: str, *args) -> int:
    lib = load()
    status = getattr(lib, name)(*args)
    if status < 0:
        msg = lib.sh_last_error().decode(errors="replace")
        if status in (-1, -2):
            raise ValueError(msg)
        raise HostError(f"{name}: status {status}: {msg}")
    return status


def ptr(a):
    """The address of a numpy array's data (None for None)."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "contiguous buffers only"
    return a.ctypes.data


def bf16(a) -> np.ndarray:
    """float values -> bfloat16 bits (uint16), rounded to nearest even."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def from_bf16(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def act(a, dtype: str) -> np.ndarray:
    """Activations in the library's element type: float32, float16 or bfloat16 (as uint16 bits)."""
    if dtype == "float32":
        return np.ascontiguousarray(a, dtype=np.float32)
    if dtype == "float16":
        return np.ascontiguousarray(a, dtype=np.float16)
    return bf16(a)


def to_f32(a, dtype: str) -> np.ndarray:
    if dtype == "bfloat16":
        return from_bf16(a)
    return np.asarray(a, dtype=np.float32)


def empty(shape, dtype: str) -> np.ndarray:
    return np.zeros(shape, dtype={"float32": np.float32, "float16": np.float16, "bfloat16": np.uint16}[dtype])
