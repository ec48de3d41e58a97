"""ctypes binding of libstrata_hip.so, the C ABI over the HIP kernels (declared in include/strata_hip.h).

Every entry point returns 0 or a negative status; `call` turns a status into an exception carrying the library's
message. Pointers are device pointers of torch tensors; the stream is the current torch stream of the tensors'
device. There is no fallback: without the built library every call raises.
"""

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(_HERE, "libstrata_hip.so")

c_i64, c_int, c_vp, c_sz = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t

# name -> argument types (all return int unless listed in _RESTYPE)
PROTOTYPES = {
    "sh_version": [],
    "sh_last_error": [],
    "sh_kind_block": [c_int, c_vp, c_vp],
    "sh_tables_bytes": [],
    "sh_dequantize": [c_int, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_int, c_vp],
    "sh_switch_matvec": [c_int, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp, c_int, c_i64, c_vp, c_vp, c_sz, c_vp],
    "sh_switch_matvec_generic": [c_int, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp, c_int, c_i64, c_vp, c_vp],
    "sh_switch_workspace": [c_int, c_i64, c_i64, c_i64, c_int],
    "sh_matvec_separate": [c_int, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_int, c_i64, c_vp, c_vp],
    "sh_window_matvec": [c_int, c_vp, c_vp, c_i64, c_i64, c_vp, c_int, c_i64, c_vp, c_vp],
    "sh_matvec_glu": [c_int, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp, c_vp, c_int, c_vp, c_vp],
    "sh_lookup_table": [c_vp, c_int, c_i64, c_i64, c_vp, c_vp],
    "sh_lookup_table_glu": [c_vp, c_vp, c_int, c_i64, c_i64, c_vp, c_vp],
    "sh_lookup_matvec": [c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp, c_int, c_i64, c_vp, c_vp],
    "sh_lookup_down_glu": [c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp, c_vp, c_int, c_vp, c_vp],
    "sh_router_matvec": [c_vp, c_int, c_i64, c_i64, c_vp, c_int, c_i64, c_vp, c_vp],
    "sh_hc_workspace": [c_i64, c_i64, c_i64, c_i64, c_i64],
    "sh_hc_residual": [c_vp, c_vp, c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_int, c_i64, c_i64, c_i64, c_i64, c_i64,
                       ctypes.c_float, c_vp, c_vp, c_vp, c_vp, c_sz, c_vp],
    "sh_top_k": [c_vp, c_int, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp],
    "sh_moe_combine": [c_vp, c_vp, c_vp, c_vp, c_int, c_i64, c_i64, c_i64, c_vp, c_vp],
    "sh_tiles_workspace": [c_i64],
    "sh_tiles_most": [c_i64, c_i64],
    "sh_tiles_of": [c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp, c_sz, c_vp],
    "sh_moe_workspace": [c_i64, c_i64, c_i64, c_i64, c_int],
    "sh_moe_decode": [c_int, c_int, c_vp, c_vp, c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_vp, c_int,
                      c_i64, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp, c_sz, c_vp],
    "sh_stack_workspace": [c_int, c_i64, c_i64, c_i64, c_i64, c_int],
    "sh_stack_matvec": [c_int, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_int, c_i64, c_vp, c_vp, c_sz, c_vp],
    "sh_stack_takes": [c_int, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_int, c_i64],
    "sh_moe_decode_phase": [c_int, c_int, c_int, c_vp, c_vp, c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int,
                            c_vp, c_int, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp, c_sz, c_vp],
    "sh_moe_set_tail_combine": [c_int],
    "sh_moe_set_one_launch": [c_int],
    "sh_tiles_set_share": [c_int],
    "sh_moe_scratch_bytes": [],
    "sh_moe_decode_noalloc": [c_int, c_int, c_vp, c_vp, c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_vp,
                              c_int, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp],
    "sh_scaled_matvec": [c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_int, c_i64, c_vp, c_vp],
    "sh_scaled_floats": [c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_int, c_vp],
    "sh_tile_matmul": [c_int, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_int, c_i64, c_vp, c_vp, c_vp],
    "sh_tile_glu": [c_int, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_int, c_i64, c_vp, c_i64, c_vp, c_vp,
                    c_vp],
    "sh_tile_down": [c_int, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_int, c_i64, c_vp, c_vp, c_i64, c_vp, c_vp],
    "sh_paged_attn_workspace": [c_i64, c_i64, c_i64, c_i64, c_i64],
    "sh_paged_attn": [c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, ctypes.c_float, c_int, c_vp,
                      c_vp, c_sz, c_vp],
    "sh_paged_attn_gated": [c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, ctypes.c_float, c_int,
                            c_vp, c_i64, c_i64, c_vp, c_vp, c_sz, c_vp],
    "sh_cells_attn_paged": [c_vp, c_vp, c_vp, c_vp, c_i64, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64,
                            ctypes.c_float, c_int, c_vp, c_i64, c_i64, c_vp, c_vp, c_sz, c_vp],
    "sh_qk_rope": [c_vp, c_int, c_i64, c_i64, c_i64, c_i64, c_vp, ctypes.c_float, c_vp, c_vp, c_i64, c_vp, c_int, c_vp],
    "sh_kv_append": [c_vp, c_vp, c_i64, c_i64, c_i64, c_int, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp],
    "sh_cells_attn_workspace": [c_i64, c_i64, c_i64, c_i64, c_i64],
    "sh_cells_attn": [c_vp, c_vp, c_vp, c_i64, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, ctypes.c_float, c_int,
                      c_vp, c_vp, c_sz, c_vp],
}
_RESTYPE = {"sh_last_error": ctypes.c_char_p, "sh_tables_bytes": c_sz, "sh_tiles_workspace": c_sz,
            "sh_tiles_most": c_i64, "sh_switch_workspace": c_sz,
            "sh_moe_workspace": c_sz, "sh_hc_workspace": c_sz, "sh_stack_workspace": c_sz, "sh_paged_attn_workspace": c_sz,
            "sh_cells_attn_workspace": c_sz, "sh_moe_scratch_bytes": c_sz}

_lib = None


class StrataHipError(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """The library, loaded once; raises if it has not been built (python -m strata_hip.build)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY):
            raise StrataHipError(f"{LIBRARY} is not built: run `python __graft_entry__.py build` or "
                                 f"`python -m strata_hip.build`")
        lib = ctypes.CDLL(LIBRARY)
        for name, args in PROTOTYPES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                continue
            fn.argtypes = args
            fn.restype = _RESTYPE.get(name, c_int)
        _lib = lib
    return _lib


def call(name: str, *args) -> int:
    status = getattr(load(), name)(*args)
    if status < 0:
        msg = load().sh_last_error().decode(errors="replace")
        if status == -1 or status == -2:
            raise ValueError(msg)
        raise StrataHipError(f"{name}: status {status}: {msg}")
    return status


DTYPE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE[dtype]
    except KeyError:
        raise ValueError(f"activations of {dtype}: float32, float16 or bfloat16 expected") from None


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    if t.device.type != "cuda":
        raise ValueError(f"tensor on {t.device}: the HIP kernels take tensors on the GPU")
    return torch.cuda.current_stream(t.device).cuda_stream
