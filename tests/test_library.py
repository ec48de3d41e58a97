"""The C ABI library loads and exports every entry point include/strata_hip.h declares (no GPU needed: nothing
here launches a kernel)."""

import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "strata_hip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sh_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = declared()
    for n in ("sh_dequantize", "sh_switch_matvec", "sh_top_k", "sh_moe_combine", "sh_tiles_of"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from strata_hip import _lib

    if not os.path.exists(_lib.LIBRARY):
        pytest.fail(f"{_lib.LIBRARY} is not built (python __graft_entry__.py build)")
    lib = ctypes.CDLL(_lib.LIBRARY)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_host_only_entry_points_answer_without_a_gpu():
    from strata_hip import _lib, tables

    lib = _lib.load()
    assert lib.sh_version() >= 1
    assert lib.sh_tables_bytes() == tables.BYTES
    wpb, bpb = ctypes.c_int(), ctypes.c_int()
    assert lib.sh_kind_block(3, ctypes.byref(wpb), ctypes.byref(bpb)) == 0 and (wpb.value, bpb.value) == (256, 110)
    assert lib.sh_kind_block(99, None, None) < 0
    assert b"unknown block kind" in lib.sh_last_error()
    assert lib.sh_tiles_most(20480, 512) == 20480 // 16 + 512


def test_shape_errors_are_reported_before_any_launch():
    from strata_hip import _lib

    lib = _lib.load()
    # IQ3_S rows of 640 weights do not end on a block: rejected on the host, nothing launched
    st = lib.sh_dequantize(3, 1, 1, 1, 4, 640, 1, 0, None)
    assert st == -2 and b"do not end on a block" in lib.sh_last_error()
    st = lib.sh_top_k(1, 0, 4, 4096, 10, 1, None, None)
    assert st == -2


def test_the_one_launch_layer_cannot_be_switched_on():
    """The one-launch MoE layer is switched off until its fault's fix has run on a GPU: asking for it is refused on
    the host, and the setting stays off."""
    from strata_hip import _lib

    lib = _lib.load()
    assert lib.sh_moe_set_one_launch(0) == 0
    assert lib.sh_moe_set_one_launch(1) == -7 and b"switched off" in lib.sh_last_error()
    assert lib.sh_moe_set_one_launch(0) == 0


def test_hyper_connection_shapes_are_checked_before_any_launch():
    from strata_hip import _lib

    lib = _lib.load()
    assert lib.sh_hc_workspace(8, 4, 2560, 128, 4) > 8 * 4 * 2560 * 4  # normed, partial sums, low-rank values
    p = 16
    # 17 tokens, 3 streams, rank 48, inject rows that are not the streams: each refused on the host
    for args, what in (((17, 4, 128, 32, 4), b"tokens"), ((2, 3, 128, 32, 3), b"streams"),
                       ((2, 4, 96, 32, 4), b"multiple of 64"), ((2, 4, 128, 48, 4), b"rank"),
                       ((2, 4, 128, 32, 2), b"inject rows")):
        st = lib.sh_hc_residual(p, p, p, 1, p, p, p, p, 1, *args, 1e-6, p, p, p, p, 1 << 30, None)
        assert st == -2 and what in lib.sh_last_error(), (args, lib.sh_last_error())
