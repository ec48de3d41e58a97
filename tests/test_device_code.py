"""The library's gfx950 code, disassembled from the built libstrata_hip.so on the CPU (code built here, nothing
launched): every direct load into LDS is issued outside the wait-state windows the hardware needs and the compiler
does not enforce before inline assembly (5 after a VALU instruction writes an SGPR the load reads, 1 after M0 is
written), and no instruction writes through the scalar data cache."""

import os
import re
import shutil
import subprocess

import pytest

from strata_hip import _lib

OBJDUMP = "/opt/rocm/llvm/bin/llvm-objdump"
SGPR = re.compile(r"^s(\d+)$|^s\[(\d+):(\d+)\]$")
SCALAR_WRITES = ("s_store", "s_buffer_store", "s_scratch_store", "s_atomic", "s_buffer_atomic", "s_dcache_wb",
                 "s_dcache_discard")


def sgprs(op: str) -> set:
    m = SGPR.match(op)
    if not m:
        return set()
    if m.group(1) is not None:
        return {int(m.group(1))}
    return set(range(int(m.group(2)), int(m.group(3)) + 1))


def disassemble(library: str, workdir) -> dict:
    """{kernel: [(mnemonic, [operands])]} of every gfx950 code object bundled in `library`."""
    lib = os.path.join(workdir, "lib.so")
    shutil.copy(library, lib)
    subprocess.run([OBJDUMP, "--offloading", lib], cwd=workdir, check=True, capture_output=True)
    funcs = {}
    for obj in sorted(p for p in os.listdir(workdir) if p.endswith("gfx950")):
        text = subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", os.path.join(workdir, obj)], check=True,
                              capture_output=True, text=True).stdout
        name = None
        for line in text.splitlines():
            m = re.match(r"^[0-9a-f]+ <(\S+)>:$", line)
            if m:
                name = m.group(1)
                funcs[name] = []
                continue
            if name and line.startswith("\t"):
                ins = line.split("//")[0].strip()
                if ins:
                    mnem, _, ops = ins.partition(" ")
                    funcs[name].append((mnem, [o.strip() for o in ops.split(",")] if ops else []))
    return funcs


def load_hazards(funcs: dict):
    """(direct-load sites, [(kernel, index, what)] of those inside a wait-state window)"""
    sites, bad = 0, []
    for name, ins in funcs.items():
        for i, (mnem, ops) in enumerate(ins):
            if not mnem.startswith("global_load_lds"):
                continue
            sites += 1
            read = set().union(*(sgprs(o) for o in ops[1:]))
            waits, j = 0, i - 1
            while j >= 0 and waits < 5:
                m, o = ins[j]
                if m == "s_nop":
                    waits += int(o[0], 0) + 1
                    j -= 1
                    continue
                if m.startswith("v_") and o and sgprs(o[0]) & read:
                    bad.append((name, i, f"{m} {','.join(o)} {waits} wait states before"))
                    break
                if o and o[0] == "m0" and waits < 1:
                    bad.append((name, i, f"{m} m0 directly before"))
                    break
                waits += 1
                j -= 1
    return sites, bad


def scalar_writes(funcs: dict):
    return [(name, m) for name, ins in funcs.items() for m, _ in ins if m.startswith(SCALAR_WRITES)]


@pytest.fixture(scope="module")
def code(tmp_path_factory):
    if not os.path.exists(OBJDUMP) or not os.path.exists(_lib.LIBRARY):
        pytest.skip("llvm-objdump or the built library is missing")
    funcs = disassemble(_lib.LIBRARY, tmp_path_factory.mktemp("device_code"))
    assert funcs, "no device code found"
    return funcs


def test_direct_loads_wait_out_the_sgpr_and_m0_windows(code):
    sites, bad = load_hazards(code)
    assert sites > 100
    assert not bad, bad[:10]


def test_nothing_writes_through_the_scalar_data_cache(code):
    found = scalar_writes(code)
    assert not found, found[:10]
