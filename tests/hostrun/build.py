"""Compile the library's HIP sources for the host (test infrastructure: the CPU tests run the kernels themselves with
it; the package never loads it).

    python tests/hostrun/build.py [--asan] [--cov]

The sources in strata-mlx_amd/csrc are copied to tests/hostrun/_out/src with four mechanical rewrites the host
compiler needs, and compiled as C++ against hip/hip_runtime.h of this directory (the device environment restated
for the host) into tests/hostrun/_out/libstrata_host.so (libstrata_host_asan.so with AddressSanitizer):
  - `extern __shared__ T name[];` becomes a pointer to the workgroup's dynamic LDS;
  - inline assembly: a direct load into LDS (global_load_lds_dwordx4) becomes hostrun::load_lds of its source and M0;
    waits and scheduling hints (s_waitcnt, s_nop, empty statements) become nothing;
  - SH_LDS_ADDR takes the offset into the dynamic LDS;
  - in the direct-load helpers the operands they make scalar are each lane's own (see _uniform_direct_loads).
A build is reused while the hash of the sources and of this directory's files matches the one it was made from.
"""

import hashlib
import os
import re
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
# HOSTRUN_CSRC / HOSTRUN_OUT: another tree's sources into another output (two versions of a kernel side by side)
CSRC = os.environ.get("HOSTRUN_CSRC", os.path.join(ROOT, "strata-mlx_amd", "csrc"))
OUT = os.environ.get("HOSTRUN_OUT", os.path.join(HERE, "_out"))
CXX = os.environ.get("HOSTRUN_CXX", "/opt/rocm/llvm/bin/clang++")


def library_path(asan: bool = False, cov: bool = False) -> str:
    return os.path.join(OUT, "libstrata_host" + ("_asan" if asan else "") + ("_cov" if cov else "") + ".so")


def _inputs():
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp", ".h")))
    own = [os.path.join(HERE, "hostrun.cpp"), os.path.join(HERE, "hip", "hip_runtime.h"), os.path.abspath(__file__)]
    return [os.path.join(CSRC, f) for f in srcs], own


def source_hash() -> str:
    srcs, own = _inputs()
    h = hashlib.sha256()
    for p in srcs + own:
        h.update(os.path.basename(p).encode())
        with open(p, "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def _close(text: str, i: int) -> int:
    """Index just past the parenthesis that closes the one at text[i]."""
    depth, j = 0, i
    while j < len(text):
        c = text[j]
        if c == '"':
            j += 1
            while text[j] != '"':
                j += 2 if text[j] == "\\" else 1
        elif c == "(":
            depth += 1
        elif c == ")":
            depth -= 1
            if depth == 0:
                return j + 1
        j += 1
    raise ValueError("unbalanced asm statement")


def _split_top(s: str, sep: str):
    parts, depth, cur, j = [], 0, "", 0
    while j < len(s):
        c = s[j]
        if c == '"':
            k = j + 1
            while s[k] != '"':
                k += 2 if s[k] == "\\" else 1
            cur += s[j:k + 1]
            j = k + 1
            continue
        if c == "(":
            depth += 1
        elif c == ")":
            depth -= 1
        if c == sep and depth == 0:
            parts.append(cur)
            cur = ""
        else:
            cur += c
        j += 1
    parts.append(cur)
    return parts


def _operands(section: str) -> dict:
    """{constraint: expression} of an operand list `"v"(a), "s"(b), ...`."""
    ops = {}
    for item in _split_top(section, ","):
        item = item.strip()
        if not item:
            continue
        m = re.match(r'"([^"]*)"\s*\((.*)\)\s*$', item, re.S)
        if not m:
            raise ValueError(f"asm operand {item!r}")
        ops[m.group(1)] = m.group(2)
    return ops


def _asm(stmt: str) -> str:
    body = stmt[stmt.index("(") + 1:-1]
    sections = _split_top(body, ":")
    template = "".join(re.findall(r'"((?:[^"\\]|\\.)*)"', sections[0]))
    if "global_load_lds_dwordx4" in template:
        ins = _operands(sections[2])
        m0 = ins["{m0}"]
        if ", off" in template:
            return f"::hostrun::load_lds((const void*)({ins['v']}), (uint32_t)({m0}))"
        return (f"::hostrun::load_lds((const char*)({ins['s']}) + (uint32_t)({ins['v']}), "
                f"(uint32_t)({m0}))")
    m = re.fullmatch(r"v_mov_b32 %0, %1", template.strip())
    if m:  # a move into a vector register
        return f"(({_operands(sections[1])['=v']}) = ({_operands(sections[2])['s']}))"
    if "global_" in template or "buffer_" in template or "ds_" in template or "v_" in template:
        raise ValueError(f"no host form for the inline assembly {template!r}")
    return "((void)0)"  # waits, s_nop, scheduling fences


def _uniform_direct_loads(text: str) -> str:
    """In the direct-load helpers, the operands they move to scalar registers (wave-uniform by contract) are each
    lane's own: the helpers are also called under lane conditions, where a cross-lane operation would wait for lanes
    that never come."""
    for name in ("lds_dma16", "lds_dma16p"):
        m = re.search(r"void " + name + r"\(.*?\n}\n", text, re.S)
        if m:
            body = m.group(0).replace("__builtin_amdgcn_readfirstlane(", "::hostrun::lane_value(")
            text = text[:m.start()] + body + text[m.end():]
    return text


def rewrite(text: str) -> str:
    text = _uniform_direct_loads(text)
    text = re.sub(r"extern\s+__shared__\s+([\w:]+)\s+(\w+)\[\];",
                  r"\1* const \2 = (\1*)::hostrun::lds_base();", text)
    text = re.sub(r"#define SH_LDS_ADDR\(arr\) .*", "#define SH_LDS_ADDR(arr) (::hostrun::lds_addr(arr))", text)
    out, i = [], 0
    for m in re.finditer(r"\basm\s*(?:volatile\s*)?\(", text):
        if m.start() < i:
            continue
        end = _close(text, m.end() - 1)
        out.append(text[i:m.start()])
        stmt = text[m.start():end]
        out.append(_asm(stmt) + "\n" * stmt.count("\n"))  # (line numbers kept: coverage and messages)
        i = end
    out.append(text[i:])
    return "".join(out)


def build(asan: bool = False, verbose: bool = True, cov: bool = False) -> str:
    """The library, rebuilt when its sources changed; one build at a time across processes (a lock file). cov: line
    coverage (gcov's notes and counts beside the objects in _out/obj_cov)."""
    import fcntl

    os.makedirs(OUT, exist_ok=True)
    with open(os.path.join(OUT, ".lock"), "w") as lock:
        fcntl.flock(lock, fcntl.LOCK_EX)
        return _build(asan, verbose, cov)


def _build(asan: bool, verbose: bool, cov: bool = False) -> str:
    lib = library_path(asan, cov)
    stamp = lib + ".hash"
    h = source_hash()
    if os.path.exists(lib) and os.path.exists(stamp) and open(stamp).read().strip() == h:
        return lib
    src_dir = os.path.join(OUT, "src")
    obj_dir = os.path.join(OUT, "obj" + ("_asan" if asan else "") + ("_cov" if cov else ""))
    os.makedirs(src_dir, exist_ok=True)
    os.makedirs(obj_dir, exist_ok=True)
    srcs, _ = _inputs()
    units = []
    for p in srcs:
        name = os.path.basename(p)
        with open(p) as f:
            text = rewrite(f.read())
        dst = os.path.join(src_dir, name)
        with open(dst, "w") as f:
            f.write(text)
        if not name.endswith(".h"):
            units.append(dst)
    units.append(os.path.join(HERE, "hostrun.cpp"))
    flags = ["-std=c++17", "-O2", "-fPIC", "-g0", "-w", "-x", "c++", "-I", HERE, "-I", src_dir,
             "-fno-strict-aliasing"]
    if asan:
        flags += ["-fsanitize=address", "-fno-omit-frame-pointer"]
    if cov:
        flags += ["--coverage"]

    def compile_one(src):
        obj = os.path.join(obj_dir, os.path.basename(src) + ".o")
        r = subprocess.run([CXX, *flags, "-c", src, "-o", obj], capture_output=True, text=True)
        return obj, r.returncode, r.stderr

    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as pool:
        results = list(pool.map(compile_one, units))
    bad = [(o, e) for o, rc, e in results if rc]
    if bad:
        raise RuntimeError("host build failed:\n" + "\n".join(f"{o}:\n{e[-4000:]}" for o, e in bad))
    link = [CXX, "-shared", "-fPIC", "-o", lib + ".tmp", *[o for o, _, _ in results]]
    if asan:
        link += ["-fsanitize=address", "-shared-libasan"]
    if cov:
        link += ["--coverage"]
    r = subprocess.run(link, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"host link failed:\n{r.stderr}")
    os.replace(lib + ".tmp", lib)
    with open(stamp, "w") as f:
        f.write(h)
    if verbose:
        print(f"built {lib}", file=sys.stderr)
    return lib


if __name__ == "__main__":
    build(asan="--asan" in sys.argv, cov="--cov" in sys.argv)
