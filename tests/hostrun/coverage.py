"""Line coverage of the library's sources by whatever ran on the coverage host build (test infrastructure).

    python tests/hostrun/build.py --cov
    STRATA_HOSTRUN=1 HOSTRUN_COV=1 python -m pytest tests -m gpu ...     (any selection; counts add up)
    python tests/hostrun/coverage.py [--lines]

gcov reads the counts the runs left beside the objects (tests/hostrun/_out/obj_cov) and this prints, for every
source of strata-mlx_amd/csrc, the share of its executable lines that ran, and with --lines the ranges that did
not. The rewritten copies the host build compiles keep the sources' line numbers, so the ranges are those of
strata-mlx_amd/csrc.
"""

import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "_out")
OBJ = os.path.join(OUT, "obj_cov")
SRC = os.path.join(OUT, "src")
ROOT = os.path.dirname(os.path.dirname(HERE))


def gcov_lines() -> dict:
    """{source file name: {line: count or None (not executable)}} over every object with counts. gcov runs from the
    repository root (the objects name their sources relative to it) and prints to its standard output; a line of a
    template appears once in sum and once an instantiation: it ran if any entry ran."""
    cover = {}
    src_rel = os.path.relpath(SRC, ROOT)
    row_re = re.compile(r"^\s*([0-9]+\*?|-|#####|=====):\s*([0-9]+):(.*)$")
    for f in sorted(os.listdir(OBJ)):
        if not f.endswith(".gcda") or f.startswith("hostrun"):
            continue
        obj = os.path.relpath(OBJ, ROOT)
        text = subprocess.run(["gcov", "-t", "-p", "-o", obj, os.path.join(obj, f)], cwd=ROOT, capture_output=True,
                              text=True, errors="replace").stdout
        src = None
        for row in text.splitlines():
            m = row_re.match(row)
            if not m:
                continue
            count, num, body = m.group(1), int(m.group(2)), m.group(3)
            if num == 0:
                if body.startswith("Source:"):
                    path = body[len("Source:"):].strip()
                    src = os.path.basename(path) if os.path.dirname(path) == src_rel else None
                continue
            if src is None:
                continue
            lines = cover.setdefault(src, {})
            if count == "-":
                lines.setdefault(num, None)
            else:
                c = 0 if count in ("#####", "=====") else int(count.rstrip("*"))
                lines[num] = max(lines.get(num) or 0, c)
    return cover


def ranges(nums):
    out, start, prev = [], None, None
    for n in sorted(nums):
        if start is None:
            start = prev = n
        elif n == prev + 1:
            prev = n
        else:
            out.append((start, prev))
            start = prev = n
    if start is not None:
        out.append((start, prev))
    return out


def main():
    cover = gcov_lines()
    if not cover:
        sys.exit("no counts: build with --cov and run tests with STRATA_HOSTRUN=1 HOSTRUN_COV=1 first")
    tot_run = tot_all = 0
    for name in sorted(cover):
        lines = cover[name]
        exe = [n for n, c in lines.items() if c is not None]
        ran = [n for n in exe if lines[n] > 0]
        tot_run += len(ran)
        tot_all += len(exe)
        print(f"{name:14s} {len(ran):5d} / {len(exe):5d} lines ran ({100.0 * len(ran) / max(1, len(exe)):.1f} %)")
        if "--lines" in sys.argv:
            missed = ranges([n for n in exe if lines[n] == 0])
            print("    not run: " + ", ".join(f"{a}" if a == b else f"{a}-{b}" for a, b in missed))
    print(f"{'all':14s} {tot_run:5d} / {tot_all:5d} lines ran ({100.0 * tot_run / max(1, tot_all):.1f} %)")


if __name__ == "__main__":
    main()
