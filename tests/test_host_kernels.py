"""The kernels themselves on the CPU: a selection of the GPU tests run against the host build of the library
(tests/hostrun: the same HIP sources compiled for x86, a workgroup's threads as fibers, cross-lane operations and
MFMA restated from the ISA's lane layouts), with CPU tensors for device memory. The GPU tests compare every kernel
with the oracle; here they run where no GPU is, in a child process (STRATA_HOSTRUN=1), spread over a few workers.

STRATA_HOSTRUN_ASAN=1 runs the same selection on the AddressSanitizer build: every global and LDS access of the
kernels bounds-checked against the buffers the tests allocate (slower: about twice the time, and a build of its
own)."""

import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)

# (file, -k expression or None): small shapes of every kernel family; the full GPU files take longer on the CPU
SELECTION = [
    ("test_gpu_route.py", None),
    ("test_gpu_attention.py", None),
    ("test_gpu_attention_entry.py", None),
    ("test_gpu_hc.py", None),
    ("test_gpu_blocks.py", "dequantize or test_switch_matvec or separate or glu or lookup or window or three_and_four"),
    ("test_gpu_moe.py", "test_moe_decode_is_the_oracles_block or float32_logits_route or repeated_calls or many_experts "
                        "or whole_blocks"),
    ("test_gpu_tiles.py", "not 4096 and not skewed"),
    ("test_gpu_dropin.py", "not reference_models_shape and not install_routers"),
    ("test_gpu_stream.py", "not benchmark_shape and not many_items"),
]


def _run(asan: bool) -> subprocess.CompletedProcess:
    sys.path.insert(0, os.path.join(HERE, "hostrun"))
    import build as hb

    hb.build(asan=asan, verbose=False)  # before the workers start: one build, not one a worker
    env = dict(os.environ, STRATA_HOSTRUN="1", PYTHONDONTWRITEBYTECODE="1", OMP_NUM_THREADS="1")
    if asan:
        rt = subprocess.run(["/opt/rocm/llvm/bin/clang++", "-print-file-name=libclang_rt.asan-x86_64.so"],
                    capture_output=True, text=True).stdout.strip()
        env.update(HOSTRUN_ASAN="1", LD_PRELOAD=rt, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1")
    results = []
    for f, k in SELECTION:
        cmd = [sys.executable, "-m", "pytest", os.path.join("tests", f), "-m", "gpu", "-q", "-x", "-p",
               "no:cacheprovider", "-n", "4", "--timeout", "600"]
        if k:
            cmd += ["-k", k]
        r = subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True)
        results.append((f, r))
        if r.returncode not in (0, 5):  # 5: nothing selected
            return f, r
    return None, results


@pytest.mark.parametrize("asan", [False, True], ids=["host", "asan"])
def test_gpu_tests_pass_on_the_host_build(asan):
    if asan and os.environ.get("STRATA_HOSTRUN_ASAN") != "1":
        pytest.skip("the AddressSanitizer pass runs with STRATA_HOSTRUN_ASAN=1")
    failed, r = _run(asan)
    if failed:
        pytest.fail(f"{failed} on the host build:\n{r.stdout[-6000:]}\n{r.stderr[-4000:]}")
