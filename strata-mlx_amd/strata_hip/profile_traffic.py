"""The workload for reading k_moe_front's HBM traffic with rocprofv3 counters (FETCH_SIZE, then WRITE_SIZE, one
counter a run), and the summary of the two runs.

    rocprofv3 --pmc FETCH_SIZE --output-format csv -d DIR/fetch -o f -- python3 -m strata_hip.profile_traffic run
    rocprofv3 --pmc WRITE_SIZE --output-format csv -d DIR/write -o w -- python3 -m strata_hip.profile_traffic run
    python3 -m strata_hip.profile_traffic summarize DIR > profiles/moe_front_traffic.json

`run` first copies 256 MiB device to device (hipMemcpyAsync's copy kernel, whose HBM bytes are known: 256 MiB read,
256 MiB written),
then launches the front of the benchmark's MoE layer (512 experts, d_model 2048, ffn 512, Q2_0, top-10) over 48
distinct layers at each batch 1, 2, 4, 8. `summarize` scales each counter by what it read for the copy (its
calibration) and reports the bytes a front launch moves, against its algorithmic bytes.
"""

import csv
import glob
import json
import os
import sys

COPY_BYTES = 256 * 2**20
BATCHES = (1, 2, 4, 8)


def run():
    import torch

    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(os.path.dirname(here))
    for p in (os.path.dirname(here), root):
        if p not in sys.path:
            sys.path.insert(0, p)
    import bench
    import strata_hip
    from strata_hip import fused as SF
    from strata_hip import tables as T

    strata_hip.load()
    T.use(T.synthetic(0))
    dev = torch.device("cuda:0")
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    layers, _ = bench.build_layers(48, dev, "Q2_0")
    algo = {}
    for b in BATCHES:
        g = torch.Generator(device=dev)
        g.manual_seed(1000 + b)
        lg = [torch.randn(b, bench.E, device=dev, generator=g).to(torch.bfloat16) for _ in layers]
        xs = [torch.randn(b, bench.D, device=dev, generator=g).to(torch.bfloat16) for _ in layers]
        uniq = [int(torch.unique(SF.top_k(l, bench.K)).numel()) for l in lg]
        for m, l, x in zip(layers, lg, xs):
            m(l, x, phase=1)
        torch.cuda.synchronize()
        algo[b] = sum(bench.front_bytes(u, b) for u in uniq) / len(uniq)
        print(f"B={b}: front launches {len(layers)}, algorithmic bytes a launch {algo[b]:.0f}", flush=True)
    print(json.dumps({"algorithmic_bytes_per_launch": algo}), flush=True)


def _counters(d, name):
    """[(dispatch id, kernel name, value)] of counter `name` in a rocprofv3 csv directory, in dispatch order"""
    out = []
    for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            if r["Counter_Name"] == name:
                out.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
    return sorted(out)


def summarize(d):
    fetch, write = _counters(os.path.join(d, "fetch"), "FETCH_SIZE"), _counters(os.path.join(d, "write"), "WRITE_SIZE")
    # the calibration: the copy (hipMemcpyAsync's copy kernel), 256 MiB read and 256 MiB written
    cf = next(v for _, k, v in fetch if "copyBuffer" in k)
    cw = next(v for _, k, v in write if "copyBuffer" in k)
    kf, kw = COPY_BYTES / cf, COPY_BYTES / cw
    f = [v for _, k, v in fetch if "k_moe_front" in k]
    w = [v for _, k, v in write if "k_moe_front" in k]
    if not f or len(f) != len(w) or len(f) % len(BATCHES):
        raise SystemExit(f"k_moe_front dispatches: {len(f)} read, {len(w)} written")
    per = {}
    n = len(f) // len(BATCHES)  # in launch order: 48 a batch
    for i, b in enumerate(BATCHES):
        per[str(b)] = {"fetch_bytes": round(sum(f[i * n:(i + 1) * n]) / n * kf),
                       "write_bytes": round(sum(w[i * n:(i + 1) * n]) / n * kw)}
    mean = sum(v["fetch_bytes"] + v["write_bytes"] for v in per.values()) / len(per)
    print(json.dumps({
        "kernel": "k_moe_front", "workload": "MoE layer front, 512 experts, d_model 2048, ffn 512, Q2_0, top-10, "
                                             "48 distinct layers at each batch 1, 2, 4, 8",
        "counters": "rocprofv3 --pmc FETCH_SIZE, then --pmc WRITE_SIZE (KiB a dispatch)",
        "commands": ["cd /tmp && export TMPDIR=/tmp PYTHONPATH=$R/strata-mlx_amd:$R  (R: the repository root, "
                     "OUT: an output directory)",
                     "rocprofv3 --pmc FETCH_SIZE --output-format csv -d $OUT/fetch -o f -- "
                     "python3 -m strata_hip.profile_traffic run",
                     "rocprofv3 --pmc WRITE_SIZE --output-format csv -d $OUT/write -o w -- "
                     "python3 -m strata_hip.profile_traffic run",
                     "python3 -m strata_hip.profile_traffic summarize $OUT"],
        "calibration": {"copy_bytes": COPY_BYTES, "fetch_kib_read": cf, "write_kib_read": cw,
                        "fetch_scale": kf, "write_scale": kw},
        "per_batch": per, "traffic_bytes_per_launch": round(mean)}, indent=1))


if __name__ == "__main__":
    if len(sys.argv) < 2 or sys.argv[1] not in ("run", "summarize"):
        raise SystemExit(__doc__)
    run() if sys.argv[1] == "run" else summarize(sys.argv[2])
