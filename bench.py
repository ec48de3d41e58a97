"""MoE-layer decode on one MI355X: microseconds a layer and effective HBM GB/s, Q2_0 experts, batch 1-8 tokens.

Workload (synthetic, seeded): d_model 2048, 512 routed experts + 1 shared, expert width 512, SwiGLU, every expert
weight in GGUF Q2_0 blocks (453 MB a layer); router logits bf16 N(0,1), softmax then top-10 with renormalised
weights; hidden states bf16 N(0,1). A step is one decode pass through 48 distinct such layers (21.7 GB of expert
blocks, far beyond the 256 MB Infinity Cache) at each verify width B = 1, 2, 4, 8, as the reference times its
48-layer chains. Each width's 48 layers are one captured graph on one stream, so layer after layer runs in order.

value = algorithmic bytes of all timed layers / their time, where a layer's bytes are the blocks of the experts its
tokens actually chose (counted from the routing) plus the shared expert, plus activations in and out:
(U + 1) * 884,736 + B * 9,216 + 4,096.

roofline: the dominant kernel, k_moe_front (route, then gate/up with SwiGLU: two thirds of the expert bytes), its
launches timed by HIP events around a graph of them alone; its algorithmic bytes are the gate and up blocks of the
chosen and the shared experts, the logits and hidden states in, swiglu(gate, up) out. traffic: the HBM bytes a
launch moves by the FETCH_SIZE / WRITE_SIZE counters (profiles/moe_front_traffic.json), reported only when that
summary was read on this source of the kernel (its hash of csrc/moe.hip matches), else null. cpu_baseline: the numpy
oracle's restatement of the reference's dequantize + matmul path on the host, over a bounded sample of the same
layers, on one thread and on all cores.

    python bench.py [--steps K] [--warmup W] [--layers 48] [--batches 1,2,4,8] [--no-cpu]

The counter summary (two runs under rocprofv3, one counter each, then the summary; R the repository root, OUT an
output directory, from /tmp with TMPDIR=/tmp):

    rocprofv3 --pmc FETCH_SIZE --output-format csv -d $OUT/fetch -o f -- python3 $R/bench.py --traffic-run
    rocprofv3 --pmc WRITE_SIZE --output-format csv -d $OUT/write -o w -- python3 $R/bench.py --traffic-run
    python3 $R/bench.py --traffic-summarize $OUT > $R/profiles/moe_front_traffic.json

--traffic-run first copies 256 MiB device to device (hipMemcpyAsync's copy kernel: 256 MiB read, 256 MiB written,
the counters' calibration), then launches the front of the benchmark's layer over 48 distinct layers at each batch
1, 2, 4, 8; --traffic-summarize scales each counter by what it read for the copy and reports the bytes a front
launch moves.
"""

import argparse
import csv
import glob
import hashlib
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "strata-mlx_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "MoE-layer decode µs + effective HBM GB/s (Q2_0, IQ3_S), batch 1-8 tokens"
E, D, F, K = 512, 2048, 512, 10
EXPERT_BYTES = 3 * 294_912  # gate + up + down of one Q2_0 expert
EXPERT_BYTES_IQ3S = 3 * 450_560  # of one IQ3_S expert (512 x 2048 at 110 bytes a 256)
HBM_PEAK_GBS = 8000.0


def layer_bytes(u: int, b: int, expert_bytes: int = EXPERT_BYTES) -> int:
    return (u + 1) * expert_bytes + b * 9_216 + 4_096


def front_bytes(u: int, b: int, expert_bytes: int = EXPERT_BYTES) -> int:
    # gate + up blocks of the chosen and the shared experts, logits and x in, swiglu(gate, up) out
    return (u + 1) * 2 * expert_bytes // 3 + b * E * 2 + b * D * 2 + (b * K + b) * F * 2


MOE_SOURCE = os.path.join(ROOT, "strata-mlx_amd", "csrc", "moe.hip")
TRAFFIC_JSON = os.path.join(ROOT, "profiles", "moe_front_traffic.json")
COPY_BYTES = 256 * 2**20
TRAFFIC_BATCHES = (1, 2, 4, 8)


def source_hash() -> str:
    with open(MOE_SOURCE, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def front_traffic():
    """HBM bytes a k_moe_front launch moves, averaged over the batches the counters were read at; None without the
    committed counter summary or when it was read on another source of the kernel."""
    if not os.path.exists(TRAFFIC_JSON):
        return None
    with open(TRAFFIC_JSON) as f:
        summary = json.load(f)
    if summary.get("source_sha256") != source_hash():
        print("# traffic: the counter summary was read on another source of csrc/moe.hip; reported as null",
              file=sys.stderr)
        return None
    return summary.get("traffic_bytes_per_launch")


def traffic_run():
    """The workload the two counter runs read: the calibration copy, then the front launches."""
    import torch

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
    layers, _ = build_layers(48, dev, "Q2_0")
    algo = {}
    for b in TRAFFIC_BATCHES:
        g = torch.Generator(device=dev)
        g.manual_seed(1000 + b)
        lg = [torch.randn(b, E, device=dev, generator=g).to(torch.bfloat16) for _ in layers]
        xs = [torch.randn(b, D, device=dev, generator=g).to(torch.bfloat16) for _ in layers]
        uniq = [int(torch.unique(SF.top_k(l, K)).numel()) for l in lg]
        for m, l, x in zip(layers, lg, xs):
            m(l, x, phase=1)
        torch.cuda.synchronize()
        algo[b] = sum(front_bytes(u, b) for u in uniq) / len(uniq)
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


def traffic_summarize(d):
    fetch, write = _counters(os.path.join(d, "fetch"), "FETCH_SIZE"), _counters(os.path.join(d, "write"), "WRITE_SIZE")
    cf = next(v for _, k, v in fetch if "copyBuffer" in k)  # the copy: 256 MiB read and 256 MiB written
    cw = next(v for _, k, v in write if "copyBuffer" in k)
    kf, kw = COPY_BYTES / cf, COPY_BYTES / cw
    f = [v for _, k, v in fetch if "k_moe_front" in k]
    w = [v for _, k, v in write if "k_moe_front" in k]
    if not f or len(f) != len(w) or len(f) % len(TRAFFIC_BATCHES):
        raise SystemExit(f"k_moe_front dispatches: {len(f)} read, {len(w)} written")
    per = {}
    n = len(f) // len(TRAFFIC_BATCHES)  # in launch order: 48 a batch
    for i, b in enumerate(TRAFFIC_BATCHES):
        per[str(b)] = {"fetch_bytes": round(sum(f[i * n:(i + 1) * n]) / n * kf),
                       "write_bytes": round(sum(w[i * n:(i + 1) * n]) / n * kw)}
    mean = sum(v["fetch_bytes"] + v["write_bytes"] for v in per.values()) / len(per)
    print(json.dumps({
        "kernel": "k_moe_front", "source_sha256": source_hash(),
        "workload": "MoE layer front, 512 experts, d_model 2048, ffn 512, Q2_0, top-10, 48 distinct layers at each "
                    "batch 1, 2, 4, 8",
        "counters": "rocprofv3 --pmc FETCH_SIZE, then --pmc WRITE_SIZE (KiB a dispatch)",
        "commands": ["cd /tmp && export TMPDIR=/tmp  (R: the repository root, OUT: an output directory)",
                     "rocprofv3 --pmc FETCH_SIZE --output-format csv -d $OUT/fetch -o f -- python3 $R/bench.py "
                     "--traffic-run",
                     "rocprofv3 --pmc WRITE_SIZE --output-format csv -d $OUT/write -o w -- python3 $R/bench.py "
                     "--traffic-run",
                     "python3 $R/bench.py --traffic-summarize $OUT"],
        "calibration": {"copy_bytes": COPY_BYTES, "fetch_kib_read": cf, "write_kib_read": cw,
                        "fetch_scale": kf, "write_scale": kw},
        "per_batch": per, "traffic_bytes_per_launch": round(mean)}, indent=1))


# instruction-mix counters (two passes of at most eight SQ counters) and the kernels they are read for
COUNTER_PASSES = {  # six a pass: derived counters can take more than one of the block's eight
    "insts": ["SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_LDS", "SQ_INSTS_SALU", "SQ_WAVES", "SQ_BUSY_CYCLES"],
    "lds": ["SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_WAIT_ANY",
            "SQ_ACTIVE_INST_LDS", "SQ_CYCLES"],
}
COUNTER_KERNELS = {"prefill": "k_tile_stream", "stack_iq3s": "k_stack_mv", "stream_q2_f32": "k_stream_mv"}


def counters_run(workload):
    """The workload an instruction-mix counter run reads: the C5 prefill layer's two stream passes (prefill), the
    C2 IQ3_S stream at one token (stack_iq3s) or the C1 stream, Q2_0 with float32 vectors (stream_q2_f32), a few
    launches each."""
    import numpy as np
    import torch

    import strata_hip
    from strata_hip import blocks as SB
    from strata_hip import fused as SF
    from strata_hip import synth
    from strata_hip import tables as T

    strata_hip.load()
    T.use(T.synthetic(0))
    dev = torch.device("cuda:0")
    if workload == "prefill":
        rng = np.random.default_rng(5)
        logits = synth.zipf_logits(rng, 2048, E).to(dev)
        x = torch.from_numpy(rng.standard_normal((2048, D)).astype(np.float32)).to(torch.bfloat16).to(dev)
        gate = SB.BlockSwitchLinear(synth.random_blocks_gpu("IQ3_S", E * F, D, 11, dev), "IQ3_S", (E, F, D))
        up = SB.BlockSwitchLinear(synth.random_blocks_gpu("IQ3_S", E * F, D, 12, dev), "IQ3_S", (E, F, D))
        down = SB.BlockSwitchLinear(synth.random_blocks_gpu("IQ3_S", E * D, F, 13, dev), "IQ3_S", (E, D, F))
        idx = SF.top_k(logits, K)
        for _ in range(3):
            SB._tiled_glu(x[None], idx[None], up, gate, down)
    elif workload in ("stack_iq3s", "stream_q2_f32"):
        kind, dt = ("IQ3_S", torch.bfloat16) if workload == "stack_iq3s" else ("Q2_0", torch.float32)
        R, C = 3072, 2048
        n = -(-600_000_000 // (R * SB.row_bytes(kind, C)))
        blocks = synth.random_blocks_gpu(kind, n * R, C, 7, dev)
        x = torch.randn(n, 1, C, device=dev).to(dt)
        for _ in range(3):
            SB.stack_matvec(blocks, kind, (n, R, C), x)
    else:
        raise SystemExit(f"--counters-run: {workload} (one of {sorted(COUNTER_KERNELS)})")
    torch.cuda.synchronize()
    print(f"{workload}: done", flush=True)


def counters_summarize(d, workload):
    """Markdown: each counter's mean a dispatch of the workload's kernel over the passes' directories under d
    (d/insts, d/lds), and the ratios read from them."""
    kernel = COUNTER_KERNELS[workload]
    mean = {}
    for pas, names in COUNTER_PASSES.items():
        for name in names:
            vals = [v for _, k, v in _counters(os.path.join(d, pas), name) if kernel in k]
            if vals:
                mean[name] = sum(vals) / len(vals)
    if not mean:
        raise SystemExit(f"no {kernel} dispatches under {d}")
    lines = [f"# {kernel}: instruction mix ({workload})", "",
             "Counters a dispatch (rocprofv3 --pmc, two passes; mean over the workload's dispatches):", "",
             "| counter | a dispatch |", "| :--- | ---: |"]
    lines += [f"| {k} | {v:,.0f} |" for k, v in mean.items()]
    mfma = mean.get("SQ_INSTS_MFMA") or 0
    ratios = []
    if mfma:
        for k in ("SQ_INSTS_VALU", "SQ_INSTS_LDS", "SQ_INSTS_SALU"):
            if k in mean:
                ratios.append(f"{k} per MFMA: {mean[k] / mfma:.2f}")
    if mean.get("SQ_INSTS_LDS") and "SQ_LDS_BANK_CONFLICT" in mean:
        ratios.append(f"LDS bank-conflict cycles per LDS instruction: "
                      f"{mean['SQ_LDS_BANK_CONFLICT'] / mean['SQ_INSTS_LDS']:.3f}")
    if mean.get("SQ_BUSY_CYCLES") and "SQ_VALU_MFMA_BUSY_CYCLES" in mean:
        ratios.append(f"MFMA busy / SQ busy cycles: {mean['SQ_VALU_MFMA_BUSY_CYCLES'] / mean['SQ_BUSY_CYCLES']:.3f}")
    lines += ["", *[f"- {r}" for r in ratios], "", "Commands (cd /tmp, TMPDIR=/tmp; R the repository root):", ""]
    for pas, names in COUNTER_PASSES.items():
        lines.append(f"    timeout -s KILL 120 rocprofv3 --pmc {' '.join(names)} --output-format csv -d $OUT/{pas} "
                     f"-o {pas} -- python3 $R/bench.py --counters-run {workload}")
    lines.append(f"    python3 $R/bench.py --counters-summarize $OUT {workload}")
    print("\n".join(lines))


def build_layers(n_layers, dev, kind):
    import torch

    from strata_hip import blocks as SB
    from strata_hip import fused as SF
    from strata_hip import synth

    layers, raw = [], []
    for l in range(n_layers):
        s = 100 * (l + 1)
        g = synth.random_blocks_gpu(kind, E * F, D, s + 1, dev)
        u = synth.random_blocks_gpu(kind, E * F, D, s + 2, dev)
        d = synth.random_blocks_gpu(kind, E * D, F, s + 3, dev)
        sg = synth.random_blocks_gpu(kind, F, D, s + 4, dev)
        su = synth.random_blocks_gpu(kind, F, D, s + 5, dev)
        sd = synth.random_blocks_gpu(kind, D, F, s + 6, dev)
        gen = torch.Generator(device=dev)
        gen.manual_seed(s + 7)
        wg = (torch.randn(D, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
        lin = [SB.BlockSwitchLinear(t, kind, shape) for t, shape in
               ((g, (E, F, D)), (u, (E, F, D)), (d, (E, D, F)), (sg, (1, F, D)), (su, (1, F, D)), (sd, (1, D, F)))]
        layers.append(SF.MoEDecode(*lin, wg, K))
        raw.append((g, u, d, sg, su, sd, wg))
    return layers, raw


def matvec_stream(dev, steps, warmup):
    """C2: 3072 x 2048 matvecs straight from GGUF blocks, as streaming throughput over distinct matrices (a stack of
    more than 600 MB, past the 256 MB Infinity Cache, in one launch) and as one matrix alone, B = 1, 4, 8 bf16."""
    import torch

    from strata_hip import blocks as SB
    from strata_hip import synth

    R, C = 3072, 2048
    res = {}
    for kind in ("Q2_0", "IQ3_S"):
        mat = R * SB.row_bytes(kind, C)
        n = -(-600_000_000 // mat)
        blocks = synth.random_blocks_gpu(kind, n * R, C, 7, dev)
        res[kind] = {}
        for b in (1, 4, 8):
            x = torch.randn(n, b, C, device=dev).to(torch.bfloat16)
            one = x[:1].contiguous()
            out = {}
            for name, nm, xx in (("stream", n, x), ("single", 1, one)):
                SB.stack_matvec(blocks, kind, (nm, R, C), xx)
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    for _ in range(1 if name == "stream" else 20):
                        SB.stack_matvec(blocks, kind, (nm, R, C), xx)
                for _ in range(warmup):
                    g.replay()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(steps):
                    g.replay()
                e1.record()
                torch.cuda.synchronize()
                calls = steps * (1 if name == "stream" else 20)
                sec = e0.elapsed_time(e1) * 1e-3 / calls
                nbytes = nm * (mat + b * C * 2 + b * R * 2)
                out[name] = (sec, nbytes)
            ss, sb = out["stream"]
            us, ub = out["single"]
            res[kind][str(b)] = {"stream_GBps": round(sb / ss / 1e9, 1), "stream_frac": round(sb / ss / 1e9 / HBM_PEAK_GBS, 4),
                                 "matrices": n, "single_us": round(us * 1e6, 2), "single_GBps": round(ub / us / 1e9, 1)}
            print(f"# C2 {kind} B={b}: {res[kind][str(b)]}", file=sys.stderr, flush=True)
        del blocks
        torch.cuda.empty_cache()
    return res


def matvec_sweep(dev, steps, warmup):
    """C1 and C2's sweep, 3072 x 2048 at B = 1 over distinct matrices (a stack past the Infinity Cache): Q2_0 with
    float32 activations (x [1, 2048] float32, out float32: the exact path) and every kind with bf16 activations
    (Q2_0 and IQ3_S by the MFMA kernels, the others, and float32, by the exact-weight stream). Two forms: one matrix
    a launch (graph-captured launches: window_matvec as a layer calls it), and the whole stack in one launch
    (stack_matvec: the streaming throughput). Bytes a matrix: its blocks + x + out."""
    import torch

    from strata_hip import blocks as SB
    from strata_hip import synth

    R, C = 3072, 2048
    res = {}
    cases = [("Q2_0", torch.float32)] + [(k, torch.bfloat16) for k in sorted(SB.BLOCK)]
    for kind, dt in cases:
        mat = R * SB.row_bytes(kind, C)
        n = -(-600_000_000 // mat)
        blocks = synth.random_blocks_gpu(kind, n * R, C, 9, dev).reshape(n, -1)
        x = torch.randn(1, C, device=dev).to(dt)
        SB.window_matvec(blocks[0], kind, R, C, x)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for m in range(n):
                SB.window_matvec(blocks[m], kind, R, C, x)
        for _ in range(warmup):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        sec = e0.elapsed_time(e1) * 1e-3 / (steps * n)
        nbytes = mat + C * x.element_size() + R * x.element_size()
        key = f"{kind}_{'fp32' if dt == torch.float32 else 'bf16'}"
        res[key] = {"us": round(sec * 1e6, 2), "GBps": round(nbytes / sec / 1e9, 1),
                    "frac": round(nbytes / sec / 1e9 / HBM_PEAK_GBS, 4), "matrices": n}
        del g
        # the stack in one launch, each matrix its own vector
        xs = torch.randn(n, 1, C, device=dev).to(dt)
        SB.stack_matvec(blocks, kind, (n, R, C), xs)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            SB.stack_matvec(blocks, kind, (n, R, C), xs)
        for _ in range(warmup):
            g.replay()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        sec = e0.elapsed_time(e1) * 1e-3 / steps
        res[key].update(stream_us=round(sec * 1e6, 1), stream_GBps=round(n * nbytes / sec / 1e9, 1),
                        stream_frac=round(n * nbytes / sec / 1e9 / HBM_PEAK_GBS, 4))
        print(f"# C1/C2 sweep {key} B=1: {res[key]}", file=sys.stderr, flush=True)
        del blocks, g, xs
        torch.cuda.empty_cache()
    return res


def attention_decode(dev, steps, warmup):
    """C4: paged GQA decode attention, 16 query heads over 2 KV heads of 256, pages of 16, contexts 4K / 32K / 128K,
    B = 1, 2, 4, 8 queries causal among themselves. Each context's layers are distinct KV pools (shuffled page
    tables) totalling >= 512 MB, so the Infinity Cache holds none of them; a captured graph runs every layer once.
    Bytes a call: K and V of the context (2,048 B a position) + page table + q and out."""
    import torch

    from strata_hip import attention as SA

    Hq, Hkv, Dh = 16, 2, 256
    res = {}
    for ctx in (4096, 32768, 131072):
        n_pages = ctx // 16
        pool = ctx * 2 * Hkv * Dh * 2
        n_layers = max(2, -(-512 * 2**20 // pool))
        gen = torch.Generator(device=dev)
        gen.manual_seed(ctx)
        ks = [torch.randn(n_pages, Hkv, 16, Dh, device=dev, generator=gen).to(torch.bfloat16) for _ in range(n_layers)]
        vs = [torch.randn(n_pages, Hkv, 16, Dh, device=dev, generator=gen).to(torch.bfloat16) for _ in range(n_layers)]
        tabs = [torch.randperm(n_pages, device=dev, generator=gen).to(torch.int32) for _ in range(n_layers)]
        res[str(ctx)] = {}
        for b in (1, 2, 4, 8):
            qs = [torch.randn(b, Hq, Dh, device=dev, generator=gen).to(torch.bfloat16) for _ in range(n_layers)]
            stream = torch.cuda.Stream()
            stream.wait_stream(torch.cuda.current_stream())  # the inputs were made on the default stream
            with torch.cuda.stream(stream):
                for i in range(n_layers):
                    SA.paged_decode_attention(qs[i], ks[i], vs[i], tabs[i], ctx)
                torch.cuda.synchronize()
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=stream):
                    for i in range(n_layers):
                        SA.paged_decode_attention(qs[i], ks[i], vs[i], tabs[i], ctx)
                for _ in range(warmup):
                    graph.replay()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for _ in range(steps):
                    graph.replay()
                e1.record(stream)
                torch.cuda.synchronize()
            sec = e0.elapsed_time(e1) * 1e-3 / (steps * n_layers)
            nbytes = ctx * 2 * Hkv * Dh * 2 + n_pages * 4 + 2 * b * Hq * Dh * 2
            res[str(ctx)][str(b)] = {"us": round(sec * 1e6, 2), "GBps": round(nbytes / sec / 1e9, 1),
                                     "frac": round(nbytes / sec / 1e9 / HBM_PEAK_GBS, 4), "layers": n_layers}
            print(f"# C4 ctx={ctx} B={b}: {res[str(ctx)][str(b)]}", file=sys.stderr, flush=True)
        del ks, vs, tabs
        torch.cuda.empty_cache()
    return res


def prefill_layer(dev, steps, warmup):
    """C5: a 2048-token prompt chunk through one MoE layer's routed experts: top-10 of 512 under Zipf(1.1)
    popularity, IQ3_S experts (gate / up 512 x 2048, down 2048 x 512), pairs in tiles of 16 by tiles_of, the
    three grouped GEMMs on MFMA with the weights dequantized into LDS as bf16 (gate and up with the SwiGLU in one
    pass, down with the un-permutation in another). Timed: tiles_of + both passes, as one captured graph (the
    layer's whole prompt path after routing). MFMA use = 2 * pairs * (3 * 512 * 2048) flops / time against the
    2.5 PFLOP/s dense bf16 peak. us_one_wave_a_tile: the same with each tile multiplied by one wave
    (sh_tiles_set_share(0)), the form before short expert runs were shared."""
    import numpy as np
    import torch

    from strata_hip import blocks as SB
    from strata_hip import synth

    T_, E_, K_, D_, F_ = 2048, 512, 10, 2048, 512
    rng = np.random.default_rng(5)
    logits = synth.zipf_logits(rng, T_, E_).to(dev)
    x = torch.from_numpy(rng.standard_normal((T_, D_)).astype(np.float32)).to(torch.bfloat16).to(dev)
    gate = SB.BlockSwitchLinear(synth.random_blocks_gpu("IQ3_S", E_ * F_, D_, 11, dev), "IQ3_S", (E_, F_, D_))
    up = SB.BlockSwitchLinear(synth.random_blocks_gpu("IQ3_S", E_ * F_, D_, 12, dev), "IQ3_S", (E_, F_, D_))
    down = SB.BlockSwitchLinear(synth.random_blocks_gpu("IQ3_S", E_ * D_, F_, 13, dev), "IQ3_S", (E_, D_, F_))
    from strata_hip import fused as SF
    idx = SF.top_k(logits, K_)
    pairs = idx.numel()
    torch.cuda.synchronize()

    def layer():
        return SB._tiled_glu(x[None], idx[None], up, gate, down)

    from strata_hip import _lib

    lib = _lib.load()

    def timed(share):
        """The layer as a graph captured with the stream kernels' tile sharing on or off (read at launch)."""
        before = lib.sh_tiles_set_share(share)
        try:
            stream = torch.cuda.Stream()
            stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(stream):
                layer()
                torch.cuda.synchronize()
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=stream):
                    layer()
                for _ in range(warmup):
                    graph.replay()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for _ in range(steps):
                    graph.replay()
                e1.record(stream)
                torch.cuda.synchronize()
        finally:
            lib.sh_tiles_set_share(before)
        return e0.elapsed_time(e1) * 1e-3 / steps

    sec = timed(1)
    sec_alone = timed(0)
    flops = 2 * pairs * 3 * F_ * D_
    counts = torch.bincount(idx.reshape(-1).long(), minlength=E_)
    tiles = int(((counts + 15) // 16).sum())
    res = {"us": round(sec * 1e6, 1), "TFLOPs": round(flops / sec / 1e12, 1),
           "mfma_frac": round(flops / sec / 2.5e15, 4), "us_one_wave_a_tile": round(sec_alone * 1e6, 1),
           "pairs": pairs, "tiles": tiles,
           "top_expert_pairs": int(counts.max()), "experts_used": int((counts > 0).sum())}
    print(f"# C5 prefill: {res}", file=sys.stderr, flush=True)
    return res


_CPU = {}  # a worker's view of the sampled layers' blocks (mapped files), set by _cpu_attach


def _cpu_attach(names, kind):
    """Pool initializer: map the parent's file copies of the sampled layers' routed stacks (read-only)."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    _CPU["limits"] = threadpool_limits(limits=1)  # one BLAS thread a worker
    _CPU["kind"] = kind
    _CPU["layers"] = [[np.memmap(path, dtype=np.uint8, mode="r", shape=shape) for path, shape in layer]
                      for layer in names]


def _cpu_expert(l, e, xs):
    """One routed expert of a sampled layer for the token rows xs (n, D): its down(swiglu(gate, up)) rows, as the
    reference's CPU path computes them (the expert dequantized, float32 products, bfloat16 roundings)."""
    from oracle import blocks as OB
    from oracle import route as OR

    g, u, d = _CPU["layers"][l][:3]
    kind = _CPU["kind"]
    mg, mu, md = (OB.dequantize(m[e], kind, shape, {}) for m, shape in ((g, (F, D)), (u, (F, D)), (d, (D, F))))
    h = OR.swiglu(OR.to_bf16(xs @ mg.T), OR.to_bf16(xs @ mu.T), "bfloat16")
    return OR.to_bf16(h @ md.T)


def _expert_products(xs, mats, kind):
    from oracle import blocks as OB
    from oracle import route as OR

    mg, mu, md = (OB.dequantize(m, kind, shape, {}) for m, shape in zip(mats, ((F, D), (F, D), (D, F))))
    h = OR.swiglu(OR.to_bf16(xs @ mg.T), OR.to_bf16(xs @ mu.T), "bfloat16")
    return OR.to_bf16(h @ md.T)


def cpu_baseline(raw, inputs, kind, seconds, check_outputs, procs=1, max_layers=9):
    """The oracle's restatement of the reference's CPU path (dequantize the touched experts, numpy matmul in
    float32, the reference's routing, SwiGLU and combine roundings) on the host cores, over the first `max_layers`
    layers: in this process (procs = 1, one BLAS thread), or spread over `procs` worker processes, an expert a task
    (each worker one BLAS thread, the layers' routed stacks in files it maps). Returns GB/s of algorithmic bytes, the
    seconds spent, the layer decodes done, the layers used and the check against the GPU's outputs."""
    import multiprocessing as mp
    import shutil
    import tempfile

    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import route as OR

    n_layers = min(len(raw), max_layers)
    host, names = [], []
    tmp = None
    if procs > 1:  # in memory (/dev/shm) when it has room for them twice over, else in the temporary directory
        need = sum(raw[l][i].numel() for l in range(n_layers) for i in range(3))
        shm_ok = os.path.isdir("/dev/shm") and shutil.disk_usage("/dev/shm").free > 2 * need
        tmp = tempfile.mkdtemp(prefix="cpu_baseline_", dir="/dev/shm" if shm_ok else None)
    for l in range(n_layers):
        mats, layer_names = [], []
        for i, (t, n) in enumerate(zip(raw[l][:6], (E, E, E, 1, 1, 1))):
            a = t.cpu().numpy().reshape(n, -1)
            if tmp and n == E:  # the routed stacks, as files the workers map
                path = os.path.join(tmp, f"{l}_{i}")
                m = np.memmap(path, dtype=np.uint8, mode="w+", shape=a.shape)
                m[:] = a
                m.flush()
                layer_names.append((path, a.shape))
            mats.append(a)
        mats.append(raw[l][6].float().cpu().numpy())
        host.append(mats)
        names.append(layer_names)
    pool = None
    if procs > 1:
        pool = mp.get_context("spawn").Pool(procs, initializer=_cpu_attach, initargs=(names, kind))
        pool.starmap(_cpu_expert, [(0, 0, np.zeros((1, D), np.float32))] * procs)  # workers up before the clock

    def one_layer(l, logits, x):
        g, u, d, sg, su, sd, wg = host[l]
        idx = OR.top_k(logits, K)
        w = OR.routing_weights(logits, idx)
        B = x.shape[0]
        ys = np.zeros((B, K, D), np.float32)
        used = np.unique(idx)
        tasks = [(int(e), np.nonzero(idx == e)) for e in used]
        if pool is None:
            outs = [_expert_products(x[t], (g[e], u[e], d[e]), kind) for e, (t, _) in tasks]
        else:
            outs = pool.starmap(_cpu_expert, [(l, e, x[t]) for e, (t, _) in tasks])
        for (e, (t, j)), y in zip(tasks, outs):
            ys[t, j] = y
        s = _expert_products(x, (sg[0], su[0], sd[0]), kind)
        gate = OR.to_bf16(x @ wg)
        return OR.moe_combine(ys, w, gate, s, "bfloat16"), len(used)

    total_bytes, total_time, layers_done, checks = 0, 0.0, 0, {}
    try:
        with threadpool_limits(limits=1):
            b_list = sorted(inputs)
            l = 0
            while True:
                for b in b_list:
                    logits_t, x_t, gpu_out = inputs[b][l % len(inputs[b])]
                    logits, x = logits_t.float().cpu().numpy(), x_t.float().cpu().numpy()
                    t0 = time.perf_counter()
                    out, n_unique = one_layer(l, logits, x)
                    total_time += time.perf_counter() - t0
                    total_bytes += layer_bytes(n_unique, b)
                    layers_done += 1
                    if check_outputs and l == 0 and gpu_out is not None:
                        got = gpu_out.float().cpu().numpy()
                        checks[b] = float(np.abs(got - out).max() / max(np.abs(out).max(), 1e-30))
                l += 1
                if total_time >= seconds or l >= n_layers:
                    break
    finally:
        if pool is not None:
            pool.close()
            pool.join()
        if tmp:
            shutil.rmtree(tmp, ignore_errors=True)
    return total_bytes / total_time / 1e9, total_time, layers_done, l, checks


def moe_pass(layers, batches, args, dev, iq3s=False):
    """One decode pass through the layers at each width, timed as a captured graph; and the front kernel alone."""
    import numpy as np
    import torch

    from strata_hip import fused as SF

    kind_bytes = EXPERT_BYTES_IQ3S if iq3s else EXPERT_BYTES
    per_batch, inputs = {}, {}
    all_bytes, all_time = 0, 0.0
    gu_bytes, gu_time, gu_launches = 0, 0.0, 0
    stream = torch.cuda.Stream()
    for b in batches:
        gen = torch.Generator(device=dev)
        gen.manual_seed(1000 + b)
        logits = [torch.randn(b, E, device=dev, generator=gen).to(torch.bfloat16) for _ in layers]
        xs = [torch.randn(b, D, device=dev, generator=gen).to(torch.bfloat16) for _ in layers]
        outs = [torch.empty(b, D, device=dev, dtype=torch.bfloat16) for _ in layers]
        uniq = [int(torch.unique(SF.top_k(lg, K)).numel()) for lg in logits]
        bytes_pass = sum(layer_bytes(u, b, kind_bytes) for u in uniq)
        stream.wait_stream(torch.cuda.current_stream())  # the inputs were made on the default stream
        with torch.cuda.stream(stream):
            for m, lg, x, o in zip(layers, logits, xs, outs):  # first calls allocate the workspaces
                m(lg, x, out=o)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for m, lg, x, o in zip(layers, logits, xs, outs):
                    m(lg, x, out=o)
            # the dominant kernel alone: a graph of the front launches only (route, gate and up; the MoE path's
            # phases 0 and 1 are both this kernel for this shape)
            gu_graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gu_graph, stream=stream):
                for m, lg, x, o in zip(layers, logits, xs, outs):
                    m(lg, x, phase=1)
            for _ in range(args.warmup):
                graph.replay()
                gu_graph.replay()
            torch.cuda.synchronize()
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
            marks = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]  # each pass's end
            ev[0].record(stream)
            for i in range(args.steps):
                graph.replay()
                marks[i].record(stream)
            ev[1].record(stream)
            ev[2].record(stream)
            for _ in range(args.steps):
                gu_graph.replay()
            ev[3].record(stream)
            torch.cuda.synchronize()
            # the windows the down kernel combines itself (2-4 tokens, after a release / acquire hand-off between
            # its blocks) also timed with the combine as a kernel of its own after the tail: the two forms' costs
            sep_ms = None
            if 2 <= b <= 4:
                from strata_hip import _lib

                lib = _lib.load()
                before = lib.sh_moe_set_tail_combine(0)
                try:
                    sep_graph = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(sep_graph, stream=stream):
                        for m, lg, x, o in zip(layers, logits, xs, outs):
                            m(lg, x, out=o)
                finally:
                    lib.sh_moe_set_tail_combine(before)
                for _ in range(args.warmup):
                    sep_graph.replay()
                torch.cuda.synchronize()
                es = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
                es[0].record(stream)
                for _ in range(args.steps):
                    sep_graph.replay()
                es[1].record(stream)
                torch.cuda.synchronize()
                sep_ms = es[0].elapsed_time(es[1])
                del sep_graph
            # leave the outputs of a full pass behind (the front's graph rewrote h, not the outputs)
            graph.replay()
            torch.cuda.synchronize()
        ms = ev[0].elapsed_time(ev[1])
        gu_ms = ev[2].elapsed_time(ev[3])
        n_layers = args.steps * len(layers)
        passes = np.array([(ev[0] if i == 0 else marks[i - 1]).elapsed_time(marks[i]) for i in range(args.steps)])
        per_batch[b] = {"us_per_layer": round(ms * 1e3 / n_layers, 3),
                        "us_per_layer_median": round(float(np.median(passes)) * 1e3 / len(layers), 3),
                        "us_per_layer_p10": round(float(np.percentile(passes, 10)) * 1e3 / len(layers), 3),
                        "GBps": round(bytes_pass * args.steps / (ms * 1e-3) / 1e9, 1),
                        "unique_experts_mean": round(float(np.mean(uniq)), 2),
                        "tok_per_s": round(b * args.steps / (ms * 1e-3), 1),
                        "front_us": round(gu_ms * 1e3 / n_layers, 3)}
        if sep_ms is not None:
            per_batch[b]["us_per_layer_combine_kernel"] = round(sep_ms * 1e3 / n_layers, 3)
        all_bytes += bytes_pass * args.steps
        all_time += ms * 1e-3
        gu_bytes += sum(front_bytes(u, b, kind_bytes) for u in uniq) * args.steps
        gu_time += gu_ms * 1e-3
        gu_launches += n_layers
        inputs[b] = list(zip(logits, xs, outs))
        print(f"# {'IQ3_S' if iq3s else 'Q2_0'} B={b}: {per_batch[b]}", file=sys.stderr, flush=True)

    return per_batch, inputs, all_bytes, all_time, gu_bytes, gu_time, gu_launches


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--batches", default="1,2,4,8")
    ap.add_argument("--kind", default="Q2_0")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--no-matvec", action="store_true")
    ap.add_argument("--no-attention", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-iq3s", action="store_true")
    ap.add_argument("--traffic-run", action="store_true", help="the counter runs' workload (under rocprofv3)")
    ap.add_argument("--traffic-summarize", metavar="DIR", help="the counter summary of two runs' output directory")
    ap.add_argument("--counters-run", metavar="WORKLOAD", help="an instruction-mix counter run's workload "
                    "(prefill, stack_iq3s, stream_q2_f32; under rocprofv3)")
    ap.add_argument("--counters-summarize", nargs=2, metavar=("DIR", "WORKLOAD"),
                    help="the instruction-mix summary of the two passes' output directory")
    args = ap.parse_args()
    if args.traffic_run:
        return traffic_run()
    if args.traffic_summarize:
        return traffic_summarize(args.traffic_summarize)
    if args.counters_run:
        return counters_run(args.counters_run)
    if args.counters_summarize:
        return counters_summarize(*args.counters_summarize)
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus}: this path runs and is measured on one GPU (expert parallelism across "
              f"GPUs is not implemented); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import strata_hip
    from strata_hip import fused as SF
    from strata_hip import tables as T

    strata_hip.load()
    T.use(T.synthetic(0))
    dev = torch.device("cuda:0")
    batches = [int(b) for b in args.batches.split(",")]
    t_setup = time.perf_counter()
    layers, raw = build_layers(args.layers, dev, args.kind)
    torch.cuda.synchronize()
    print(f"# {args.layers} layers of {args.kind} experts on the GPU in {time.perf_counter() - t_setup:.1f} s",
          file=sys.stderr, flush=True)

    per_batch, inputs, all_bytes, all_time, gu_bytes, gu_time, gu_launches = moe_pass(layers, batches, args, dev)
    iq3s = None
    if not args.no_iq3s:  # the metric's second kind: the same pass over IQ3_S experts (not part of `value`)
        del layers
        torch.cuda.empty_cache()
        layers_iq, _ = build_layers(args.layers, dev, "IQ3_S")
        iq3s, _, b_iq, t_iq, *_ = moe_pass(layers_iq, batches, args, dev, iq3s=True)
        iq3s = {"per_batch": {str(k): v for k, v in iq3s.items()}, "GBps": round(b_iq / t_iq / 1e9, 1)}
        del layers_iq
        torch.cuda.empty_cache()

    matvec = None if args.no_matvec else matvec_stream(dev, max(3, args.steps // 4), args.warmup)
    sweep = None if args.no_matvec else matvec_sweep(dev, max(3, args.steps // 4), args.warmup)
    attention = None if args.no_attention else attention_decode(dev, max(3, args.steps // 4), args.warmup)
    prefill = None if args.no_prefill else prefill_layer(dev, max(3, args.steps // 4), args.warmup)
    value = all_bytes / all_time / 1e9
    achieved = gu_bytes / gu_time / 1e9
    traffic = front_traffic()
    cpu = cpu1 = None
    if not args.no_cpu:
        cores = len(os.sched_getaffinity(0))
        legs = {}
        for threads in (1, cores):
            gbs, secs, n_done, n_layers_used, checks = cpu_baseline(raw, inputs, args.kind, args.cpu_seconds,
                                                                    threads == 1, threads)
            how = ("one process" if threads == 1 else
                   f"{threads} worker processes, an expert a task, the blocks in mapped files")
            legs[threads] = {"value": round(gbs, 4), "unit": "GB/s", "cores": threads, "kind": "port",
                             "sample": f"{n_done} layer decodes (layers 0..{n_layers_used - 1} at B = {args.batches}), "
                                       f"{secs:.1f} s: numpy dequantize of the touched experts + float32 matmul, "
                                       f"{how}, one BLAS thread each"}
            if checks:
                legs[threads]["check_vs_gpu_rel_err"] = {str(k): round(v, 6) for k, v in checks.items()}
            print(f"# CPU {threads} thread(s): {legs[threads]}", file=sys.stderr, flush=True)
        cpu, cpu1 = legs[cores], legs[1]
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(all_time * 1e3 / args.steps, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "moe_layer_decode", "kind": args.kind, "d_model": D, "experts": E, "shared_experts": 1,
                   "d_ff": F, "top_k": K, "batches": batches, "layers_per_pass": args.layers,
                   "step": "one decode pass through the layers at each batch width"},
        "per_batch": {str(k): v for k, v in per_batch.items()},
        "matvec_3072x2048": matvec,
        "matvec_3072x2048_one_a_launch": sweep,
        "paged_attention": attention,
        "prefill_layer": prefill,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": "k_moe_front",
                     "bytes_per_launch": round(gu_bytes / gu_launches), "launches": gu_launches,
                     "us_per_launch": round(gu_time * 1e6 / gu_launches, 3)},
        "cpu_baseline": cpu,
        "cpu_baseline_1thread": cpu1,
        "moe_iq3s": iq3s,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
