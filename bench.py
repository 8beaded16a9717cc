#!/usr/bin/env python3
"""Routed-MoE-layer throughput on one MI355X.

    python bench.py [--steps K] [--warmup W] [--tokens 512] [--decode-tokens 1]

A step is one pass of the Mixtral-8x7B-shape routed layer (hidden 4096, 8
SwiGLU experts of 14336, Q4_0, softmax top-2 renormalised) over one batch of
synthetic tokens already resident in HBM.  The headline `value` is tokens/s
at T=512 (prefill); the same line carries the T=1 decode figures under
`decode`.  Weights are uploaded as several distinct copies (like consecutive
layers of a model) and the steps cycle through them, so decode steps read
their experts from HBM rather than from the 256 MB last-level cache.

`roofline` is for the dominant kernel of the step (the expert gate/up
kernel): algorithmic flops (prefill) or bytes (decode) per launch divided by
its average duration, timed with HIP events recorded around it on its stream
inside the library.  `cpu_baseline` times the CPU restatement of the
reference's MoE path (oracle/, OpenMP over the host's cores) on a bounded
sample of the same workload.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

METRIC = "MoE-layer tokens/s at T=1 and T=512; % of HBM (decode) / MFMA (prefill) peak"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0


def log(msg: str) -> None:
    print(f"# {msg}", file=sys.stderr, flush=True)


def expert_flops(shape, t: int, k: int, up_only: bool = False) -> float:
    """2*T*k*(2*H*I) for gate+up; + 2*T*k*H*I for down; plus the shared expert."""
    H, I = shape.hidden, shape.inter
    mats = 2 if up_only else 3
    f = 2.0 * t * k * mats * H * I
    if shape.shared_inter:
        f += 2.0 * t * mats * H * shape.shared_inter
    return f


def time_steps(layers, x, out, steps: int, warmup: int):
    """(median, mean) milliseconds per step: every step between an event
    pair of its own on the stream the forward runs on (torch's current
    stream), the K steps queued back to back between two synchronisations."""
    import torch

    for i in range(warmup):
        layers[i % len(layers)].feed_forward(x, out)
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for i in range(steps):
        ev[i][0].record()
        layers[i % len(layers)].feed_forward(x, out)
        ev[i][1].record()
    torch.cuda.synchronize()
    ms = [a.elapsed_time(b) for a, b in ev]
    return float(np.median(ms)), float(np.mean(ms))


def stage_times(layers, x, out, steps: int):
    """Average milliseconds per launch of each stage, from HIP events the
    library records around every stage on the forward's stream."""
    import torch

    from moe_amd import _lib as L

    for layer in layers:
        L.check(L.lib().moe_layer_profile(layer.handle, 1))
    for i in range(steps):
        layers[i % len(layers)].feed_forward(x, out)
    torch.cuda.synchronize()
    ns = len(L.STAGES)
    ms = (C.c_double * ns)()
    n = (C.c_uint64 * ns)()
    for layer in layers:
        L.check(L.lib().moe_layer_stage_times(layer.handle, ms, n))
        L.check(L.lib().moe_layer_profile(layer.handle, 0))
    # Per step: a stage launched twice per forward (the activation encoding
    # runs before gate/up and before down) counts both launches.
    return {L.STAGES[i]: (ms[i] / steps if n[i] else 0.0) for i in range(ns)}


def selected_bytes(layer, host, x) -> tuple[int, int]:
    """(gate+up bytes, down bytes) of the distinct experts this input selects."""
    import torch

    from moe_amd.layer import State

    st = State(1)
    out = torch.empty_like(x)
    layer.feed_forward(x, out, state=st)
    hits = st.previous(0)
    s = host.shape
    from moe_amd.layer import row_bytes

    up = len(hits) * 2 * s.inter * row_bytes(s.expert_dt, s.hidden)
    down = len(hits) * s.hidden * row_bytes(s.expert_dt, s.inter)
    return up, down


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(host, t_decode: int, t_prefill: int, runs: int = 5):
    """The CPU restatement of the reference path on this host's cores: per
    T, one warm-up forward (it also pages in the weights), then the median
    of `runs` timed forwards (SURVEY's protocol for the CPU baseline)."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from moe_amd import synth
    from oracle import pyoracle

    pyoracle.build()
    ol = pyoracle.from_host_layer(host)
    cores = int(pyoracle.lib().orc_max_threads())
    res = {}
    for t in (t_decode, t_prefill):
        x = synth.activations(1, t, host.shape.hidden)
        ol.forward(x)
        times = []
        for _ in range(runs):
            t0 = time.perf_counter()
            ol.forward(x)
            times.append(time.perf_counter() - t0)
        res[t] = t / float(np.median(times))
    return res[t_decode], res[t_prefill], cores


def hbm_ceiling(mib: int) -> int:
    """The HBM read rate of a plain streaming kernel (moe_debug_stream_read)
    over `mib` MiB, with plain and with nontemporal loads, at 1, 2, 4 and 8
    blocks per CU: the ceilings the weight-streaming kernels are compared
    with beside the 8 TB/s datasheet peak."""
    import ctypes as C

    import torch

    from moe_amd import _lib as L

    dev = torch.device("cuda:0")
    buf = torch.ones(mib << 20, dtype=torch.uint8, device=dev)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    stream = torch.cuda.current_stream().cuda_stream
    rows = []
    for nt in (0, 1):
        for per_cu in (1, 2, 4, 8):
            blocks = cus * per_cu
            out = torch.empty(blocks, dtype=torch.int32, device=dev)

            def go():
                L.diag_check(L.diag().moe_debug_stream_read(C.c_void_p(buf.data_ptr()), buf.numel(),
                                                      C.c_void_p(out.data_ptr()), blocks, nt, C.c_void_p(stream)),
                        "moe_debug_stream_read")

            for _ in range(3):
                go()
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            n = 10
            t0.record()
            for _ in range(n):
                go()
            t1.record()
            torch.cuda.synchronize()
            ms = t0.elapsed_time(t1) / n
            rows.append(dict(nontemporal=nt, blocks_per_cu=per_cu, ms=round(ms, 4),
                             gb_s=round(buf.numel() / (ms * 1e-3) / 1e9, 1)))
    best = {nt: max(r["gb_s"] for r in rows if r["nontemporal"] == nt) for nt in (0, 1)}
    print(json.dumps(dict(hbm_read_ceiling_gb_s=best[0], hbm_read_ceiling_nontemporal_gb_s=best[1],
                          bytes=buf.numel(), frac_of_8tb=round(best[0] / HBM_PEAK_GBS, 4),
                          frac_of_8tb_nontemporal=round(best[1] / HBM_PEAK_GBS, 4), runs=rows)), flush=True)
    return 0


def grid_barrier_cost() -> int:
    """The cost of a grid-wide barrier (moe_debug_grid_barrier): cooperative
    launches of one block per CU and of two, with 1 and with 101 barriers
    each; per barrier = the difference / 100.  Beside them, an ordinary
    launch of a small kernel on the same stream for the launch cost."""
    import ctypes as C

    import torch

    from moe_amd import _lib as L

    dev = torch.device("cuda:0")
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    state = torch.zeros(4, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream

    def per_launch(fn, reps=20):
        for _ in range(3):
            fn()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(reps):
            fn()
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / reps * 1e3

    rows = []
    for blocks in (cus, 2 * cus):
        us = {}
        for nb in (1, 101):
            us[nb] = per_launch(lambda: L.diag_check(L.diag().moe_debug_grid_barrier(
                blocks, nb, C.c_void_p(state.data_ptr()), C.c_void_p(stream)), "moe_debug_grid_barrier"))
        rows.append(dict(blocks=blocks, us_1_barrier=round(us[1], 2), us_101_barriers=round(us[101], 2),
                         us_per_barrier=round((us[101] - us[1]) / 100, 2)))
    x = torch.ones(1 << 16, dtype=torch.float32, device=dev)
    plain = per_launch(lambda: x.add_(0.0), reps=200)
    err = int(state[2].item())
    print(json.dumps(dict(grid_barrier=rows, plain_launch_us=round(plain, 2), bound_hit=err)), flush=True)
    return 0 if err == 0 else 1


def mfma_valu_issue() -> int:
    """The issue rate of the two-pass MFMA kernels' instruction mix
    (moe_debug_mfma_valu): one block per CU, one or two waves per SIMD, each
    wave iterating 8 MFMAs (V_MFMA_F32_32X32X16_F16), 56 or 32 f32 fmas, or
    both, the fmas after the MFMAs or spread between them.  Reported: ns per
    iteration of one wave."""
    import ctypes as C

    import torch

    from moe_amd import _lib as L

    dev = torch.device("cuda:0")
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    out = torch.empty(cus * 512, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    iters = 20000
    rows = []
    for waves in (1, 2):
        for mf, va, mix in ((8, 0, 0), (0, 56, 0), (8, 56, 0), (8, 56, 1), (8, 32, 1)):
            def go(n):
                L.diag_check(L.diag().moe_debug_mfma_valu(mf, va, mix, waves, cus, n, C.c_void_p(out.data_ptr()),
                                                    C.c_void_p(stream)), "moe_debug_mfma_valu")
            go(10)
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0.record()
            go(iters)
            t1.record()
            torch.cuda.synchronize()
            ns = t0.elapsed_time(t1) * 1e6 / iters
            rows.append(dict(waves_per_simd=waves, mfmas=mf, fmas=va, interleaved=bool(mix),
                             ns_per_iteration=round(ns, 2)))
    print(json.dumps(dict(mfma_valu_issue=rows, iterations=iters, blocks=cus)), flush=True)
    return 0


def copy_calibration(mib: int) -> int:
    """Five device-to-device copies of `mib` MiB: each reads and writes exactly
    mib * 1024 KiB, so a counter run over them gives the factor between the
    counters' KiB and algorithmic bytes."""
    import torch

    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_kib_per_copy": mib * 1024, "copies": 5}), flush=True)
    return 0


DT_NAMES = {0: "F32", 2: "Q4_0", 6: "Q5_0", 8: "Q8_0"}
TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "mixtral_layer_traffic.json")


def summarize_pmc(fetch_dir: str, write_dir: str, out_json: str) -> int:
    """Turn two rocprofv3 counter passes (FETCH_SIZE, WRITE_SIZE; each
    directory holding bench_counter_collection.csv from this bench and
    copy_counter_collection.csv from --copy-calibration) into HBM bytes per
    launch for every kernel, scaled by what each counter reads for the
    copy: a copy of C KiB should fetch and write C KiB each."""
    import csv
    import re

    def per_kernel(path):
        acc = {}
        for r in csv.DictReader(open(path)):
            m = re.search(r"::(\w+_kernel(<[^>]*>)?)", r["Kernel_Name"])
            name = m.group(1) if m else r["Kernel_Name"][:60]
            acc.setdefault((name, int(r["Grid_Size"])), []).append(float(r["Counter_Value"]))
        return {k: sum(v) / len(v) for k, v in acc.items()}

    def copy_factor(path, mib):
        vals = [float(r["Counter_Value"]) for r in csv.DictReader(open(path)) if "copyBuffer" in r["Kernel_Name"]]
        return (mib * 1024.0) / (sum(vals) / len(vals))

    mib = 512
    ff = copy_factor(os.path.join(fetch_dir, "copy_counter_collection.csv"), mib)
    wf = copy_factor(os.path.join(write_dir, "copy_counter_collection.csv"), mib)
    fetch = per_kernel(os.path.join(fetch_dir, "bench_counter_collection.csv"))
    write = per_kernel(os.path.join(write_dir, "bench_counter_collection.csv"))
    kernels = []
    for (name, grid), fk in sorted(fetch.items()):
        wk = write.get((name, grid), 0.0)
        kernels.append(dict(kernel=name, grid=grid, fetch_kib=round(fk, 1), write_kib=round(wk, 1),
                            hbm_bytes=round((fk * ff + wk * wf) * 1024)))
    doc = dict(source="rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE, over `bench.py --no-cpu --steps 3 --warmup 1` "
                      f"and `bench.py --copy-calibration {mib}`",
               fetch_factor=round(ff, 4), write_factor=round(wf, 4), kernels=kernels)
    with open(out_json, "w") as f:
        json.dump(doc, f, indent=1)
    print(json.dumps(dict(written=out_json, fetch_factor=ff, write_factor=wf, kernels=len(kernels))))
    return 0


def summarize_trace(trace_dir: str, out_md: str, title: str, command: str) -> int:
    """Turn a rocprofv3 kernel trace (bench_kernel_trace.csv) into a markdown
    table of per-kernel durations, one row per (kernel, grid size): the
    grid size tells the bench phases (T=1, T=32, T=512) apart."""
    import csv
    import re

    acc = {}
    for r in csv.DictReader(open(os.path.join(trace_dir, "bench_kernel_trace.csv"))):
        m = re.search(r"::(\w+_kernel(<[^>]*>)?)", r["Kernel_Name"])
        name = m.group(1) if m else r["Kernel_Name"][:48]
        grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
        dur = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        acc.setdefault((name, grid), []).append(dur)
    total = sum(sum(v) for v in acc.values())
    lines = [f"# {title}", "", "Kernel trace (from the repo root on the GPU box):", "", "    " + command, "",
             "Rows are split by grid size (threads), which tells the bench phases apart; durations in µs.", "",
             "| kernel | grid | calls | avg | median | min | max | share |", "|---|---|---|---|---|---|---|---|"]
    for (name, grid), v in sorted(acc.items(), key=lambda kv: -sum(kv[1])):
        if sum(v) < 0.001 * total:
            continue
        v = sorted(v)
        lines.append(f"| `{name}` | {grid} | {len(v)} | {sum(v) / len(v):.2f} | {v[len(v) // 2]:.2f} | {v[0]:.2f} | "
                     f"{v[-1]:.2f} | {sum(v) / total:.1%} |")
    with open(out_md, "w") as f:
        f.write("\n".join(lines) + "\n")
    print(json.dumps(dict(written=out_md, kernels=len(acc))))
    return 0


COUNTER_PASSES = [
    "GRBM_GUI_ACTIVE SQ_BUSY_CYCLES SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_MFMA SQ_WAVE_CYCLES SQ_WAIT_INST_ANY "
    "SQ_INSTS_VALU SQ_INSTS_LDS",
    "SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_LDS SQ_ACTIVE_INST_ANY SQ_WAIT_ANY SQ_INST_CYCLES_SALU SQ_INSTS_SALU "
    "SQ_WAVES SQ_LDS_BANK_CONFLICT",
]
COUNTER_BENCHES = {
    "mixtral": ("Mixtral shape, Q4_0, T=512",
                "bench.py --no-cpu --steps 3 --warmup 1 --tokens 512 --batch-tokens 0 --copies 2"),
    "qwen3": ("Qwen3-30B-A3B shape, Q8_0, T=2048",
              "bench.py --no-cpu --steps 3 --warmup 1 --shape qwen3 --tokens 2048 --batch-tokens 0 --copies 2"),
}
COUNTER_BENCH = COUNTER_BENCHES["mixtral"][1]


def summarize_counters(dirs: list, out_md: str, shape: str = "mixtral") -> int:
    """The MFMA kernels' counters from rocprofv3 --pmc passes over
    COUNTER_BENCHES[shape] (one directory per COUNTER_PASSES entry, each
    holding bench_counter_collection.csv and bench_kernel_trace.csv): clock,
    MFMA-busy share and instruction mix per launch of the gate/up and down
    kernels of the largest grid."""
    import csv
    import re

    agg, dur, grids = {}, {}, {}
    for d in dirs:
        for r in csv.DictReader(open(os.path.join(d, "bench_counter_collection.csv"))):
            m = re.search(r"::(\w+_kernel(<[^>]*>)?)", r["Kernel_Name"])
            if not m or not m.group(1).startswith("mfma_kernel"):
                continue
            key = (m.group(1), int(r["Grid_Size"]))
            agg.setdefault(key, {}).setdefault(r["Counter_Name"], {})[r["Dispatch_Id"]] = float(r["Counter_Value"])
        for r in csv.DictReader(open(os.path.join(d, "bench_kernel_trace.csv"))):
            m = re.search(r"::(\w+_kernel(<[^>]*>)?)", r["Kernel_Name"])
            if not m or not m.group(1).startswith("mfma_kernel"):
                continue
            grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
            dur.setdefault((m.group(1), grid), []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    rows = []
    for name in sorted({k[0] for k in agg}):
        key = max((k for k in agg if k[0] == name), key=lambda k: k[1])
        c = {n: sum(v.values()) / len(v) for n, v in agg[key].items()}
        ds = dur.get(key) or [float("nan")]
        rows.append((key, c, sum(ds) / len(ds)))
    simds = 1024
    title, cmd = COUNTER_BENCHES[shape]
    tag = "mfma_pmc" if shape == "mixtral" else f"{shape}_pmc"
    lines = [f"# MFMA expert kernels ({title}): clock, MFMA busy, instruction mix", "",
             "Counter passes (from the repo root on the GPU box; at most 8 SQ counters per pass):", ""]
    for i, p in enumerate(COUNTER_PASSES):
        lines.append(f"    cd /tmp && export TMPDIR=/tmp && rocprofv3 --kernel-trace --pmc {p} --output-format csv "
                     f"-d $REPO/gpurun_out/{tag}{i + 1} -o bench -- python3 $REPO/{cmd}")
    opt = "" if shape == "mixtral" else f" --counter-shape {shape}"
    lines += ["", f"then `python bench.py --summarize-counters gpurun_out/{tag}1 gpurun_out/{tag}2 OUT{opt}`.",
              "Counters are summed over the device per dispatch and averaged over dispatches; GRBM_GUI_ACTIVE "
              "sums the 8 XCDs, SQ_VALU_MFMA_BUSY_CYCLES the 1024 SIMDs.  Launches under counter collection are "
              "serialised, so durations run a little long; the ratios are what the text uses.", "",
              "| kernel | grid | duration µs | clock GHz | MFMA insts | busy cycles / MFMA | MFMA busy % of cycles "
              "| VALU per MFMA | LDS insts | SALU insts | LDS bank conflicts |",
              "|---|---|---|---|---|---|---|---|---|---|---|"]
    for (name, grid), c, d in rows:
        cyc = c.get("GRBM_GUI_ACTIVE", 0.0) / 8
        mf, bz = c.get("SQ_INSTS_MFMA", 0.0), c.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0)
        lines.append(f"| `{name}` | {grid} | {d:.1f} | {cyc / d / 1e3:.2f} | {mf:.3g} | {bz / mf if mf else 0:.1f} | "
                     f"{100 * bz / simds / cyc if cyc else 0:.1f} | "
                     f"{(c.get('SQ_INSTS_VALU', 0.0) - mf) / mf if mf else 0:.2f} | {c.get('SQ_INSTS_LDS', 0):.3g} | "
                     f"{c.get('SQ_INSTS_SALU', 0):.3g} | {c.get('SQ_LDS_BANK_CONFLICT', 0):.3g} |")
    with open(out_md, "w") as f:
        f.write("\n".join(lines) + "\n")
    print(json.dumps(dict(written=out_md, kernels=len(rows))))
    return 0


def traffic_of(kernel_prefix: str):
    """HBM bytes per launch of the kernel whose name starts with
    kernel_prefix, from the committed counter summary (None if absent).  The
    bench launches some kernels at two sizes (T=32 and T=512); the launch
    with the largest grid is the one the headline roofline describes."""
    try:
        doc = json.load(open(TRAFFIC_FILE))
    except (OSError, ValueError):
        return None
    hits = [k for k in doc["kernels"] if k["kernel"].startswith(kernel_prefix)]
    return max(hits, key=lambda k: k.get("grid", 0))["hbm_bytes"] if hits else None


def zipf_histogram_md(out_path: str, tokens: int) -> int:
    """Write the DeepSeek-V3 Zipf workload's achieved selection histogram
    (synth.zipf_histogram at the bench's inputs) beside its Zipf targets."""
    from moe_amd import synth

    shape = synth.SHAPES["deepseek_v3_zipf"]
    h = synth.zipf_histogram(shape, 1, tokens)
    c, tg = h["counts"], h["target"]
    total = int(c.sum())
    cap = 0.45 * tokens
    lines = [
        f"# DeepSeek-V3 Zipf workload: achieved expert histogram at T={tokens}",
        "",
        f"Shape `deepseek_v3_zipf` (hidden {shape.hidden}, {shape.n_experts} experts of {shape.inter}, top-"
        f"{shape.top_k}, sigmoid scores + correction bias, {shape.n_group} groups / top-{shape.topk_group}), "
        f"layer seed 1, inputs `activations(1, {tokens}, {shape.hidden})` (the bench's).  Selections per expert "
        "under the layer's routing rule, sorted, against `zipf_targets` (Zipf s = "
        f"{shape.zipf} over the {shape.n_experts} ranks, total T·k = {total}, no rank above the 0.45·T = "
        f"{cap:.0f} cap).  Counted on the host in float64 with the calibration's own rule "
        "(`synth.zipf_histogram`); the GPU parity run of the same workload routes its top expert to the same "
        "count.",
        "",
        "Command (from the repo root; CPU only):",
        "",
        f"    python bench.py --zipf-histogram profiles/deepseek_v3_zipf_histogram.md --tokens {tokens}",
        "",
        f"* experts hit: {h['hit']} of {shape.n_experts}",
        f"* top expert: {int(c[0])} tokens ({c[0] / tokens:.1%} of T; target {tg[0]:.0f})",
        f"* L1 distance to the targets: {np.abs(c - tg).sum():.0f} selections ({np.abs(c - tg).sum() / total:.1%} of "
        "T·k)",
        f"* selections held by the top 8 / top 32 experts: {c[:8].sum() / total:.1%} / {c[:32].sum() / total:.1%} "
        f"(targets {tg[:8].sum() / total:.1%} / {tg[:32].sum() / total:.1%})",
        "",
        "| rank | achieved | target |",
        "|---|---|---|",
    ]
    ranks = list(range(1, 17)) + [24, 32, 48, 64, 96, 128, 153, 154, 192, 256]
    for r in ranks:
        if r <= len(c):
            lines.append(f"| {r} | {int(c[r - 1])} | {tg[r - 1]:.1f} |")
    bands = [(17, 32), (33, 64), (65, 128), (129, 256)]
    lines += ["", "| ranks | achieved (sum) | target (sum) |", "|---|---|---|"]
    for a, b in bands:
        lines.append(f"| {a}–{b} | {int(c[a - 1:b].sum())} | {tg[a - 1:b].sum():.0f} |")
    with open(out_path, "w") as f:
        f.write("\n".join(lines) + "\n")
    print(json.dumps(dict(zipf_histogram=out_path, hit=h["hit"], top=int(c[0]),
                          l1=round(float(np.abs(c - tg).sum()), 1))), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--shape", default="mixtral")
    ap.add_argument("--tokens", type=int, default=512)
    ap.add_argument("--decode-tokens", type=int, default=1)
    ap.add_argument("--batch-tokens", type=int, default=32,
                    help="a few-tokens batch also measured (BASELINE's HBM-bound T=32 row); 0 to skip")
    ap.add_argument("--copies", type=int, default=4, help="distinct weight copies cycled through")
    ap.add_argument("--cpu-runs", type=int, default=5, help="timed CPU forwards per T (median)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--mode", type=int, default=0, help="kernel path (moe_layer_set_mode): 0 automatic")
    ap.add_argument("--no-tiled", action="store_true",
                    help="do not keep the tiled expert copies (moe_layer_set_tiled) that few-tokens calls stream")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="write the HBM traffic summary from two rocprofv3 counter passes and exit")
    ap.add_argument("--summarize-trace", nargs=2, metavar=("TRACE_DIR", "OUT_MD"),
                    help="write a markdown table of kernel durations from a rocprofv3 kernel trace and exit")
    ap.add_argument("--summarize-counters", nargs="+", metavar="DIR",
                    help="write the MFMA kernels' counter summary from the rocprofv3 passes of COUNTER_PASSES "
                         "(directories, then the output markdown path) and exit")
    ap.add_argument("--counter-shape", choices=sorted(COUNTER_BENCHES), default="mixtral",
                    help="workload whose counter passes --summarize-counters reads")
    ap.add_argument("--grid-barrier", action="store_true",
                    help="time grid-wide barriers in cooperative launches and exit")
    ap.add_argument("--mfma-valu", action="store_true",
                    help="time MFMA and VALU issue alone and together (moe_debug_mfma_valu) and exit")
    ap.add_argument("--hbm-ceiling", type=int, default=0, metavar="MIB",
                    help="only time a plain streaming read of MIB MiB (moe_debug_stream_read) and exit")
    ap.add_argument("--zipf-histogram", metavar="OUT_MD",
                    help="write the DeepSeek-V3 Zipf workload's achieved expert histogram at --tokens (CPU) and exit")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only copy MIB MiB device-to-device 5 times (a plain copy kernel of known size, the "
                         "reference point for the FETCH_SIZE / WRITE_SIZE counters) and exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (every GPU box here has one GPU); "
              "run with --gpus 1", file=sys.stderr)
        return 2
    if args.zipf_histogram:
        return zipf_histogram_md(args.zipf_histogram, args.tokens)
    if args.copy_calibration:
        return copy_calibration(args.copy_calibration)
    if args.hbm_ceiling:
        return hbm_ceiling(args.hbm_ceiling)
    if args.grid_barrier:
        return grid_barrier_cost()
    if args.mfma_valu:
        return mfma_valu_issue()
    if args.summarize_pmc:
        return summarize_pmc(args.summarize_pmc[0], args.summarize_pmc[1], TRAFFIC_FILE)
    if args.summarize_counters:
        return summarize_counters(args.summarize_counters[:-1], args.summarize_counters[-1], args.counter_shape)
    if args.summarize_trace:
        return summarize_trace(args.summarize_trace[0], args.summarize_trace[1],
                               "Mixtral-8x7B-shape routed layer (Q4_0, top-2), T=1, T=32 and T=512: kernel durations",
                               "cd /tmp && export TMPDIR=/tmp && rocprofv3 --kernel-trace --stats --output-format csv "
                               "-d $REPO/gpurun_out/prof -o bench -- python3 $REPO/bench.py --no-cpu --steps 20")

    import torch

    from moe_amd import synth
    from moe_amd.layer import Context

    shape = synth.SHAPES[args.shape]
    log(f"generating {shape.name} layer (seed 1)")
    t0 = time.time()
    host = synth.build_host_layer(shape, 1)
    log(f"generated {host.buf.nbytes / 1e6:.0f} MB in {time.time() - t0:.1f}s; uploading {args.copies} copies")
    ctx = Context(0)
    layers = [synth.make_layer(ctx, host, layer_index=0) for _ in range(args.copies)]
    if args.mode:
        for layer in layers:
            layer.set_mode(args.mode)
    if not args.no_tiled:
        for layer in layers:
            layer.set_tiled(True)
    dev = torch.device("cuda:0")
    k = layers[0].k

    results = {}
    for t in [args.decode_tokens] + ([args.batch_tokens] if args.batch_tokens else []) + [args.tokens]:
        for layer in layers:
            layer.reserve(t)
        x = torch.from_numpy(synth.activations(1, t, shape.hidden)).to(dev)
        out = torch.empty_like(x)
        ms, ms_mean = time_steps(layers, x, out, args.steps, args.warmup)
        stages = stage_times(layers, x, out, args.steps)
        up_bytes, down_bytes = selected_bytes(layers[0], host, x)
        results[t] = dict(ms=ms, ms_mean=ms_mean, stages=stages, up_bytes=up_bytes, down_bytes=down_bytes)
        log(f"T={t}: {ms:.4f} ms/step (median; mean {ms_mean:.4f}), {t / ms * 1e3:.0f} tok/s; stages " +
            ", ".join(f"{k_}={v * 1e3:.1f}us" for k_, v in stages.items()))

    # Prefill (headline): MFMA-bound gate/up kernel.
    tp = results[args.tokens]
    up_ms = tp["stages"]["expert_up"]
    up_flops = expert_flops(shape, args.tokens, k, up_only=True)
    achieved = up_flops / (up_ms * 1e-3) / 1e12
    layer_tflops = expert_flops(shape, args.tokens, k) / (tp["ms"] * 1e-3) / 1e12
    # Decode: HBM-bound gate/up kernel.
    td = results[args.decode_tokens]
    dec_up_ms = td["stages"]["expert_up"]
    # Selected gate/up rows, x in, h out as activation units (144 bytes per
    # 64 values: what the one-token gate/up kernel writes).
    dec_bytes = td["up_bytes"] + args.decode_tokens * shape.hidden * 4 + \
        args.decode_tokens * k * (shape.inter // 64) * 144
    dec_gbs = dec_bytes / (dec_up_ms * 1e-3) / 1e9
    layer_bytes = td["up_bytes"] + td["down_bytes"] + shape.n_experts * shape.hidden * 4 + \
        2 * args.decode_tokens * shape.hidden * 4
    layer_gbs = layer_bytes / (td["ms"] * 1e-3) / 1e9

    batch = None
    if args.batch_tokens:
        tb = results[args.batch_tokens]
        b_bytes = tb["up_bytes"] + tb["down_bytes"] + shape.n_experts * shape.hidden * 4 + \
            2 * args.batch_tokens * shape.hidden * 4
        b_gbs = b_bytes / (tb["ms"] * 1e-3) / 1e9
        batch = {"tokens": args.batch_tokens, "value": round(args.batch_tokens / (tb["ms"] * 1e-3), 1),
                 "unit": "tokens/s", "ms_per_step": round(tb["ms"], 5), "ms_mean": round(tb["ms_mean"], 5),
                 "roofline": {"bound": "hbm", "kernel": "whole layer (hit experts' bytes once)",
                              "achieved": round(b_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                              "frac": round(b_gbs / HBM_PEAK_GBS, 4)},
                 "stages_us": {k_: round(v * 1e3, 2) for k_, v in tb["stages"].items()}}

    cpu = None
    if not args.no_cpu:
        log("timing the CPU restatement (oracle/) on the host cores")
        dec, pre, cores = cpu_baseline(host, args.decode_tokens, args.tokens, args.cpu_runs)
        cpu = dict(value=round(pre, 2), unit="tokens/s", cores=cores, kind="port", cpu_model=cpu_model(),
                   median_of=args.cpu_runs,
                   sample=f"the same layer, weights and inputs: per T one warm-up forward, then the median of "
                          f"{args.cpu_runs} timed forwards, at T={args.tokens} (value) and T={args.decode_tokens} "
                          f"(decode_value)",
                   tokens=args.tokens, decode_tokens=args.decode_tokens, decode_value=round(dec, 2))

    # The committed counter summary covers the default workload only.
    profiled = args.shape == "mixtral" and args.tokens == 512 and args.decode_tokens == 1 and not args.mode
    line = {
        "metric": METRIC,
        "value": round(args.tokens / (tp["ms"] * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(tp["ms"], 5),
        "ms_mean": round(tp["ms_mean"], 5),
        "timing": f"median of {args.steps} steps, each between its own HIP event pair",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32-class (22-bit activation pieces)",
        "arithmetic": "f32 precision on the matrix cores: activations as two f16 pieces (22 significant bits, "
                      "per-row power-of-two scale), weights as their exact integer codes in f16; per 32-value "
                      "block (hi + lo) * q accumulated in f32 by V_MFMA_F32_32X32X16_F16 (2 MFMAs per product), "
                      "then the block's f32 scale applied with one fma (roofline flops count each product once)",
        "data": "synthetic",
        "config": {"workload": f"{shape.name}_moe_layer_T{args.tokens}", "hidden": shape.hidden,
                   "inter": shape.inter, "experts": shape.n_experts, "top_k": shape.top_k,
                   "weights": DT_NAMES.get(shape.expert_dt, str(shape.expert_dt)), "tokens": args.tokens,
                   "weight_copies": args.copies, "tiled_copies": not args.no_tiled},
        "roofline": {"bound": "mfma", "kernel": f"mfma_kernel<{DT_NAMES.get(shape.expert_dt)}, up> (expert gate/up, "
                                                f"MFMA grouped GEMM)",
                     "achieved": round(achieved, 2), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4), "traffic": traffic_of("mfma_kernel<2, true") if profiled else None,
                     "mfma_pipe_frac": round(2 * achieved / MFMA_F16_PEAK_TFLOPS, 4),
                     "layer_frac": round(layer_tflops / MFMA_F16_PEAK_TFLOPS, 4)},
        "cpu_baseline": cpu,
        "decode": {"tokens": args.decode_tokens, "value": round(args.decode_tokens / (td["ms"] * 1e-3), 1),
                   "unit": "tokens/s", "ms_per_step": round(td["ms"], 5), "ms_mean": round(td["ms_mean"], 5),
                   "dtype": "f32-class (three int8 activation levels)",
                   "arithmetic": "f32 precision: quantised codes dotted exactly (v_dot4_i32_i8) with activations "
                                 "held as three int8 levels (error 2^-24 of each 32-value block's range), f32 "
                                 "scales and sums",
                   "roofline": {"bound": "hbm", "kernel": "decode_up_unit_kernel (one-token gate/up, integer-dot "
                                                          "GEMV, h encoded in its blocks)",
                                "achieved": round(dec_gbs, 1),
                                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(dec_gbs / HBM_PEAK_GBS, 4),
                                "traffic": traffic_of("decode_up_unit_kernel") if profiled else None,
                                "layer_frac": round(layer_gbs / HBM_PEAK_GBS, 4)},
                   "stages_us": {k_: round(v * 1e3, 2) for k_, v in td["stages"].items()}},
        "batch": batch,
        "stages_us": {k_: round(v * 1e3, 2) for k_, v in tp["stages"].items()},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
