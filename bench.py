"""Benchmark of the quantized-linear hot path on one MI355X.

Headline (the benchmark's `metric`, its configs[1]): the RWKV-7 1.5B decode GEMV
sweep -- 24 layers x {r, k, v, o [2048,2048], FFN key [8192,2048], FFN value
[2048,8192]} + head [65536,2048], 4-bit g64 with bf16 scales/biases, weights
~N(0,0.02) with a distinct seed per layer and projection (755 MB of packed
weights, larger than the 256 MB MALL), bf16 activations ~N(0,1), M=1.
One step = the whole sweep: one planned grouped call (rq_grouped_plan_run),
a single launch over the 145 independent GEMVs.  `value` = effective weight-stream GB/s:
(R*K*bits/8 + 2*R*(K/gs)*2 bytes summed over the sweep) / step time, with all
inputs resident in HBM.

Alongside: the same sweep at M=8, one GEMV launch per projection (eagerly, and
replayed from one HIP graph), config 1 (0.1B FFN key: quantize, dequantize,
GEMV at M=1/16 as single calls), the prefill
GEMM (benchmark config 3, RWKV-7 2.9B shapes, M=4096/2048/512) and its
transposed product in TFLOP/s, the QLoRA dX product at config-4 shapes, the
config-5 mixed-bit model (7.2B shapes, 3-bit layers + 8-bit head: decode
sweep GB/s, prefill M=2048 TFLOP/s), and the CPU oracle's GEMV timed on the
host cores on a bounded sample.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3]

HBM traffic of the headline kernel (`roofline.traffic`) comes from two
rocprofv3 counter passes over `--pmc-workload` (the headline plan run three
times, then three plain 1 GiB copies that calibrate the counters), reduced by
`--pmc-report FETCH_DIR WRITE_DIR`; the reduced figures are kept in
profiles/qmv_config2_sweep_m1_traffic.txt and read back here.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "rwkv-metal_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
XCDS, CUS = 8, 256             # MI355X: 8 XCDs x 32 CUs
BF16_PEAK_TFLOPS = 2516.6      # MI355X dense bf16 MFMA (256 CU x 2.4 GHz x 4096 flop/clk)
GEMM_WARMUP = 10               # untimed GEMM launches before each timed GEMM region
D, FFN, VOCAB, LAYERS = 2048, 8192, 65536, 24
PROJ = [("r", D, D), ("k", D, D), ("v", D, D), ("o", D, D), ("ffn_key", FFN, D),
        ("ffn_value", D, FFN)]
PROJ_ID = {"r": 0, "k": 1, "v": 2, "o": 3, "ffn_key": 4, "ffn_value": 5, "head": 6}


def weight_bytes(R, K, bits=4, gs=64, sb=2):
    return R * K * bits // 8 + 2 * R * (K // gs) * sb


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # One step of the headline is ~0.13 ms: 100 warmup steps (~13 ms of
    # back-to-back launches) get past the clock/power transient that follows
    # the quantization phase and any idle gap; 200 timed steps are ~26 ms.
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="bounded CPU-baseline sample length")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="headline sweep only")
    ap.add_argument("--pmc-workload", nargs="?", const="gemv",
                    choices=("gemv", "gemm", "gemm_pair", "decode"),
                    help="run the headline plan (gemv) or the config-3 [10240, 2560] prefill "
                         "GEMM at M=4096 (gemm) 3x, then 3 calibration copies; gemm_pair: "
                         "qmm_t_k64 and qmm_n_k64 on [2048, 2048] at M=4096 and qmm_t_k64 on "
                         "[10240, 2560] at M=4096, 3x each; decode: the config-2 sweep as one "
                         "planned launch at M=1, then at M=8, 3x each; print nothing")
    ap.add_argument("--qlora-step-workload", action="store_true",
                    help="run 5 + 20 config-4 QLoRA layer steps (LoRALinear autograd, the "
                         "bench's fused path) for a kernel trace; print the per-step time")
    ap.add_argument("--pmc-counters", metavar="DIR",
                    help="per-kernel averages of every counter in a rocprofv3 --pmc csv output")
    ap.add_argument("--pmc-report", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="reduce two rocprofv3 --pmc csv outputs of --pmc-workload")
    ap.add_argument("--pmc-kernel", default=None,
                    help="kernel name the report reduces (default: the workload's own)")
    ap.add_argument("--kt-report", metavar="DIR",
                    help="print rocprofv3 --kernel-trace --stats csv output as a table")
    return ap.parse_args()


DECODE_STEADY_S = 0.2  # untimed steady-state launches before each decode sweep measurement
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "qmv_config2_sweep_m1_traffic.txt")
PMC_RUNS, COPY_BYTES, COPY_RUNS = 3, 1 << 30, 3
HEAD_KERNEL = "qmv_stream_table"


GEMM_KERNEL = "qmm_t_k64"
PMC_GEMM = (4096, 10240, 2560)  # M, R, K: config 3's ffn_key-shaped prefill


def pmc_workload(torch, rq, dev, which="gemv"):
    """What the counter passes profile: the headline plan (one launch), or one
    config-3 prefill GEMM, PMC_RUNS times, then COPY_RUNS copies of COPY_BYTES
    (read COPY_BYTES, write COPY_BYTES) as the last dispatches of the process."""
    if which == "decode":
        probs, _ = make_sweep(rq, torch, dev, M=1, timed=False)
        ws = [w for _, _, w in probs]
        for M in (1, 8):
            xs = [torch.randn(M, x.shape[-1], device=dev).to(torch.bfloat16) for _, x, _ in probs]
            run = rq.GroupedQmv(xs, ws, 64, 4).run
            for _ in range(PMC_RUNS):
                run()
            torch.cuda.synchronize()
        return
    if which == "gemm_pair":
        runs = []
        for (R, K), transposes in (((2048, 2048), (True, False)), ((10240, 2560), (True,))):
            w = (torch.randn(R, K, device=dev) * 0.02).to(torch.bfloat16)
            wq, s, b = rq.quantize(w, 64, 4)
            for tr in transposes:
                x = torch.randn(4096, K if tr else R, device=dev).to(torch.bfloat16)
                runs.append(rq.BoundQmm(x, wq, s, b, tr, 64, 4).run)
        torch.cuda.synchronize()
        for run in runs:
            for _ in range(PMC_RUNS):
                run()
            torch.cuda.synchronize()
        return
    if which == "gemm":
        M, R, K = PMC_GEMM
        w = (torch.randn(R, K, device=dev) * 0.02).to(torch.bfloat16)
        run = rq.BoundQmm(torch.randn(M, K, device=dev).to(torch.bfloat16),
                          *rq.quantize(w, 64, 4), True, 64, 4).run
    else:
        probs, _ = make_sweep(rq, torch, dev, M=1)
        run = rq.GroupedQmv([x for _, x, _ in probs], [w for _, _, w in probs], 64, 4).run
    torch.cuda.synchronize()
    for _ in range(PMC_RUNS):
        run()
    torch.cuda.synchronize()
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(COPY_RUNS):
        dst.copy_(src)
    torch.cuda.synchronize()


def _pmc_rows(d):
    import csv
    import glob
    files = sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True))
    if not files:
        raise SystemExit(f"no *counter_collection.csv under {d}")
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
    # one value per dispatch (counters are summed over the per-dispatch rows)
    per = {}
    for did, name, v in rows:
        n, acc = per.get(did, (name, 0.0))
        per[did] = (n, acc + v)
    return [(did, *per[did]) for did in sorted(per)]


def pmc_report(fetch_dir, write_dir, kernel=HEAD_KERNEL):
    """Print the calibrated HBM traffic of the headline kernel per step and
    per launch.  FETCH_SIZE / WRITE_SIZE are KiB per dispatch; the factor that
    turns them into bytes is COPY_BYTES over what the calibration copies read
    (resp. wrote)."""
    out = {}
    for tag, d in (("fetch", fetch_dir), ("write", write_dir)):
        rows = _pmc_rows(d)
        copies = rows[-COPY_RUNS:]
        head = [r for r in rows if kernel in r[1]]
        if not head or len(head) % PMC_RUNS:
            raise SystemExit(f"{tag}: {len(head)} {kernel} dispatches, not a multiple of "
                             f"{PMC_RUNS}")
        copy_kib = sum(r[2] for r in copies) / len(copies)
        factor = COPY_BYTES / copy_kib
        out[tag] = {"copy_kernel": copies[0][1][:80], "copy_kib": copy_kib, "factor": factor,
                    "launches_per_step": len(head) // PMC_RUNS,
                    "bytes_per_step": sum(r[2] for r in head) / PMC_RUNS * factor}
    launches = out["fetch"]["launches_per_step"]
    step = out["fetch"]["bytes_per_step"] + out["write"]["bytes_per_step"]
    for tag in ("fetch", "write"):
        o = out[tag]
        print(f"{tag}: calibration copy {o['copy_kernel']!r} reads/writes {COPY_BYTES} B, "
              f"counter {o['copy_kib']:.1f} KiB -> factor {o['factor']:.4f} B per counted KiB")
        print(f"{tag}_bytes_per_step: {o['bytes_per_step']:.0f}")
    print(f"launches_per_step: {launches}")
    print(f"traffic_bytes_per_step: {step:.0f}")
    print(f"traffic_bytes_per_launch: {step / launches:.0f}")


def kt_report(d):
    """Markdown table of the kernel statistics rocprofv3 wrote under `d`
    (*kernel_stats.csv), plus per-grid-size medians of the library's kernels
    from *kernel_trace.csv."""
    import csv
    import glob
    import statistics
    stats = sorted(glob.glob(os.path.join(d, "**", "*kernel_stats.csv"), recursive=True))
    if not stats:
        raise SystemExit(f"no *kernel_stats.csv under {d}")
    print("| kernel | calls | avg us | min us | max us | % time |")
    print("|---|---|---|---|---|---|")
    with open(stats[0], newline="") as fh:
        for r in csv.DictReader(fh):
            name = r["Name"].replace("(anonymous namespace)::", "")
            name = name.split("(")[0] if not name.startswith("void (") else name
            print(f"| `{name[:110]}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                  f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | "
                  f"{float(r['Percentage']):.2f} |")
    traces = sorted(glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True))
    if traces:
        per = {}
        with open(traces[0], newline="") as fh:
            for r in csv.DictReader(fh):
                if not any(k in r["Kernel_Name"] for k in ("qmv_", "qmm_", "quantize_kernel", "lora_down")):
                    continue
                key = (r["Kernel_Name"].replace("(anonymous namespace)::", "").split("(")[0],
                       int(r["Grid_Size_X"]) // max(1, int(r["Workgroup_Size_X"])))
                per.setdefault(key, []).append(
                    (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        print()
        print("| kernel | workgroups | dispatches | median us |")
        print("|---|---|---|---|")
        for (name, wg), v in sorted(per.items()):
            print(f"| `{name[:100]}` | {wg} | {len(v)} | {statistics.median(v):.2f} |")


def pmc_counters(d):
    """Per-kernel, per-grid averages of every counter in a rocprofv3 --pmc
    output, for the library's kernels; plus each kernel's MFMA-busy fraction
    where the pass holds SQ_VALU_MFMA_BUSY_CYCLES and GRBM_GUI_ACTIVE:
    MFMA-busy cycles over the kernel's active cycles on every SIMD
    (256 CUs x 4 SIMDs), rocprofv3's own MfmaUtil expression.  A
    v_mfma_f32_16x16x32_bf16 counts 16 busy cycles, so the fraction is also
    the kernel's MFMA rate over the dense peak at the clock it ran at."""
    import csv
    import glob
    files = sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True))
    if not files:
        raise SystemExit(f"no *counter_collection.csv under {d}")
    per = {}
    for f in files:
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                name = r["Kernel_Name"].replace("(anonymous namespace)::", "").split("(")[0]
                if not any(k in name for k in ("qmv_", "qmm_", "lora_", "quantize_kernel")):
                    continue
                grid = int(r.get("Grid_Size", r.get("Grid_Size_X", 0)) or 0)
                key = (name, grid, int(r["Dispatch_Id"]))
                c = per.setdefault(key, {})
                cn, v = r["Counter_Name"], float(r["Counter_Value"])
                # GRBM counters are whole-GPU cycle counts repeated per instance: max;
                # the SQ counters are per-instance parts of one total: sum
                c[cn] = max(c.get(cn, 0.0), v) if cn.startswith("GRBM_") else c.get(cn, 0.0) + v
    agg = {}
    for (name, grid, _), c in per.items():
        a = agg.setdefault((name, grid), {"n": 0})
        a["n"] += 1
        for k, v in c.items():
            a[k] = a.get(k, 0.0) + v
    for (name, grid), a in sorted(agg.items()):
        n = a.pop("n")
        print(f"{name} grid={grid} dispatches={n}")
        for k in sorted(a):
            print(f"  {k}: {a[k] / n:.6g}")
        if "SQ_VALU_MFMA_BUSY_CYCLES" in a and "GRBM_GUI_ACTIVE" in a:
            # the csv's GRBM_GUI_ACTIVE is the sum over the 8 XCDs' instances (8 x the
            # kernel's cycles); MfmaUtil takes one instance (reduce max)
            cycles = a["GRBM_GUI_ACTIVE"] / n / XCDS
            frac = a["SQ_VALU_MFMA_BUSY_CYCLES"] / n / (cycles * CUS * 4)
            print(f"  kernel_cycles (GRBM_GUI_ACTIVE / {XCDS}): {cycles:.6g}")
            print(f"  mfma_busy_frac: {frac:.4f}")


def read_traffic():
    """traffic_bytes_per_launch from the committed counter summary, or None."""
    try:
        with open(TRAFFIC_FILE) as fh:
            for line in fh:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def make_sweep(rq, torch, dev, M, bits=4, gs=64, timed=True):
    """Quantize the config-2 weights on the GPU (seed per layer/projection).
    Also returns the quantize and dequantize kernels' GB/s on the head weight
    (R*K*2 bytes of bf16 weights + the packed bytes, read or written), each
    timed as one region of repeated calls (timed=False: None, None)."""
    probs = []
    qgbs = dgbs = None
    for layer in range(LAYERS + 1):
        items = PROJ if layer < LAYERS else [("head", VOCAB, D)]
        for name, R, K in items:
            seed = 2_000_000 + 1000 * layer + PROJ_ID[name]
            g = torch.Generator(device=dev).manual_seed(seed)
            w = (torch.randn(R, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
            wq, s, b = rq.quantize(w, gs, bits)
            if name == "head" and timed:
                nb = R * K * 2 + weight_bytes(R, K, bits, gs)
                qgbs = nb / time_region(torch, lambda: rq.quantize(w, gs, bits), 20, 5) / 1e9
                dgbs = nb / time_region(torch, lambda: rq.dequantize(wq, s, b, gs, bits), 20, 5) / 1e9
            del w
            gx = torch.Generator(device=dev).manual_seed(seed + 500)
            x = torch.randn(M, K, generator=gx, device=dev).to(torch.bfloat16)
            probs.append((name, x, (wq, s, b)))
    return probs, (qgbs, dgbs)


def config1(torch, rq, dev, args):
    """benchmark config 1 (RWKV-7 0.1B FFN key, W [3072, 768], 4-bit g64): the
    quantize -> dequantize round trip and y = x . W^T at M = 1 and 16, each
    timed as back-to-back single calls (launch-latency-bound at this size:
    1.3 MB of packed weights)."""
    R, K, gs, bits = 3072, 768, 64, 4
    g = torch.Generator(device=dev).manual_seed(1_000_004)
    w = (torch.randn(R, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    wq, s, b = rq.quantize(w, gs, bits)
    out = {}
    n = max(20, args.steps)
    out["quantize_us"] = round(time_region(torch, lambda: rq.quantize(w, gs, bits), n, 10) * 1e6, 2)
    out["dequantize_us"] = round(time_region(torch, lambda: rq.dequantize(wq, s, b, gs, bits), n, 10) * 1e6, 2)
    # the same calls replayed from a HIP graph: the GPU side without the host
    # work (argument checks, output allocation, the launch) that bounds the
    # single calls above
    for name, fn in (("quantize", lambda: rq.quantize(w, gs, bits)),
                     ("dequantize", lambda: rq.dequantize(wq, s, b, gs, bits))):
        reps = 20
        fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps):
                fn()
        out[f"{name}_hip_graph_us"] = round(time_region(torch, graph.replay, 10, 3) / reps * 1e6, 2)
        del graph
    for M in (1, 16):
        x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
        bq = rq.BoundQmm(x, wq, s, b, True, gs, bits)
        t = time_region(torch, bq.run, n, 10)
        out[f"qmm_m{M}_us"] = round(t * 1e6, 2)
        out[f"qmm_m{M}_weight_gbs"] = round(weight_bytes(R, K, bits, gs) / t / 1e9, 1)
    return out


C5_SHAPE, C5_LAYERS = (4096, 16384, 65536), 32  # D, FFN, vocab of RWKV-7 7.2B


def config5_sweep(torch, rq, dev):
    """The config-5 decode inputs on the GPU: every layer's 3-bit g64
    r/k/v/o [4096, 4096], ffn_key [16384, 4096], ffn_value [4096, 16384]
    (one seed per layer and projection) with M = 1 activations, and the 8-bit
    g64 head [65536, 4096].  Returns (ws, xs, head, xh, weight bytes)."""
    D5, F5, V5 = C5_SHAPE
    shapes = [(D5, D5)] * 4 + [(F5, D5), (D5, F5)]
    ws, xs, nbytes = [], [], 0
    for layer in range(C5_LAYERS):
        for i, (R, K) in enumerate(shapes):
            g = torch.Generator(device=dev).manual_seed(5_000_000 + 10 * layer + i)
            w = (torch.randn(R, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
            ws.append(rq.quantize(w, 64, 3))
            xs.append(torch.randn(1, K, generator=g, device=dev).to(torch.bfloat16))
            nbytes += weight_bytes(R, K, 3)
            del w
    g = torch.Generator(device=dev).manual_seed(5_999_999)
    w = (torch.randn(V5, D5, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    head = rq.quantize(w, 64, 8)
    del w
    xh = torch.randn(1, D5, generator=g, device=dev).to(torch.bfloat16)
    nbytes += weight_bytes(V5, D5, 8)
    return ws, xs, head, xh, nbytes


def config5(torch, rq, dev, args):
    """benchmark config 5: RWKV-7 7.2B shapes (D=4096, FFN 16384, vocab 65536),
    3-bit g64 r/k/v/o and FFN, 8-bit g64 head, bf16 scales/biases.  Decode:
    all 32 layers' 3-bit projections in one planned launch plus the 8-bit
    head in a second, M=1, GB/s of packed weights + scales/biases.  Prefill:
    each shape at M=2048, TFLOP/s."""
    D5, F5, V5 = C5_SHAPE
    ws, xs, head, xh, nbytes = config5_sweep(torch, rq, dev)
    p3 = rq.GroupedQmv(xs, ws, 64, 3)
    p8 = rq.GroupedQmv([xh], [head], 64, 8)

    def step():
        p3.run()
        p8.run()
    steady_state(torch, step, DECODE_STEADY_S)
    t = time_region(torch, step, max(5, args.steps // 2), 2)
    out = {"decode_m1_gbs": round(nbytes / t / 1e9, 1),
           "decode_weight_bytes": nbytes,
           "decode_planned": p3.plan is not None and p8.plan is not None}
    del p3, xs
    gemm_steady_state(torch, rq, dev)
    pre = {}
    for name, R, K, wq3 in (("rkvo", D5, D5, ws[0]), ("ffn_key", F5, D5, ws[4]),
                            ("ffn_value", D5, F5, ws[5]), ("head_8bit", V5, D5, head)):
        bits = 8 if name == "head_8bit" else 3
        x = torch.randn(2048, K, device=dev).to(torch.bfloat16)
        tt = time_region(torch, rq.BoundQmm(x, *wq3, True, 64, bits).run,
                         max(5, args.steps // 4), GEMM_WARMUP)
        pre[name] = round(2.0 * 2048 * R * K / tt / 1e12, 1)
    out["prefill_m2048_tflops"] = pre
    return out


def qlora_layers(torch, rq, dev, ws, xdt=None):
    """Config 4's QLoRA layer: for each projection a LoRALinear (r = alpha =
    16, A ~ N(0, 1/D), B ~ N(0, 0.01) std, bf16) over the frozen 4-bit g64
    base `ws[i]`, with x [8, 512, K] and dY [8, 512, R] in `xdt` (bf16 by
    default; fp32 is the reference's residual stream).  Returns the
    (layer, x, dY) triples and the step's flops (base forward + dX GEMMs and
    the adapter GEMMs)."""
    xdt = xdt or torch.bfloat16
    r, alpha, M = 16, 16.0, 8 * 512
    layers, flops = [], 0.0
    for name, R, K in PROJ:
        wq, s, b = ws[PROJ.index((name, R, K))]
        base = rq.QuantizedLinear(K, R, bias=False, group_size=64, bits=4, device=dev)
        base.weight, base.scales, base.biases = wq, s, b
        lay = rq.LoRALinear(rank=r, alpha=alpha, base_module=base)
        g = torch.Generator(device=dev).manual_seed(4_000_000 + R * 7 + K)
        with torch.no_grad():
            lay.lora_a.copy_((torch.randn(r, K, generator=g, device=dev) / K ** 0.5).to(torch.bfloat16))
            lay.lora_b.copy_((torch.randn(R, r, generator=g, device=dev) * 0.01).to(torch.bfloat16))
        x = torch.randn(8, 512, K, device=dev).to(xdt).requires_grad_(True)
        dy = torch.randn(8, 512, R, device=dev).to(xdt)
        layers.append((lay, x, dy))
        flops += 4.0 * M * R * K + 6.0 * M * r * (R + K)
    return layers, flops


def qlora_step_workload(torch, rq, dev):
    """What a kernel trace of the config-4 QLoRA layer step profiles: 5
    untimed and 20 timed fused layer steps."""
    ws = []
    for name, R, K in PROJ:
        g = torch.Generator(device=dev).manual_seed(2_000_000 + PROJ_ID[name])
        ws.append(rq.quantize((torch.randn(R, K, generator=g, device=dev) * 0.02).to(torch.bfloat16), 64, 4))
    layers, _ = qlora_layers(torch, rq, dev, ws)

    def fused():
        layer_step(torch, layers, lambda lay, x: lay(x))
    for _ in range(5):
        fused()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(20):
        fused()
    torch.cuda.synchronize()
    print(f"config-4 QLoRA layer step: {1e3 * (time.perf_counter() - t0) / 20:.3f} ms", flush=True)


def layer_step(torch, layers, forward):
    """One training step of the layer's projections: every forward, then one
    backward pass over all of them (dX, dA, dB for each), as a training
    step's single backward call runs it."""
    ys, ins, dys = [], [], []
    for lay, x, dy in layers:
        ys.append(forward(lay, x))
        ins += [x, lay.lora_a, lay.lora_b]
        dys.append(dy)
    torch.autograd.grad(ys, ins, dys)


def qlora_step(torch, rq, dev, ws, args):
    """benchmark config 4: one QLoRA training step of one RWKV-7 1.5B layer
    (D=2048) on a frozen 4-bit g64 base -- for each of r, k, v, o, ffn_key,
    ffn_value: y = qmm(x, Wq) + (alpha/r) (x A^T) B^T, r = alpha = 16,
    A ~ N(0, 1/D), B ~ N(0, 0.01) (std), x [8, 512, K] bf16, then dX, dA, dB
    for a given dY.  `fused`: LoRALinear's path (rank 16, 4-bit: the forward
    and dX are one rq_qlora launch each, with x A^T / dY B computed inside the
    GEMM and the term added in its output stage, and dA, dB one rq_lora_grads
    launch); `composed`: the same layer as separate ops
    (quantized_matmul + two torch GEMMs + scale + add, autograd).  Reported:
    ms per layer step and the step's TFLOP/s (base forward + dX GEMMs, 4*M*R*K,
    plus the adapter GEMMs)."""
    layers, flops = qlora_layers(torch, rq, dev, ws)

    def fused():
        layer_step(torch, layers, lambda lay, x: lay(x))

    def composed():
        layer_step(torch, layers, lambda lay, x: rq.quantized_matmul(
            x, lay.linear.weight, lay.linear.scales, lay.linear.biases, True, 64, 4)
            + lay.scale * ((x @ lay.lora_a.t()) @ lay.lora_b.t()))

    out = {}
    for key, fn in (("fused", fused), ("composed", composed)):
        t = time_region(torch, fn, max(5, args.steps // 10), 3)
        out[key] = {"ms_per_layer_step": round(t * 1e3, 3),
                    "tflops": round(flops / t / 1e12, 1)}
    out["speedup_fused"] = round(out["composed"]["ms_per_layer_step"]
                                 / out["fused"]["ms_per_layer_step"], 3)
    # the same fused step with fp32 x and dY (the reference's default
    # activations, rwkv_metal/model/rwkv7_x070.py:51): y and dX fp32
    layers32, _ = qlora_layers(torch, rq, dev, ws, torch.float32)

    def fused32():
        layer_step(torch, layers32, lambda lay, x: lay(x))
    t = time_region(torch, fused32, max(5, args.steps // 10), 3)
    out["fused_fp32_x"] = {"ms_per_layer_step": round(t * 1e3, 3),
                           "tflops": round(flops / t / 1e12, 1),
                           "vs_bf16_fused": round(t * 1e3 / out["fused"]["ms_per_layer_step"], 3)}
    return out


def gemm_steady_state(torch, rq, dev, seconds=0.15):
    """Untimed MFMA-heavy GEMM work before the GEMM measurements: coming from
    the memory-bound decode sweeps, the first ~100 ms of back-to-back GEMMs
    run 5-20 % slower while the clocks settle, and a prefill or training
    step is steady-state GEMM work."""
    w = (torch.randn(10240, 2560, device=dev) * 0.02).to(torch.bfloat16)
    run = rq.BoundQmm(torch.randn(4096, 2560, device=dev).to(torch.bfloat16),
                      *rq.quantize(w, 64, 4), True, 64, 4).run
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(20):
            run()
        torch.cuda.synchronize()


def steady_state(torch, fn, seconds):
    """Untimed back-to-back launches of `fn` for `seconds` before a decode
    measurement: after the setup (quantization, allocation) the first
    ~100-1000 launches of the sweep run 1-3 % slower while the clocks settle
    (measured: 100 warm-up steps 5563-5604 GB/s, 1000 or more 5700-5720)."""
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(50):
            fn()
        torch.cuda.synchronize()


def time_region(torch, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / steps


def dependency_levels(torch, rq, xs, ws, outs, total_wbytes, args):
    """The config-2 sweep in a real decode step's order: per layer the
    independent r/k/v projections (rwkv_metal/model/rwkv7_x070.py:142-144)
    as one grouped call, then o (:204), ffn_key and ffn_value (:221, each
    reads the previous one's output), then the head (:343) -- 97 dependent
    launches.  Timed eagerly and replayed from one HIP graph."""
    n = len(PROJ)
    calls = []
    for layer in range(LAYERS):
        i0 = layer * n
        for group in ((0, 1, 2), (3,), (4,), (5,)):
            idx = [i0 + j for j in group]
            calls.append(rq.GroupedQmv([xs[i] for i in idx], [ws[i] for i in idx], 64, 4,
                                       out=[outs[i] for i in idx]).run)
    calls.append(rq.GroupedQmv([xs[-1]], [ws[-1]], 64, 4, out=[outs[-1]]).run)

    def step():
        for f in calls:
            f()
    steady_state(torch, step, DECODE_STEADY_S / 2)
    t_eager = time_region(torch, step, max(3, args.steps // 4), 1)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    t_graph = time_region(torch, graph.replay, max(3, args.steps // 4), 3)
    del graph
    return {"launches_per_step": len(calls),
            "eager_gbs": round(total_wbytes / t_eager / 1e9, 2),
            "hip_graph_gbs": round(total_wbytes / t_graph / 1e9, 2),
            "hip_graph_us_per_step": round(t_graph * 1e6, 1)}


def decode_per_shape(torch, rq, dev, args, gs=64, bits=4):
    """Config 2's GEMV per shape (r/k/v/o, ffn_key, ffn_value, head) at M = 1
    and 8, each over a rotation of distinct weight buffers of >= 512 MB (2x
    the 256 MB MALL, so neither L2 nor MALL serves a launch its weights): one
    launch per buffer, captured in one HIP graph, replayed; 5 timed regions
    of >= 20 launches after 3 warm-up replays, median per-launch time.  Each
    launch is one rq_qmm call (the split GEMV below 32768 rows, the streamed
    one for the head)."""
    import statistics
    out = {}
    for name, R, K in [("rkvo", D, D), ("ffn_key", FFN, D), ("ffn_value", D, FFN), ("head", VOCAB, D)]:
        wb = weight_bytes(R, K, bits, gs)
        nbuf = max(2, -(-(512 << 20) // wb))
        bufs = []
        for i in range(nbuf):
            g = torch.Generator(device=dev).manual_seed(2_100_000 + 7919 * i + R + K)
            w = (torch.randn(R, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
            bufs.append(rq.quantize(w, gs, bits))
            del w
        res = {"weight_bytes": wb, "buffers": nbuf}
        for M in (1, 8):
            x = torch.randn(M, K, device=dev).to(torch.bfloat16)
            bound = [rq.BoundQmm(x, wq, s, b, True, gs, bits) for wq, s, b in bufs]
            reps_per_region = max(1, -(-20 // nbuf))

            def rotation():
                for _ in range(reps_per_region):
                    for bq in bound:
                        bq.run()
            rotation()
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                rotation()
            for _ in range(3):
                graph.replay()
            torch.cuda.synchronize()
            launches = reps_per_region * nbuf
            per = []
            for _ in range(5):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                graph.replay()
                e1.record()
                torch.cuda.synchronize()
                per.append(e0.elapsed_time(e1) / 1e3 / launches)
            t = statistics.median(per)
            res[f"m{M}_us"] = round(t * 1e6, 2)
            res[f"m{M}_gbs"] = round(wb / t / 1e9, 1)
            del graph, bound
        out[name] = res
        del bufs
    return out


def dense_bf16_gemms(torch, dev, args):
    """torch.matmul (hipBLASLt) of dense bf16 operands at config 3's shapes,
    M = 4096: the vendor library's dense GEMM on the same box and clocks."""
    out, fl, tt = {}, 0.0, 0.0
    for R, K in ((2560, 2560), (10240, 2560), (2560, 10240)):
        a = torch.randn(4096, K, device=dev).to(torch.bfloat16)
        w = (torch.randn(R, K, device=dev) * 0.02).to(torch.bfloat16)
        wt = w.t()
        t = time_region(torch, lambda: torch.matmul(a, wt), max(5, args.steps // 2), GEMM_WARMUP)
        f = 2.0 * 4096 * R * K
        out[f"{R}x{K}_M4096"] = round(f / t / 1e12, 1)
        fl += f
        tt += t
        del a, w, wt
    out["aggregate"] = round(fl / tt / 1e12, 1)
    return out


MFMA_FILE = os.path.join(ROOT, "profiles", "qmm_k64_m4096_counters.txt")


def read_mfma_busy():
    """mfma_busy_frac of qmm_t_k64 on config 3 [10240, 2560] at M = 4096 from
    the committed rocprofv3 counter summary, or None."""
    try:
        with open(MFMA_FILE) as fh:
            for line in fh:
                if line.startswith("qmm_t_k64 mfma_busy_frac:"):
                    return float(line.split(":", 1)[1])
    except (OSError, ValueError):
        pass
    return None


def _cpu_model():
    """The host CPU's model name (/proc/cpuinfo, as lscpu prints it)."""
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _host_threads():
    """Threads the all-core leg uses: the cores this process may run on,
    capped by OMP_NUM_THREADS where the environment sets it (one GPU's share
    of a shared host)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def cpu_baseline(torch, seconds):
    """The oracle's GEMV (rqo_qmv_bf16, the reference algorithm restated in
    C: per-group sums of x*code and x, scale and bias once per group) on the
    host over a bounded sample of the headline workload: one config-2 layer's
    six projections at M = 1 (28.3 MB of packed weights).  Each leg (1 thread,
    then all the host threads this process may use) times 6 repetitions of
    enough passes for ~`seconds`/12 each and reports the median of the last 5
    (the first is the warm-up)."""
    import statistics
    from oracle import oracle as O
    if not os.path.exists(O._LIB_PATH):
        O.build()
    sample, sample_bytes = [], 0
    for name, R, K in PROJ:
        g = torch.Generator().manual_seed(2_000_000 + PROJ_ID[name])
        w = (torch.randn(R, K, generator=g) * 0.02).to(torch.bfloat16)
        wq, s, b = O.quantize(w, 64, 4)
        x = torch.randn(1, K, generator=g).to(torch.bfloat16)
        sample.append((x, wq, s, b))
        sample_bytes += weight_bytes(R, K)

    def one_pass(nt):
        for x, wq, s, b in sample:
            O.qmv_bf16(x, wq, s, b, 64, 4, nthreads=nt)

    legs = {}
    for nt in (1, _host_threads()):
        t0 = time.perf_counter()
        one_pass(nt)
        passes = max(1, int(seconds / 12 / max(time.perf_counter() - t0, 1e-6)))
        rates = []
        for _ in range(6):
            t0 = time.perf_counter()
            for _ in range(passes):
                one_pass(nt)
            rates.append(passes * sample_bytes / (time.perf_counter() - t0) / 1e9)
        legs[nt] = (statistics.median(rates[1:]), passes)
    threads = max(legs)
    return {"value": round(legs[threads][0], 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "value_1_thread": round(legs[1][0], 3),
            "cpu_model": _cpu_model(), "nproc": os.cpu_count(),
            "sample": (f"oracle rqo_qmv_bf16 (reference-algorithm CPU restatement, not MLX), "
                       f"one RWKV-7 1.5B layer r/k/v/o/ffn_key/ffn_value at M=1, 4-bit g64 "
                       f"({sample_bytes} B of weights); median of 5 timed repetitions after 1 "
                       f"warm-up, {legs[threads][1]} passes each on {threads} threads, "
                       f"{legs[1][1]} on 1 thread")}


def main():
    args = parse()
    if args.pmc_report:
        pmc_report(*args.pmc_report, kernel=args.pmc_kernel or HEAD_KERNEL)
        return
    if args.kt_report:
        kt_report(args.kt_report)
        return
    if args.pmc_counters:
        pmc_counters(args.pmc_counters)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(multi-GPU sharding is a design, not code, here)"}))
        sys.exit(2)
    import torch
    import rwkvq

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    bits, gs = 4, 64
    if args.pmc_workload:
        pmc_workload(torch, rwkvq, dev, args.pmc_workload)
        return
    if args.qlora_step_workload:
        qlora_step_workload(torch, rwkvq, dev)
        return

    # ---------------- headline: config-2 decode sweep, M=1, grouped launches
    probs, (quant_gbs, dequant_gbs) = make_sweep(rwkvq, torch, dev, M=1)
    total_wbytes = sum(weight_bytes(w[0].shape[0], x.shape[1]) for _, x, w in probs)
    xs = [x for _, x, _ in probs]
    ws = [w for _, _, w in probs]
    outs = [torch.empty(1, w[0].shape[0], dtype=torch.bfloat16, device=dev) for w in ws]

    plan = rwkvq.GroupedQmv(xs, ws, gs, bits, out=outs)
    steady_state(torch, plan.run, DECODE_STEADY_S)
    t_step = time_region(torch, plan.run, args.steps, args.warmup)
    value = total_wbytes / t_step / 1e9

    # The step is one planned grouped call (rq_grouped_plan_run): ONE launch
    # of qmv_stream_table over all 145 problems (7936 blocks of 64 rows,
    # K=8192 blocks first).  Average launch duration = the timed region's
    # HIP-event time (events on torch's current stream, the stream the
    # library launches on) over the launches in it; the launches run back to
    # back, so the region is kernel time.
    assert plan.plan is not None, "the config-2 sweep must run on the planned GEMV"
    launches = 1
    avg_launch = t_step / launches
    bytes_per_launch = total_wbytes / launches
    achieved = bytes_per_launch / avg_launch / 1e9
    result = {
        "metric": "q4 GEMV effective HBM GB/s (% of peak) + prefill qmm TFLOP/s, RWKV-7 1.5B",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_step * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) weights per layer/projection, N(0,1) activations)",
        "config": {
            "workload": ("config2: RWKV-7 1.5B decode GEMV sweep, 24 layers x {r,k,v,o "
                         "[2048,2048], ffn_key [8192,2048], ffn_value [2048,8192]} + head "
                         "[65536,2048], M=1, 4-bit g64 bf16 scales/biases, as ONE cross-layer "
                         "batched launch of the 145 independent GEMVs (a real decode step "
                         "cannot batch across layers: layer l+1 reads layer l's output; "
                         "extra.decode_m1_dependency_levels is that order)"),
            "weight_bytes_per_step": total_wbytes,
            "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
            "launches_per_step": launches,
        },
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic(),
                     "kernel": "qmv_stream_table<BITS=4, scales bf16, NMC=1, MI=1, GSH=6>",
                     "avg_launch_us": round(avg_launch * 1e6, 2),
                     "bytes_per_launch": int(bytes_per_launch)},
    }

    if not args.no_extra:
        extra = {}
        extra["quantize_gbs"] = round(quant_gbs, 1)
        extra["dequantize_gbs"] = round(dequant_gbs, 1)
        # M=8 sweep
        xs8 = [torch.randn(8, x.shape[1], device=dev).to(torch.bfloat16) for x in xs]
        outs8 = [torch.empty(8, w[0].shape[0], dtype=torch.bfloat16, device=dev) for w in ws]
        plan8 = rwkvq.GroupedQmv(xs8, ws, gs, bits, out=outs8)
        steady_state(torch, plan8.run, DECODE_STEADY_S)
        t8 = time_region(torch, plan8.run, args.steps, args.warmup)
        extra["decode_m8_gbs"] = round(total_wbytes / t8 / 1e9, 2)
        # one launch per projection (dependency-faithful order), M=1
        singles = [rwkvq.GroupedQmv([x], [w], gs, bits, out=[o]).run
                   for x, w, o in zip(xs, ws, outs)]

        def per_call():
            for f in singles:
                f()
        tpc = time_region(torch, per_call, max(3, args.steps // 4), 1)
        extra["decode_m1_one_launch_per_projection_gbs"] = round(total_wbytes / tpc / 1e9, 2)
        # the same 145 launches captured once in a HIP graph and replayed:
        # one graph launch per decode step instead of 145 host dispatches
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            per_call()
        tgr = time_region(torch, graph.replay, max(3, args.steps // 4), 3)
        extra["decode_m1_one_launch_per_projection_hip_graph_gbs"] = round(total_wbytes / tgr / 1e9, 2)
        del graph
        extra["decode_m1_dependency_levels"] = dependency_levels(torch, rwkvq, xs, ws, outs,
                                                                 total_wbytes, args)
        # the same order for a batch of 8 sequences
        extra["decode_m8_dependency_levels"] = dependency_levels(torch, rwkvq, xs8, ws, outs8,
                                                                 total_wbytes, args)
        extra["decode_per_shape_rotating_512mb"] = decode_per_shape(torch, rwkvq, dev, args)
        # prefill GEMM, config 3 (RWKV-7 2.9B shapes) at M = 4096 (aggregate) and
        # 2048 / 512; the transposed product (QLoRA dX) at M = 4096
        pre = {}
        tot_flops, tot_t = 0.0, 0.0
        gemm_steady_state(torch, rwkvq, dev)
        for R, K in ((2560, 2560), (10240, 2560), (2560, 10240)):
            g = torch.Generator(device=dev).manual_seed(3_000_000 + R)
            w = (torch.randn(R, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
            wq, s, b = rwkvq.quantize(w, gs, bits)
            for M in (4096, 2048, 512):
                x = torch.randn(M, K, device=dev).to(torch.bfloat16)
                t = time_region(torch, rwkvq.BoundQmm(x, wq, s, b, True, gs, bits).run,
                                max(5, args.steps // 2), GEMM_WARMUP)
                fl = 2.0 * M * R * K
                pre[f"{R}x{K}_M{M}"] = round(fl / t / 1e12, 1)
                if M == 4096:
                    tot_flops += fl
                    tot_t += t
                    # the reference's default fp32 activations (fp32 output)
                    t32 = time_region(torch, rwkvq.BoundQmm(x.float(), wq, s, b, True, gs,
                                                            bits).run,
                                      max(5, args.steps // 2), GEMM_WARMUP)
                    pre[f"{R}x{K}_M4096_fp32_x"] = round(fl / t32 / 1e12, 1)
            dy = torch.randn(4096, R, device=dev).to(torch.bfloat16)
            tn = time_region(torch, rwkvq.BoundQmm(dy, wq, s, b, False, gs, bits).run,
                             max(5, args.steps // 2), GEMM_WARMUP)
            pre[f"{R}x{K}_M4096_transposed"] = round(2.0 * 4096 * R * K / tn / 1e12, 1)
            del w
        agg = tot_flops / tot_t / 1e12
        extra["prefill_qmm_m4096"] = {"tflops": round(agg, 1),
                                      "frac_of_bf16_peak": round(agg / BF16_PEAK_TFLOPS, 4),
                                      "per_shape_tflops": pre}
        dense = dense_bf16_gemms(torch, dev, args)
        extra["dense_bf16_torch_matmul_m4096_tflops"] = dense
        result["roofline_gemm"] = {
            "bound": "mfma", "achieved": round(agg, 1), "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": round(agg / BF16_PEAK_TFLOPS, 4),
            "kernel": "qmm_t_k64<BITS=4, scales bf16> (256 x 160 / 256 x 128 tiles)",
            "workload": "config3 prefill at M=4096 over [2560,2560], [10240,2560], [2560,10240] "
                        "(aggregate flops / summed time)",
            "flops_per_step": tot_flops,
            "mfma_busy_frac": read_mfma_busy(),
            "dense_bf16_torch_matmul_same_shapes_tflops": dense["aggregate"]}
        # QLoRA backward, config 4 (D=2048, M = 8 x 512): dX = dY . W^ per projection
        bwd = {}
        for name, R, K in (("rkvo", D, D), ("ffn_key", FFN, D), ("ffn_value", D, FFN)):
            wq, s, b = ws[PROJ.index(next(p for p in PROJ if p[0] == ("r" if name == "rkvo" else name)))]
            dy = torch.randn(4096, R, device=dev).to(torch.bfloat16)
            tn = time_region(torch, rwkvq.BoundQmm(dy, wq, s, b, False, gs, bits).run,
                             max(5, args.steps // 2), GEMM_WARMUP)
            bwd[name] = round(2.0 * 4096 * R * K / tn / 1e12, 1)
        extra["qlora_dx_m4096_tflops"] = bwd
        extra["qlora_step_config4"] = qlora_step(torch, rwkvq, dev, ws, args)
        del ws, xs, xs8, outs8, plan8, singles
        extra["config1_ffn_key_0.1b"] = config1(torch, rwkvq, dev, args)
        extra["config5_mixed_bit"] = config5(torch, rwkvq, dev, args)
        result["extra"] = extra

    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(torch, args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
