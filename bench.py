"""Benchmark of the quantized-linear hot path on one MI355X.

Headline (BASELINE.json `metric`, configs[1]): the RWKV-7 1.5B decode GEMV
sweep -- 24 layers x {r, k, v, o [2048,2048], FFN key [8192,2048], FFN value
[2048,8192]} + head [65536,2048], 4-bit g64 with bf16 scales/biases, weights
~N(0,0.02) with a distinct seed per layer and projection (755 MB of packed
weights, larger than the 256 MB MALL), bf16 activations ~N(0,1), M=1.
One step = the whole sweep, run by rq_qmm_grouped (145 independent GEMVs in
ceil(145/48) launches).  `value` = effective weight-stream GB/s:
(R*K*bits/8 + 2*R*(K/gs)*2 bytes summed over the sweep) / step time, with all
inputs resident in HBM.

Alongside: the same sweep at M=8, one GEMV launch per projection, the prefill
GEMM (RWKV-7 2.9B shapes, M=4096) in TFLOP/s, and the CPU
oracle's GEMV timed on the host cores on a bounded sample.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3]
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
BF16_PEAK_TFLOPS = 2516.6      # MI355X dense bf16 MFMA (256 CU x 2.4 GHz x 4096 flop/clk)
D, FFN, VOCAB, LAYERS = 2048, 8192, 65536, 24
PROJ = [("r", D, D), ("k", D, D), ("v", D, D), ("o", D, D), ("ffn_key", FFN, D),
        ("ffn_value", D, FFN)]
PROJ_ID = {"r": 0, "k": 1, "v": 2, "o": 3, "ffn_key": 4, "ffn_value": 5, "head": 6}


def weight_bytes(R, K, bits=4, gs=64, sb=2):
    return R * K * bits // 8 + 2 * R * (K // gs) * sb


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="bounded CPU-baseline sample length")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="headline sweep only")
    return ap.parse_args()


def make_sweep(rq, torch, dev, M, bits=4, gs=64):
    """Quantize the config-2 weights on the GPU (seed per layer/projection)."""
    probs = []
    qtime = 0.0
    qbytes = 0
    for layer in range(LAYERS + 1):
        items = PROJ if layer < LAYERS else [("head", VOCAB, D)]
        for name, R, K in items:
            seed = 2_000_000 + 1000 * layer + PROJ_ID[name]
            g = torch.Generator(device=dev).manual_seed(seed)
            w = (torch.randn(R, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            wq, s, b = rq.quantize(w, gs, bits)
            e1.record()
            e1.synchronize()
            qtime += e0.elapsed_time(e1) / 1e3
            qbytes += R * K * 2 + weight_bytes(R, K, bits, gs)
            del w
            gx = torch.Generator(device=dev).manual_seed(seed + 500)
            x = torch.randn(M, K, generator=gx, device=dev).to(torch.bfloat16)
            probs.append((name, x, (wq, s, b)))
    return probs, qbytes / qtime / 1e9


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


def launch_durations(torch, fns, reps=5):
    """HIP-event duration of each launch in `fns` (one event pair per launch,
    on the stream the kernels run on), averaged over reps."""
    tot = [0.0] * len(fns)
    for _ in range(reps):
        evs = []
        for f in fns:
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            f()
            b.record()
            evs.append((a, b))
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(evs):
            tot[i] += a.elapsed_time(b) / 1e3
    return [t / reps for t in tot]


def cpu_baseline(torch, seconds):
    """The oracle's GEMV (rqo_qmv_bf16) on host cores over a bounded sample:
    one config-2 layer's six projections at M=1, repeated for ~`seconds`."""
    from oracle import oracle as O
    if not os.path.exists(O._LIB_PATH):
        O.build()
    threads = max(1, min(16, os.cpu_count() or 1))
    sample = []
    for name, R, K in PROJ:
        g = torch.Generator().manual_seed(2_000_000 + PROJ_ID[name])
        w = (torch.randn(R, K, generator=g) * 0.02).to(torch.bfloat16)
        wq, s, b = O.quantize(w, 64, 4)
        x = torch.randn(1, K, generator=g).to(torch.bfloat16)
        sample.append((x, wq, s, b, weight_bytes(R, K)))
    done_bytes, t0 = 0, time.perf_counter()
    passes = 0
    while True:
        for x, wq, s, b, nb in sample:
            O.qmv_bf16(x, wq, s, b, 64, 4, nthreads=threads)
            done_bytes += nb
        passes += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"value": round(done_bytes / el / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": (f"oracle rqo_qmv_bf16 (reference-algorithm CPU restatement, not MLX), "
                       f"one RWKV-7 1.5B layer r/k/v/o/ffn_key/ffn_value at M=1, 4-bit g64, "
                       f"{passes} passes in {el:.1f} s on {threads} threads")}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(the sharding design is described in DESIGN.md)"}))
        sys.exit(2)
    import torch
    import rwkvq

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    bits, gs = 4, 64

    # ---------------- headline: config-2 decode sweep, M=1, grouped launches
    probs, quant_gbs = make_sweep(rwkvq, torch, dev, M=1)
    total_wbytes = sum(weight_bytes(w[0].shape[0], x.shape[1]) for _, x, w in probs)
    xs = [x for _, x, _ in probs]
    ws = [w for _, _, w in probs]
    outs = [torch.empty(1, w[0].shape[0], dtype=torch.bfloat16, device=dev) for w in ws]

    plan = rwkvq.GroupedQmv(xs, ws, gs, bits, out=outs)
    t_step = time_region(torch, plan.run, args.steps, args.warmup)
    value = total_wbytes / t_step / 1e9

    # per-launch HIP-event durations of the grouped GEMV kernel
    chunks = [(xs[i:i + 48], ws[i:i + 48], outs[i:i + 48]) for i in range(0, len(xs), 48)]
    fns = [rwkvq.GroupedQmv(c[0], c[1], gs, bits, out=c[2]).run for c in chunks]
    durs = launch_durations(torch, fns)
    chunk_bytes = [sum(weight_bytes(w[0].shape[0], x.shape[1]) for x, w in zip(c[0], c[1]))
                   for c in chunks]
    kernel_time = sum(durs)
    achieved = sum(chunk_bytes) / kernel_time / 1e9
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
                         "[65536,2048], M=1, 4-bit g64 bf16 scales/biases, grouped launch"),
            "weight_bytes_per_step": total_wbytes,
            "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
            "launches_per_step": len(chunks),
        },
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "qmv_kernel<4,bf16,NMC=1,RB=4>",
                     "avg_launch_us": round(kernel_time / len(durs) * 1e6, 2),
                     "bytes_per_launch": int(sum(chunk_bytes) / len(chunk_bytes))},
    }

    if not args.no_extra:
        extra = {}
        extra["quantize_gbs"] = round(quant_gbs, 1)
        # M=8 sweep
        xs8 = [torch.randn(8, x.shape[1], device=dev).to(torch.bfloat16) for x in xs]
        outs8 = [torch.empty(8, w[0].shape[0], dtype=torch.bfloat16, device=dev) for w in ws]
        plan8 = rwkvq.GroupedQmv(xs8, ws, gs, bits, out=outs8)
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
        # prefill GEMM, config 3 at M=4096
        pre = {}
        tot_flops, tot_t = 0.0, 0.0
        for R, K in ((2560, 2560), (10240, 2560), (2560, 10240)):
            g = torch.Generator(device=dev).manual_seed(3_000_000 + R)
            w = (torch.randn(R, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
            wq, s, b = rwkvq.quantize(w, gs, bits)
            x = torch.randn(4096, K, device=dev).to(torch.bfloat16)
            t = time_region(torch, lambda: rwkvq.quantized_matmul(x, wq, s, b, True, gs, bits),
                            max(5, args.steps // 2), 2)
            fl = 2.0 * 4096 * R * K
            pre[f"{R}x{K}"] = round(fl / t / 1e12, 1)
            tot_flops += fl
            tot_t += t
            # transposed (QLoRA backward)
            dy = torch.randn(4096, R, device=dev).to(torch.bfloat16)
            tn = time_region(torch, lambda: rwkvq.quantized_matmul(dy, wq, s, b, False, gs, bits),
                             max(5, args.steps // 2), 2)
            pre[f"{R}x{K}_transposed"] = round(fl / tn / 1e12, 1)
            del w
        agg = tot_flops / tot_t / 1e12
        extra["prefill_qmm_m4096"] = {"tflops": round(agg, 1),
                                      "frac_of_bf16_peak": round(agg / BF16_PEAK_TFLOPS, 4),
                                      "per_shape_tflops": pre}
        result["extra"] = extra

    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(torch, args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
