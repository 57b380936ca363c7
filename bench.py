"""Benchmark of the IQ4_XS x Q8_1 mul_mat path on one MI355X.

Workload (the headline metric's configuration): the 27B-class decode linear
set at batch 1 -- q_proj 5120->8192, k_proj/v_proj 5120->1024, o_proj
8192->5120, gate_proj/up_proj 5120->17408, down_proj 17408->5120 -- each run
as its own quantise + GEMV through the C ABI.  One step = the seven
projections of one layer.  `--layers` distinct layer copies (default 16 =
3.07 GB of IQ4_XS) are generated on the device and rotated, so the 256 MB
Infinity Cache cannot serve repeats: every step streams its weights from HBM.
Steps are captured once into a HIP graph and replayed.

value = algorithmic bytes per step (sum of N*K*136/256 + 4K + 4N over the
seven GEMVs) / time per step.  roofline = the GEMV kernel alone: the same
bytes over its average launch duration from HIP event pairs around each
launch.  gemm = the int8-MFMA GEMM at M=512 on the same shapes, 2*M*N*K over
kernel time.  cpu_baseline = the reference's own FP64 oracle
(kernels/matmul_iq4xs/ref_cpu.cpp, compiled into oracle/_ref) -- or this
repository's restatement where that is absent -- on one host core.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "IQ4_XS GEMV HBM GB/s (% of 8 TB/s) bs=1; GEMM int8 TOPS (% MFMA peak) bs=512"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA, 5.0 POP/s
SHAPES = [("q_proj", 5120, 8192), ("k_proj", 5120, 1024), ("v_proj", 5120, 1024), ("o_proj", 8192, 5120),
          ("gate_proj", 5120, 17408), ("up_proj", 5120, 17408), ("down_proj", 17408, 5120)]
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_bs1_traffic.json")


def gemv_bytes(K: int, N: int, b: int = 1) -> int:
    return N * K * 136 // 256 + b * K * 4 + b * N * 4


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1024)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--layers", type=int, default=16)
    ap.add_argument("--gemm-m", type=int, default=512)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    return ap.parse_args()


def cpu_baseline(seconds: float) -> dict:
    """FP64 oracle GEMVs of one layer's seven projections on one host core,
    repeated until `seconds` elapse (bounded sample of the same workload)."""
    import numpy as np

    from oracle.oracle import Oracle, RefCpu, ref_available

    orc = Oracle()
    kind = "reference" if ref_available() else "port"
    fn = RefCpu().gemv_fp64 if kind == "reference" else orc.gemv_fp64
    inputs = []
    for i, (_, K, N) in enumerate(SHAPES):
        inputs.append((orc.gen_weights(K, N, seed=1000 + i), orc.gen_activations(K, seed=2000 + i), K, N))
    done_bytes, passes, t0 = 0, 0, time.perf_counter()
    while True:
        for W, x, K, N in inputs:
            fn(W, x, K, N)
            done_bytes += gemv_bytes(K, N)
        passes += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    cpu = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            cpu = next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
    except (OSError, StopIteration):
        pass
    return {"value": round(done_bytes / el / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": f"{passes} pass(es) of the 7 bs=1 projection GEMVs of one layer "
                      f"({sum(gemv_bytes(K, N) for _, K, N in SHAPES) / 1e6:.1f} MB each), FP64 oracle "
                      f"{'kernels/matmul_iq4xs/ref_cpu.cpp' if kind == 'reference' else 'oracle/iq4xs_oracle.c'}, "
                      f"{el:.1f} s on '{cpu}' ({os.cpu_count()} logical cpus visible)",
            "ms_per_step": round(el / passes * 1e3, 2)}


def main() -> int:
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the IQ4_XS path has no multi-GPU mode in this build "
              "(rows shard independently; see DESIGN.md). Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    from __graft_entry__ import load_package

    pkg = load_package()
    L = pkg.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream()  # default priority
    torch.cuda.set_stream(stream)
    s = stream.cuda_stream

    # ---- resident inputs -------------------------------------------------
    layers = []
    for l in range(args.layers):
        ws_list = []
        for i, (name, K, N) in enumerate(SHAPES):
            W = torch.empty(N * K // 256 * 136, dtype=torch.uint8, device=dev)
            L.check("iq4xs_fill_synthetic_weights", W.data_ptr(), N * K // 256, 42, (l * 7 + i) << 24, s)
            ws_list.append(W)
        layers.append(ws_list)
    xs = [pkg.synthetic_activations(K, seed=100 + i, device=dev) for i, (_, K, _) in enumerate(SHAPES)]
    ys = [torch.empty(N, device=dev) for (_, _, N) in SHAPES]
    wss = [torch.empty(L.iq4xs_workspace_bytes(K, 1), dtype=torch.uint8, device=dev) for (_, K, _) in SHAPES]
    torch.cuda.synchronize()

    def one_step(l: int) -> None:
        for i, (_, K, N) in enumerate(SHAPES):
            L.check("iq4xs_mul_mat", layers[l][i].data_ptr(), xs[i].data_ptr(), ys[i].data_ptr(), K, N, 1,
                    pkg.LAYOUT_MK, wss[i].data_ptr(), wss[i].numel(), s)

    step_bytes = sum(gemv_bytes(K, N) for _, K, N in SHAPES)

    # ---- whole-step timing: graph of one rotation over all layers ----------
    launch = "eager"
    graph = None
    if not args.no_graph:
        try:
            for l in range(args.layers):
                one_step(l)  # warm every code path before capture
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for l in range(args.layers):
                    one_step(l)
            launch = "hipgraph"
        except Exception as e:  # capture unsupported: fall back to eager launches
            print(f"[bench] graph capture failed ({e}); timing eager launches", file=sys.stderr)
            graph = None
    reps = max(1, -(-args.steps // args.layers))
    steps = reps * args.layers
    warm_reps = max(1, -(-args.warmup // args.layers))

    def run_rotation() -> None:
        if graph is not None:
            graph.replay()
        else:
            for l in range(args.layers):
                one_step(l)

    for _ in range(warm_reps):
        run_rotation()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(reps):
        run_rotation()
    t1.record(stream)
    torch.cuda.synchronize()
    ms_total = t0.elapsed_time(t1)
    ms_per_step = ms_total / steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    # ---- GEMV kernel alone: event pair around every launch ----------------
    ev_pairs = []
    for l in range(args.layers):
        for i, (_, K, N) in enumerate(SHAPES):
            L.check("iq4xs_quantize_q8_1", xs[i].data_ptr(), K, 1, pkg.LAYOUT_MK, wss[i].data_ptr(), wss[i].numel(), s)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            L.check("iq4xs_mul_mat_q8_1", layers[l][i].data_ptr(), wss[i].data_ptr(), ys[i].data_ptr(), K, N, 1,
                    pkg.LAYOUT_MK, pkg.PATH_GEMV, s)
            b.record(stream)
            ev_pairs.append((i, a, b))
    torch.cuda.synchronize()
    per_shape_us = {name: [] for name, _, _ in SHAPES}
    for i, a, b in ev_pairs:
        per_shape_us[SHAPES[i][0]].append(a.elapsed_time(b) * 1e3)
    gemv_us = sum(sum(v) for v in per_shape_us.values())
    gemv_launches = len(ev_pairs)
    achieved = step_bytes * args.layers / (gemv_us * 1e-6) / 1e9
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    # ---- GEMM at M = gemm_m on the same shapes -----------------------------
    M = args.gemm_m
    gemm_ops, gemm_us, gemm_shape_us = 0, 0.0, {}
    for i, (name, K, N) in enumerate(SHAPES):
        X = pkg.synthetic_activations(K * M, seed=300 + i, device=dev)
        ws = pkg.quantize_q8_1(X, K, M)
        Y = torch.empty((M, N), device=dev)
        W = layers[0][i]
        for _ in range(3):
            pkg.mul_mat_q8_1(W, ws, K, N, M, out=Y)
        times = []
        for r in range(10):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            pkg.mul_mat_q8_1(layers[r % args.layers][i], ws, K, N, M, out=Y)
            b.record(stream)
            times.append((a, b))
        torch.cuda.synchronize()
        us = sorted(a.elapsed_time(b) * 1e3 for a, b in times)[len(times) // 2]
        gemm_shape_us[name] = round(us, 2)
        gemm_ops += 2 * M * N * K
        gemm_us += us
        del X, ws, Y
    gemm_tops = gemm_ops / (gemm_us * 1e-6) / 1e12

    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm_reps * args.layers,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded IQ4_XS weights d~U(0.005,0.02), ls~U{0..63}, codes~U{0..15}; x~N(0,1)), "
                "generated on the device",
        "config": {"workload": "qwen27b-class decode linear set, bs=1: 7 projection GEMVs per step "
                               "(quantise + GEMV each), weights HBM-resident",
                   "shapes_KxN": {n: [K, N] for n, K, N in SHAPES}, "batch": 1,
                   "layers_rotated": args.layers, "weight_bytes_resident": step_bytes * args.layers,
                   "launch": launch, "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "gemv_iq4xs_kernel<1,2,false>",
                     "avg_launch_us": round(gemv_us / gemv_launches, 3),
                     "per_shape_avg_us": {k: round(sum(v) / len(v), 3) for k, v in per_shape_us.items()}},
        "gemm": {"M": M, "tops": round(gemm_tops, 2), "peak_tops": INT8_PEAK_TOPS,
                 "frac": round(gemm_tops / INT8_PEAK_TOPS, 4), "per_shape_us": gemm_shape_us,
                 "kernel": "gemm_iq4xs_mfma_kernel<false>"},
        "cpu_baseline": cpu,
        "host": platform.node(),
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
