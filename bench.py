"""Benchmark of the IQ4_XS x Q8_1 mul_mat path on one MI355X.

Workload (the headline metric's configuration): the 27B-class decode linear
set at batch 1 -- q_proj 5120->8192, k_proj/v_proj 5120->1024, o_proj
8192->5120, gate_proj/up_proj 5120->17408, down_proj 17408->5120 -- each run
as its own call of the C ABI (fp32 activations in, fp32 outputs out: the Q8_1
quantisation is part of the call).  One step = the seven projections of one
layer.  `--layers` distinct layer copies (default 16 = 3.07 GB of IQ4_XS) are
generated on the device and rotated, so the 256 MB Infinity Cache cannot
serve repeats: every step streams its weights from HBM.  Consecutive steps
walk the copies in rotation order; the --warmup untimed steps and then the
--steps timed steps are each captured as HIP graphs of up to 64 consecutive
steps (calls back to back, as a decode chain captures its layers) and
replayed, so exactly that many steps run.

value     algorithmic bytes per step (sum of N*K*136/256 + 4K + 4N over the
          seven GEMVs) / time per step.
roofline  the GEMV kernel alone, on prequantised Q8_1 activations: a graph of
          the seven GEMV launches of every layer copy (no quantiser), timed
          with HIP events on the launch stream; achieved = the same
          algorithmic bytes / average launch duration.
dequant   IQ4_XS -> fp32 (dequant_iq4xs_gpu) over the seven weight matrices.
extra     bs = 2, 4, 8 (the same GEMV-only measurement with 1 % x20
          outliers) and the matrix-core GEMM at M = 512 and 2048 (2*M*N*K over
          the average of back-to-back launches rotated over the layer copies).
producers iq4xs_rms_norm_q8_1 (K=5120, with residual) and iq4xs_swiglu_q8_1
          (K=17408) at M = 1 and 512.
model_stream  64 distinct layers resident (12.30 GB) run as a data chain
          through the producers: one bs=1 token (graph) and one bs=512 pass.
cpu_baseline  the reference's own FP64 oracle (kernels/matmul_iq4xs/ref_cpu.cpp,
          compiled into oracle/_ref) -- or this repository's restatement where
          that is absent -- on one host core, on a bounded sample; beside it
          (int8_host) the integer path on the host's cores (Q8_1 quantiser +
          AVX2 int8 dots, OpenMP), for half that time.
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
    ap.add_argument("--roofline-reps", type=int, default=32, help="replays of the GEMV-only rotation graph")
    ap.add_argument("--gemm-m", type=int, nargs="*", default=[512, 2048])
    ap.add_argument("--batches", type=int, nargs="*", default=[2, 4, 8])
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--repeats", type=int, default=20, help="replays timed one by one for median / p95")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--model-layers", type=int, default=64,
                    help="whole-model weight stream: distinct resident layers (0 = skip)")
    ap.add_argument("--rows", choices=["gemv", "gemv_dp4a", "gemm_wmma"], default=None,
                    help="print the reference bench's per-shape JSON rows for this op (harness/bench_rows: "
                         "bench_gemv.cpp / bench_gemv_dp4a.cpp / bench_gemm_wmma.cpp keys, bench.h statistics) "
                         "and exit")
    ap.add_argument("--rows-runs", type=int, default=10, help="runs per row in --rows mode (the reference's 10)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="also run a plain device copy of MIB MiB (4 times): the known-size reference that "
                         "scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    return ap.parse_args()


def cpu_baseline(seconds: float) -> dict:
    """FP64 oracle GEMVs of one layer's seven projections on one host core,
    repeated until `seconds` elapse (bounded sample of the same workload)."""
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
    # the integer path on the host: Q8_1 quantiser + int8 sub-block dots
    # (AVX2) on every allowed core, same seven GEMVs, output equal to the
    # kernel semantics
    threads = max(1, min(os.cpu_count() or 1, int(os.environ.get("OMP_NUM_THREADS") or (os.cpu_count() or 1))))
    i_bytes, i_passes, t1 = 0, 0, time.perf_counter()
    while True:
        for W, x, K, N in inputs:
            orc.gemv_q8_1_host(W, x, K, N, threads)
            i_bytes += gemv_bytes(K, N)
        i_passes += 1
        i_el = time.perf_counter() - t1
        if i_el >= seconds / 2:
            break
    step_mb = sum(gemv_bytes(K, N) for _, K, N in SHAPES) / 1e6
    return {"value": round(done_bytes / el / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": f"{passes} pass(es) of the 7 bs=1 projection GEMVs of one layer "
                      f"({step_mb:.1f} MB each), FP64 oracle "
                      f"{'kernels/matmul_iq4xs/ref_cpu.cpp' if kind == 'reference' else 'oracle/iq4xs_oracle.c'}, "
                      f"{el:.1f} s on '{cpu}' ({os.cpu_count()} logical cpus visible)",
            "ms_per_step": round(el / passes * 1e3, 2),
            "int8_host": {"value": round(i_bytes / i_el / 1e9, 4), "unit": "GB/s", "cores": threads, "kind": "port",
                          "ms_per_step": round(i_el / i_passes * 1e3, 2),
                          "sample": f"{i_passes} pass(es) of the same 7 GEMVs through oracle orc_gemv_q8_1_host "
                                    f"(Q8_1 quantiser + AVX2 int8 sub-block dots, OpenMP over rows, {threads} "
                                    f"threads; output bit-identical to the kernel semantics), {i_el:.1f} s"}}


def spread(samples, name: str) -> dict:
    """Median and 95th percentile of repeated timings (one graph replay each)."""
    v = sorted(samples)
    p95 = v[min(len(v) - 1, int(0.95 * len(v) + 0.5) - 1)] if v else None
    return {"repeats": len(v), f"median_{name}": round(v[len(v) // 2], 4), f"p95_{name}": round(p95, 4)}


class Timer:
    """Events recorded on the launch stream around a callable run `reps` times."""

    def __init__(self, torch, stream):
        self.torch, self.stream = torch, stream

    def __call__(self, fn, reps: int) -> float:
        torch = self.torch
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(self.stream)
        for _ in range(reps):
            fn()
        b.record(self.stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3  # microseconds


def capture(torch, stream, fn, use_graph: bool):
    """A graph of fn (one warm run first), or fn itself when graphs are off or fail."""
    fn()
    torch.cuda.synchronize()
    if not use_graph:
        return fn, "eager"
    try:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            fn()
        g.replay()
        torch.cuda.synchronize()
        return g.replay, "hipgraph"
    except Exception as e:  # capture unsupported: fall back to eager launches
        print(f"[bench] graph capture failed ({e}); timing eager launches", file=sys.stderr)
        return fn, "eager"


MODEL_GAIN = 1.0 / 1145.0  # rms gains that keep the synthetic chain inside fp16's range (see ModelChain)
MODEL_EPS = 1e-6
MODEL_SEED = 42


def model_weight_first_block(l: int, i: int) -> int:
    """Seed offset of projection i of model layer l (distinct from the rotated layer copies)."""
    return (1 << 40) + ((l * 7 + i) << 24)


def make_model_weights(torch, L, n_layers: int, stream, dev):
    """n_layers distinct layers of the seven projections, generated on the device."""
    s = stream.cuda_stream
    weights = []
    for l in range(n_layers):
        row = []
        for i, (_, K, N) in enumerate(SHAPES):
            W = torch.empty(N * K // 256 * 136, dtype=torch.uint8, device=dev)
            L.check("iq4xs_fill_synthetic_weights", W.data_ptr(), N * K // 256, MODEL_SEED,
                    model_weight_first_block(l, i), s)
            row.append(W)
        weights.append(row)
    return weights


class ModelChain:
    """The whole-model weight stream as a data chain over resident layers: each
    layer's output feeds the next layer's Q8_1 producer.  Per layer (row m of
    every tensor is one token; bs=1 is M=1, prefill M=512):
        h += down_prev; A = Q8_1(rmsnorm(h) * g_attn)       iq4xs_rms_norm_q8_1
        q, k, v = W_q A, W_k A, W_v A                       iq4xs_mul_mat_q8_1
        o = W_o Q8_1(q)      iq4xs_mul_mat (attention itself is outside
                              this path: its output has q's shape and takes
                              its place)
        h += o; A = Q8_1(rmsnorm(h) * g_ffn)
        gate, up = W_gate A, W_up A
        C = Q8_1(silu(gate) * up)                           iq4xs_swiglu_q8_1
        down_prev = W_down C
    variant "grouped" runs q,k,v and gate,up as one iq4xs_mul_mat_q8_1_group
    launch each; "fused" (M = 1) runs each rms norm and the group after it as
    one iq4xs_rms_norm_mul_mat_group launch, which writes h into the other of
    two buffers (it has no in-place form); "fused_swiglu" (M = 1) is "fused"
    with the FFN's norm, gate/up and SwiGLU as one
    iq4xs_rms_norm_mul_mat_swiglu launch writing S = silu(gate) * up in fp32,
    and down as iq4xs_mul_mat on S (the quantiser in the GEMV's prologue):
    four launches per layer.  Every variant computes the same bits.  The norm gains are 1/1145 so that the synthetic weights (rms ~16
    per element) keep every activation well inside the fp16 range of the Q8_1
    scale.

    check (optional) is called after every stage with the stage's name and its
    inputs and outputs (torch tensors, copies taken before in-place updates),
    for the parity tests; the chain synchronises around it."""

    STAGES = ("rms_attn", "qkv", "o", "rms_ffn", "gate_up", "swiglu", "down")

    def __init__(self, torch, pkg, L, weights, M: int, stream, variant: str = "plain", seed: int = 700):
        import ctypes

        assert variant in ("plain", "grouped", "fused", "fused_swiglu") and (variant in ("plain", "grouped") or M == 1)
        self.torch, self.pkg, self.L, self.weights, self.M, self.variant = torch, pkg, L, weights, M, variant
        self.s = stream.cuda_stream
        dev = weights[0][0].device
        self.H_DIM, self.Q_DIM, self.FF_DIM = SHAPES[0][1], SHAPES[0][2], SHAPES[4][2]
        self.gain = torch.full((self.H_DIM,), MODEL_GAIN, device=dev)
        self.h = pkg.synthetic_activations(M * self.H_DIM, seed=seed, device=dev)
        self.h_alt = torch.empty_like(self.h)  # the fused norm writes h into the other buffer
        self.S = torch.empty((M, SHAPES[4][2]), device=dev)  # fused_swiglu: silu(gate) * up
        self.bufs = {name: torch.zeros((M, N), device=dev) for name, _, N in SHAPES}
        self.wsA = torch.empty(L.iq4xs_workspace_bytes(self.H_DIM, M), dtype=torch.uint8, device=dev)
        self.wsB = torch.empty(L.iq4xs_workspace_bytes(self.Q_DIM, M), dtype=torch.uint8, device=dev)
        self.wsC = torch.empty(L.iq4xs_workspace_bytes(self.FF_DIM, M), dtype=torch.uint8, device=dev)

        def group_args(Ws, names):
            n = len(Ws)
            return (n, (ctypes.c_void_p * n)(*[w.data_ptr() for w in Ws]),
                    (ctypes.c_void_p * n)(*[self.bufs[nm].data_ptr() for nm in names]),
                    (ctypes.c_int64 * n)(*[self.bufs[nm].shape[1] for nm in names]))

        self.gargs = [(group_args(w[0:3], ["q_proj", "k_proj", "v_proj"]), group_args(w[4:6], ["gate_proj", "up_proj"]))
                      for w in weights]

    def _mm(self, W, ws, name, K, N):
        self.L.check("iq4xs_mul_mat_q8_1", W.data_ptr(), ws.data_ptr(), self.bufs[name].data_ptr(), K, N, self.M,
                     self.pkg.LAYOUT_MK, self.pkg.PATH_AUTO, self.s)

    def _group(self, l, which, ws, K):
        n, wp, yp, nn = self.gargs[l][which]
        self.L.check("iq4xs_mul_mat_q8_1_group", n, wp, yp, nn, ws.data_ptr(), K, self.M, self.pkg.LAYOUT_MK, self.s)

    def _rms_group(self, l, which, X, R, H):
        n, wp, yp, nn = self.gargs[l][which]
        self.L.check("iq4xs_rms_norm_mul_mat_group", n, wp, yp, nn, X.data_ptr(), R.data_ptr(), H.data_ptr(),
                     self.gain.data_ptr(), MODEL_EPS, self.H_DIM, self.s)

    def _rms(self, R):
        self.L.check("iq4xs_rms_norm_q8_1", self.h.data_ptr(), R.data_ptr(), self.h.data_ptr(), self.gain.data_ptr(),
                     MODEL_EPS, self.H_DIM, self.M, self.wsA.data_ptr(), self.wsA.numel(), self.s)

    def layer(self, l: int, check=None) -> None:
        torch, Wl, b = self.torch, self.weights[l], self.bufs
        snap = (lambda t: t.clone()) if check else (lambda t: None)

        def done(stage, **kw):
            if check:
                torch.cuda.synchronize()
                check(l, stage, **kw)

        # attention norm -> q, k, v
        h_in, r_in = snap(self.h), snap(b["down_proj"])
        if self.variant in ("fused", "fused_swiglu"):  # h + down_prev -> h_alt, norm, q/k/v: one launch
            self._rms_group(l, 0, self.h, b["down_proj"], self.h_alt)
            done("rms_qkv_fused", h_in=h_in, r_in=r_in, h_out=self.h_alt, q=b["q_proj"], k=b["k_proj"],
                 v=b["v_proj"])
        else:
            self._rms(b["down_proj"])
            done("rms_attn", h_in=h_in, r_in=r_in, h_out=self.h, ws=self.wsA)
            if self.variant == "grouped":
                self._group(l, 0, self.wsA, self.H_DIM)
            else:
                for i in range(3):
                    self._mm(Wl[i], self.wsA, *SHAPES[i])
            done("qkv", ws=self.wsA, q=b["q_proj"], k=b["k_proj"], v=b["v_proj"])
        # o from fp32 q (the stand-in for attention's output): iq4xs_mul_mat quantises it, in the GEMV's
        # prologue at bs=1 (K = 8192), in its own launch for prefill
        self.L.check("iq4xs_mul_mat", Wl[3].data_ptr(), b["q_proj"].data_ptr(), b["o_proj"].data_ptr(), self.Q_DIM,
                     SHAPES[3][2], self.M, self.pkg.LAYOUT_MK, self.wsB.data_ptr(), self.wsB.numel(), self.s)
        done("o", x=b["q_proj"], o=b["o_proj"])
        # FFN norm -> gate, up
        if self.variant == "fused_swiglu":  # h_alt + o -> h, norm, gate/up, S = silu(gate) * up: one launch
            h_in, r_in = snap(self.h_alt), snap(b["o_proj"])
            self.L.check("iq4xs_rms_norm_mul_mat_swiglu", Wl[4].data_ptr(), Wl[5].data_ptr(), self.FF_DIM,
                         self.h_alt.data_ptr(), b["o_proj"].data_ptr(), self.h.data_ptr(), self.gain.data_ptr(),
                         MODEL_EPS, self.H_DIM, b["gate_proj"].data_ptr(), b["up_proj"].data_ptr(),
                         self.S.data_ptr(), self.s)
            done("rms_gate_up_swiglu", h_in=h_in, r_in=r_in, h_out=self.h, gate=b["gate_proj"], up=b["up_proj"],
                 s=self.S)
            self.L.check("iq4xs_mul_mat", Wl[6].data_ptr(), self.S.data_ptr(), b["down_proj"].data_ptr(), self.FF_DIM,
                         SHAPES[6][2], self.M, self.pkg.LAYOUT_MK, self.wsC.data_ptr(), self.wsC.numel(), self.s)
            done("down_from_s", x=self.S, down=b["down_proj"])
            return
        if self.variant == "fused":  # h_alt + o -> h, norm, gate/up: one launch
            h_in, r_in = snap(self.h_alt), snap(b["o_proj"])
            self._rms_group(l, 1, self.h_alt, b["o_proj"], self.h)
            done("rms_gate_up_fused", h_in=h_in, r_in=r_in, h_out=self.h, gate=b["gate_proj"], up=b["up_proj"])
        else:
            h_in, r_in = snap(self.h), snap(b["o_proj"])
            self._rms(b["o_proj"])
            done("rms_ffn", h_in=h_in, r_in=r_in, h_out=self.h, ws=self.wsA)
            if self.variant == "grouped":
                self._group(l, 1, self.wsA, self.H_DIM)
            else:
                self._mm(Wl[4], self.wsA, *SHAPES[4])
                self._mm(Wl[5], self.wsA, *SHAPES[5])
            done("gate_up", ws=self.wsA, gate=b["gate_proj"], up=b["up_proj"])
        self.L.check("iq4xs_swiglu_q8_1", b["gate_proj"].data_ptr(), b["up_proj"].data_ptr(), self.FF_DIM, self.M,
                     self.wsC.data_ptr(), self.wsC.numel(), self.s)
        done("swiglu", gate=b["gate_proj"], up=b["up_proj"], ws=self.wsC)
        self._mm(Wl[6], self.wsC, *SHAPES[6])
        done("down", ws=self.wsC, down=b["down_proj"])

    def run(self, n_layers: int | None = None, check=None) -> None:
        for l in range(len(self.weights) if n_layers is None else n_layers):
            self.layer(l, check)

    def state(self) -> list:
        """The buffers a token leaves behind: h (the residual stream) and every projection output."""
        h = self.h
        return [h] + [self.bufs[name] for name, _, _ in SHAPES]

    def finite(self) -> bool:
        self.torch.cuda.synchronize()
        ts = self.state() + ([self.h_alt] if self.variant in ("fused", "fused_swiglu") else [])
        ts += [self.S] if self.variant == "fused_swiglu" else []
        return all(bool(self.torch.isfinite(t).all()) for t in ts)


def model_stream(torch, pkg, L, stream, timer, args, use_graph) -> dict:
    """`--model-layers` distinct layers of the seven projections resident at
    once (64 layers = 12.30 GB), run as ModelChain's data chain: one bs=1
    token per variant (graph) and one bs=512 pass (plain and grouped).
    Bandwidth is charged for the projections' bytes only; the time includes
    the producers."""
    dev = torch.device("cuda:0")
    weights = make_model_weights(torch, L, args.model_layers, stream, dev)
    total_w = sum(N * K // 256 * 136 for _, K, N in SHAPES) * args.model_layers
    layer_bytes = sum(gemv_bytes(K, N) for _, K, N in SHAPES)
    out = {"layers": args.model_layers, "weight_bytes": total_w, "chain": "rmsnorm+residual -> q,k,v; q -> o; "
           "rmsnorm+residual -> gate,up; swiglu -> down (producers write Q8_1)"}
    notes = {"bs1": None,
             "bs1_grouped": "same chain; q,k,v and gate,up each one iq4xs_mul_mat_q8_1_group launch",
             "bs1_rms_fused": "same chain; each rms norm and the q,k,v / gate,up group after it are one "
                              "iq4xs_rms_norm_mul_mat_group launch",
             "bs1_rms_swiglu_fused": "same chain; as bs1_rms_fused, with the FFN's norm, gate/up and swiglu one "
                                     "iq4xs_rms_norm_mul_mat_swiglu launch (fp32 silu(gate)*up) and down quantising "
                                     "it in its prologue: 4 launches per layer"}
    for key, variant in (("bs1", "plain"), ("bs1_grouped", "grouped"), ("bs1_rms_fused", "fused"),
                         ("bs1_rms_swiglu_fused", "fused_swiglu")):
        chain = ModelChain(torch, pkg, L, weights, 1, stream, variant)
        run, launch = capture(torch, stream, chain.run, use_graph)
        timer(run, 2)
        us = timer(run, 8) / 8
        gbs = layer_bytes * args.model_layers / (us * 1e-6) / 1e9
        out[key] = {"us_per_token": round(us, 1), "GBps": round(gbs, 1), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                    "tokens_per_s_upper_bound": round(1e6 / us, 1), "finite": chain.finite()}
        if key == "bs1":
            out[key]["launch"] = launch
        else:
            out[key]["note"] = notes[key]
        del run, chain
    M = 512
    ops = sum(2 * M * N * K for _, K, N in SHAPES) * args.model_layers
    for key, variant in (("bs512", "plain"), ("bs512_grouped", "grouped")):
        chain = ModelChain(torch, pkg, L, weights, M, stream, variant)
        chain.run()
        torch.cuda.synchronize()
        us = timer(chain.run, 1)
        out[key] = {"ms_per_pass": round(us / 1e3, 2), "tops": round(ops / (us * 1e-6) / 1e12, 1),
                    "frac_of_int8_peak": round(ops / (us * 1e-6) / 1e12 / INT8_PEAK_TOPS, 4),
                    "tokens_per_s": round(M / (us * 1e-6), 1), "finite": chain.finite()}
        if variant == "plain":
            out[key]["includes"] = "the producers and the q re-quantisation of every layer"
        else:
            out[key]["note"] = "same chain; q,k,v and gate,up each one iq4xs_mul_mat_q8_1_group launch"
        del chain
    return out


def main() -> int:
    args = parse()
    if args.rows:  # the reference-format rows come from the C++ harness, a child process
        import subprocess

        harness = os.path.join(ROOT, "qwen_3.8_27b_optimizations_amd", "harness", "_build", "bench_rows")
        if not os.path.exists(harness):
            print(f"{harness} is missing: build it with __graft_entry__.build()", file=sys.stderr)
            return 2
        return subprocess.run([harness, "--op", args.rows, "--runs", str(args.rows_runs)]).returncode
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the IQ4_XS path has no multi-GPU mode in this build "
              "(rows shard independently across GPUs; the sharding design is documented with the "
              "library). Run with --gpus 1.", file=sys.stderr)
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
    timer = Timer(torch, stream)
    use_graph = not args.no_graph

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
    step_bytes = sum(gemv_bytes(K, N) for _, K, N in SHAPES)
    n_launch = args.layers * len(SHAPES)

    # ---- roofline: the GEMV kernel alone on prequantised activations --------
    def gemv_rotation(wsb, yb, M) -> None:
        for l in range(args.layers):
            for i, (_, K, N) in enumerate(SHAPES):
                L.check("iq4xs_mul_mat_q8_1", layers[l][i].data_ptr(), wsb[i].data_ptr(), yb[i].data_ptr(), K, N,
                        M, pkg.LAYOUT_MK, pkg.PATH_GEMV, s)

    for i, (_, K, _) in enumerate(SHAPES):
        L.check("iq4xs_quantize_q8_1", xs[i].data_ptr(), K, 1, pkg.LAYOUT_MK, wss[i].data_ptr(), wss[i].numel(), s)
    grun, _ = capture(torch, stream, lambda: gemv_rotation(wss, ys, 1), use_graph)
    timer(grun, 2)
    gemv_us = timer(grun, args.roofline_reps) / args.roofline_reps
    launch_stats = spread([timer(grun, 1) / n_launch for _ in range(args.repeats)], "launch_us")
    avg_launch_us = gemv_us / n_launch
    achieved = step_bytes * args.layers / (gemv_us * 1e-6) / 1e9
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    # ---- grouped decode set: q/k/v and gate/up as one launch each ----------
    import ctypes

    def group_args(Ws, Ys):
        n = len(Ws)
        return (n, (ctypes.c_void_p * n)(*[w.data_ptr() for w in Ws]), (ctypes.c_void_p * n)(*[y.data_ptr() for y in Ys]),
                (ctypes.c_int64 * n)(*[y.numel() for y in Ys]))

    groups = [(group_args(layers[l][0:3], ys[0:3]), group_args(layers[l][4:6], ys[4:6])) for l in range(args.layers)]

    def grouped_rotation(wsb, yb, M, grp) -> None:
        for l in range(args.layers):
            (n, wp, yp, nn), (n2, wp2, yp2, nn2) = grp[l]
            L.check("iq4xs_mul_mat_q8_1_group", n, wp, yp, nn, wsb[0].data_ptr(), SHAPES[0][1], M, pkg.LAYOUT_MK, s)
            L.check("iq4xs_mul_mat_q8_1", layers[l][3].data_ptr(), wsb[3].data_ptr(), yb[3].data_ptr(), SHAPES[3][1],
                    SHAPES[3][2], M, pkg.LAYOUT_MK, pkg.PATH_GEMV, s)
            L.check("iq4xs_mul_mat_q8_1_group", n2, wp2, yp2, nn2, wsb[4].data_ptr(), SHAPES[4][1], M, pkg.LAYOUT_MK,
                    s)
            L.check("iq4xs_mul_mat_q8_1", layers[l][6].data_ptr(), wsb[6].data_ptr(), yb[6].data_ptr(), SHAPES[6][1],
                    SHAPES[6][2], M, pkg.LAYOUT_MK, pkg.PATH_GEMV, s)

    gr_run, _ = capture(torch, stream, lambda: grouped_rotation(wss, ys, 1, groups), use_graph)
    timer(gr_run, 2)
    gr_us = timer(gr_run, args.roofline_reps) / args.roofline_reps
    gr_gbs = step_bytes * args.layers / (gr_us * 1e-6) / 1e9
    grouped = {"GBps": round(gr_gbs, 1), "frac": round(gr_gbs / HBM_PEAK_GBS, 4),
               "us_per_layer": round(gr_us / args.layers, 2), "launches_per_layer": 4,
               "note": "iq4xs_mul_mat_q8_1_group: q,k,v in one launch, gate,up in one; o, down alone; "
                       "prequantised Q8_1, same rotation and byte count as the roofline leg"}
    del gr_run

    # ---- headline: whole steps (quantise + GEMV per projection) ------------
    # A step is the seven calls of one layer copy; consecutive steps walk the
    # 16 copies in rotation order.  The warm-up steps and the timed steps are
    # each captured as graphs of up to GRAPH_STEPS consecutive steps (the calls
    # back to back, as a decode chain captures its layers), so exactly --warmup
    # untimed and --steps timed steps run and no graph-launch boundary falls
    # between two steps except every GRAPH_STEPS.  Capturing runs each graph
    # once first: that priming pass is set-up, not warm-up.  The legs above
    # have already kept the GPU busy for ~0.1 s, so the clocks have settled
    # before the timed region.
    GRAPH_STEPS = 64

    def steps_fn(first: int, count: int):
        def run() -> None:
            for j in range(count):
                l = (first + j) % args.layers
                for i, (_, K, N) in enumerate(SHAPES):
                    L.check("iq4xs_mul_mat", layers[l][i].data_ptr(), xs[i].data_ptr(), ys[i].data_ptr(), K, N, 1,
                            pkg.LAYOUT_MK, wss[i].data_ptr(), wss[i].numel(), s)
        return run

    def step_graphs(first: int, count: int):
        caps = [capture(torch, stream, steps_fn(first + c0, min(GRAPH_STEPS, count - c0)), use_graph)
                for c0 in range(0, count, GRAPH_STEPS)]

        def run_all() -> None:
            for r, _ in caps:
                r()
        return run_all, caps[-1][1]

    warm_run = step_graphs(0, args.warmup)[0] if args.warmup > 0 else None
    timed_run, launch = step_graphs(args.warmup, args.steps)
    if warm_run is not None:
        timer(warm_run, 1)
    us_total = timer(timed_run, 1)
    ms_per_step = us_total / args.steps / 1e3
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    del warm_run, timed_run
    # spread: each sample times one rotation of back-to-back steps (one graph)
    rot_run = step_graphs(0, args.layers)[0]
    step_stats = spread([timer(rot_run, 1) / args.layers / 1e3 for _ in range(args.repeats)], "ms_per_step")
    del rot_run

    if args.copy_probe:
        src = torch.empty(args.copy_probe << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        src.fill_(1)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # ---- small batch (bs = 2, 4, 8), GEMV kernel on prequantised columns ----
    small = {}
    for M in args.batches:
        X = [pkg.synthetic_activations(K * M, seed=500 + M + i, outliers=True, device=dev)
             for i, (_, K, _) in enumerate(SHAPES)]
        wsb = [pkg.quantize_q8_1(X[i], K, M) for i, (_, K, _) in enumerate(SHAPES)]
        yb = [torch.empty((M, N), device=dev) for (_, _, N) in SHAPES]
        brun, _ = capture(torch, stream, lambda: gemv_rotation(wsb, yb, M), use_graph)
        timer(brun, 2)
        us = timer(brun, max(4, args.roofline_reps // 4)) / max(4, args.roofline_reps // 4)
        b_bytes = sum(gemv_bytes(K, N, M) for _, K, N in SHAPES) * args.layers
        small[str(M)] = {"GBps": round(b_bytes / (us * 1e-6) / 1e9, 1),
                         "frac": round(b_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                         "us_per_layer": round(us / args.layers, 2)}
        # the same rotation with q,k,v and gate,up each one grouped launch
        # (matrix-core matrices of one wave count share a launch)
        # group_args reads N from the outputs' element count: M rows of N
        bgroups = [(group_args(layers[l][0:3], [y[0] for y in yb[0:3]]),
                    group_args(layers[l][4:6], [y[0] for y in yb[4:6]])) for l in range(args.layers)]
        bgrun, _ = capture(torch, stream, lambda: grouped_rotation(wsb, yb, M, bgroups), use_graph)
        timer(bgrun, 2)
        gus = timer(bgrun, max(4, args.roofline_reps // 4)) / max(4, args.roofline_reps // 4)
        small[str(M)]["grouped"] = {"GBps": round(b_bytes / (gus * 1e-6) / 1e9, 1),
                                    "frac": round(b_bytes / (gus * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                                    "us_per_layer": round(gus / args.layers, 2)}
        del X, wsb, yb, brun, bgrun, bgroups

    # ---- IQ4_XS -> fp32 dequantiser (136 B in, 1024 B out per super-block) --
    dq_bytes, dq_us = 0, 0.0
    for i, (_, K, N) in enumerate(SHAPES):
        nblk = N * K // 256
        out = torch.empty(nblk * 256, dtype=torch.float32, device=dev)
        L.check("dequant_iq4xs_gpu", layers[0][i].data_ptr(), out.data_ptr(), nblk, 64, s)
        ctr = [1]

        def dq():
            L.check("dequant_iq4xs_gpu", layers[ctr[0] % args.layers][i].data_ptr(), out.data_ptr(), nblk, 64, s)
            ctr[0] += 1

        dq_us += timer(dq, 4) / 4
        dq_bytes += nblk * (136 + 1024)
        del out
    dequant = {"GBps": round(dq_bytes / (dq_us * 1e-6) / 1e9, 1),
               "frac_of_hbm_peak": round(dq_bytes / (dq_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
               "bytes_per_superblock": "136 read + 1024 written", "shapes": "the seven projections of one layer"}

    # ---- fused producers -> Q8_1 (decode M=1 and prefill M=512) ------------
    producers = {}
    H_DIM, FF_DIM, REPS = SHAPES[0][1], SHAPES[4][2], 32
    for M in (1, 512):
        X = pkg.synthetic_activations(M * H_DIM, seed=900, device=dev)
        R = pkg.synthetic_activations(M * H_DIM, seed=901, device=dev)
        Hh = torch.empty_like(X)
        gn = torch.ones(H_DIM, device=dev)
        G = pkg.synthetic_activations(M * FF_DIM, seed=902, device=dev)
        U = pkg.synthetic_activations(M * FF_DIM, seed=903, device=dev)
        wr = torch.empty(L.iq4xs_workspace_bytes(H_DIM, M), dtype=torch.uint8, device=dev)
        wg = torch.empty(L.iq4xs_workspace_bytes(FF_DIM, M), dtype=torch.uint8, device=dev)

        def rms_reps():
            for _ in range(REPS):
                L.check("iq4xs_rms_norm_q8_1", X.data_ptr(), R.data_ptr(), Hh.data_ptr(), gn.data_ptr(), 1e-6,
                        H_DIM, M, wr.data_ptr(), wr.numel(), s)

        def swiglu_reps():
            for _ in range(REPS):
                L.check("iq4xs_swiglu_q8_1", G.data_ptr(), U.data_ptr(), FF_DIM, M, wg.data_ptr(), wg.numel(), s)

        row = {}
        for name, fn, nbytes in (("rms_norm_q8_1", rms_reps, M * (H_DIM * 13 + H_DIM // 32 * 4)),
                                 ("swiglu_q8_1", swiglu_reps, M * (FF_DIM * 9 + FF_DIM // 32 * 4))):
            run_p, _ = capture(torch, stream, fn, use_graph)
            us = timer(run_p, 4) / (4 * REPS)
            row[name] = {"K": H_DIM if name == "rms_norm_q8_1" else FF_DIM, "us": round(us, 2),
                         "GBps": round(nbytes / (us * 1e-6) / 1e9, 1), "bytes": nbytes}
            del run_p
        producers[str(M)] = row
        del X, R, Hh, G, U, wr, wg
    producers["bytes"] = ("rms: x, residual read + h written (4 B each), codes 1 B + ds 4 B per 32; "
                          "swiglu: gate, up read (4 B each), codes + ds written")

    # ---- GEMM at M = 512 / 2048 on the same shapes -------------------------
    gemm = {}
    for M in args.gemm_m:
        ops, us_sum, per_shape = 0, 0.0, {}
        for i, (name, K, N) in enumerate(SHAPES):
            X = pkg.synthetic_activations(K * M, seed=300 + i, device=dev)
            ws = pkg.quantize_q8_1(X, K, M)
            Y = torch.empty((M, N), device=dev)
            nrep = 8 if M >= 2048 else 16
            for _ in range(2):
                pkg.mul_mat_q8_1(layers[0][i], ws, K, N, M, out=Y)
            ctr = [0]

            def one():
                pkg.mul_mat_q8_1(layers[ctr[0] % args.layers][i], ws, K, N, M, out=Y)
                ctr[0] += 1

            us = timer(one, nrep) / nrep
            per_shape[name] = round(us, 2)
            ops += 2 * M * N * K
            us_sum += us
            del X, ws, Y
        tops = ops / (us_sum * 1e-6) / 1e12
        gemm[str(M)] = {"tops": round(tops, 2), "frac": round(tops / INT8_PEAK_TOPS, 4), "per_shape_us": per_shape}
        # the same seven projections with q,k,v and gate,up as one grouped launch each
        import ctypes

        K0 = SHAPES[0][1]
        X = pkg.synthetic_activations(K0 * M, seed=300, device=dev)
        ws = pkg.quantize_q8_1(X, K0, M)
        Xo = pkg.synthetic_activations(SHAPES[3][1] * M, seed=303, device=dev)
        wso = pkg.quantize_q8_1(Xo, SHAPES[3][1], M)
        Xd = pkg.synthetic_activations(SHAPES[6][1] * M, seed=306, device=dev)
        wsd = pkg.quantize_q8_1(Xd, SHAPES[6][1], M)
        Ys = [torch.empty((M, N), device=dev) for (_, _, N) in SHAPES]

        def gargs(l, idx):
            n = len(idx)
            return (n, (ctypes.c_void_p * n)(*[layers[l][i].data_ptr() for i in idx]),
                    (ctypes.c_void_p * n)(*[Ys[i].data_ptr() for i in idx]),
                    (ctypes.c_int64 * n)(*[SHAPES[i][2] for i in idx]))

        ga = [(gargs(l, [0, 1, 2]), gargs(l, [4, 5])) for l in range(args.layers)]
        gctr = [0]

        def grouped_layer():
            l = gctr[0] % args.layers
            gctr[0] += 1
            (n, wp, yp, nn), (n2, wp2, yp2, nn2) = ga[l]
            L.check("iq4xs_mul_mat_q8_1_group", n, wp, yp, nn, ws.data_ptr(), K0, M, pkg.LAYOUT_MK, s)
            pkg.mul_mat_q8_1(layers[l][3], wso, SHAPES[3][1], SHAPES[3][2], M, out=Ys[3])
            L.check("iq4xs_mul_mat_q8_1_group", n2, wp2, yp2, nn2, ws.data_ptr(), K0, M, pkg.LAYOUT_MK, s)
            pkg.mul_mat_q8_1(layers[l][6], wsd, SHAPES[6][1], SHAPES[6][2], M, out=Ys[6])

        for _ in range(2):
            grouped_layer()
        nrep = 4 if M >= 2048 else 8
        g_us = timer(grouped_layer, nrep) / nrep
        gemm[str(M)]["grouped"] = {"tops": round(ops / (g_us * 1e-6) / 1e12, 2),
                                   "frac": round(ops / (g_us * 1e-6) / 1e12 / INT8_PEAK_TOPS, 4),
                                   "us_per_layer": round(g_us, 1),
                                   "note": "q,k,v and gate,up each one iq4xs_mul_mat_q8_1_group launch; o, down alone"}
        del X, ws, Xo, wso, Xd, wsd, Ys

    # ---- whole-model weight stream (64 distinct layers resident) -----------
    model = None
    if args.model_layers:
        del layers
        torch.cuda.synchronize()
        model = model_stream(torch, pkg, L, stream, timer, args, use_graph)

    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded IQ4_XS weights d~U(0.005,0.02), ls~U{0..63}, codes~U{0..15}; x~N(0,1)), "
                "generated on the device",
        "config": {"workload": "qwen27b-class decode linear set, bs=1: 7 projection GEMVs per step "
                               "(fp32 activations quantised to Q8_1 inside each call), weights HBM-resident",
                   "shapes_KxN": {n: [K, N] for n, K, N in SHAPES}, "batch": 1,
                   "layers_rotated": args.layers, "weight_bytes_resident": step_bytes * args.layers,
                   "launch": launch, "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
                   "step_spread": step_stats},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "iq4xs::gemv_tile_kernel<1, 2, false, false, false, 0> (bs=1, prequantised Q8_1)",
                     "avg_launch_us": round(avg_launch_us, 3), "launches_timed": n_launch * args.roofline_reps,
                     "launch_spread": launch_stats},
        "grouped_gemv": grouped,
        "small_batch_gemv": small,
        "gemm": {"peak_tops": INT8_PEAK_TOPS, "by_M": gemm,
                 "kernel": "gemm_f16_kernel: 128x128 tiles, exact integer products on v_mfma_f32_32x32x16_f16"},
        "dequant": dequant,
        "producers": producers,
        "model_stream": model,
        "cpu_baseline": cpu,
        "host": platform.node(),
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
