"""The reference-format bench harness (qwen_3.8_27b_optimizations_amd/harness/
bench_rows): its rows carry exactly the reference benches' keys, in order, and
its statistics are bench.h's.  The key lists below are the ones the reference's
bench mains print (file:line cited); the CPU tests run the harness in its
--schema and --stats-selftest modes, which touch no GPU."""
import json
import math
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HARNESS = os.path.join(ROOT, "qwen_3.8_27b_optimizations_amd", "harness", "_build", "bench_rows")

# kernels/matmul_iq4xs/bench_gemv.cpp:63-78
GEMV_KEYS = ["op", "shape", "K", "N", "M", "bytes", "stock_median_us", "stock_p95_us", "stock_gb_s",
             "gfx1100_median_us", "gfx1100_p95_us", "gfx1100_gb_s", "speedup", "winner"]
# kernels/matmul_iq4xs/bench_gemv_dp4a.cpp:110-133
GEMV_DP4A_KEYS = ["op", "shape", "K", "N", "M", "bytes", "runs", "variant", "real_dp4a_median_us",
                  "real_dp4a_mean_us", "real_dp4a_stddev_us", "real_dp4a_p95_us", "real_dp4a_gb_s",
                  "coop_dp4a_median_us", "coop_dp4a_mean_us", "coop_dp4a_stddev_us", "coop_dp4a_p95_us",
                  "coop_dp4a_gb_s", "speedup", "speedup_median", "speedup_mean", "speedup_mean_minus_1sigma",
                  "winner", "note"]
# kernels/matmul_iq4xs/bench_gemm_wmma.cpp:216-256
GEMM_WMMA_KEYS = ["op", "shape", "K", "N", "M", "bytes", "flops", "runs", "variant", "tile", "P", "banking",
                  "stock_median_us", "stock_mean_us", "stock_stddev_us", "stock_p95_us", "stock_tflops",
                  "stock_gb_s", "tiled_median_us", "tiled_tflops", "wmma_median_us", "wmma_mean_us",
                  "wmma_stddev_us", "wmma_p95_us", "wmma_stream_median_us", "wmma_stream_p95_us",
                  "wmma_stream_tflops", "wmma_stream_gb_s", "speedup", "speedup_median", "speedup_vs_stock_dp4a",
                  "speedup_mean", "speedup_mean_minus_1sigma", "TFLOPS_median", "GB/s", "winner", "note"]
OPS = {"gemv_iq4xs": GEMV_KEYS, "gemv_iq4xs_dp4a_coop": GEMV_DP4A_KEYS, "gemm_iq4xs_wmma_stream": GEMM_WMMA_KEYS}


def harness():
    if not os.path.exists(HARNESS):
        subprocess.run(["make", "-s", "-C", os.path.dirname(os.path.dirname(HARNESS))], check=True)
    return HARNESS


def ordered_rows(text):
    return json.loads(text, object_pairs_hook=lambda kv: kv)


def test_schema_matches_the_reference_benches():
    out = subprocess.run([harness(), "--schema"], capture_output=True, text=True, check=True, timeout=30).stdout
    rows = ordered_rows(out)
    assert [dict(r)["op"] for r in rows] == list(OPS)
    for r in rows:
        assert [k for k, _ in r] == OPS[dict(r)["op"]]


def test_statistics_are_bench_h():
    """bench.h:63-95: median of an odd count is the middle value, p95 the value at
    ceil(0.95 n) - 1, population stdev, GB/s = bytes / (median_us * 1e3)."""
    out = subprocess.run([harness(), "--stats-selftest"], capture_output=True, text=True, check=True,
                         timeout=30).stdout
    st = json.loads(out)
    t = np.array([5.0, 1.0, 4.0, 2.0, 3.0, 10.0, 7.0, 6.0, 9.0, 8.0, 11.0])
    s = np.sort(t)
    assert st["count"] == len(t)
    assert st["median_us"] == s[len(s) // 2]
    assert st["p95_us"] == s[math.ceil(0.95 * len(s)) - 1]
    assert st["min_us"] == s[0] and st["max_us"] == s[-1]
    assert abs(st["mean_us"] - t.mean()) < 1e-9 and abs(st["stdev_us"] - t.std()) < 1e-5
    assert abs(st["gb_s"] - 1e6 / (st["median_us"] * 1e3)) < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("op,want", [("gemv", "gemv_iq4xs"), ("gemv_dp4a", "gemv_iq4xs_dp4a_coop"),
                                     ("gemm_wmma", "gemm_iq4xs_wmma_stream")])
def test_harness_runs_on_gpu(op, want):
    print(f"[harness] --op {op}", flush=True)
    r = subprocess.run([harness(), "--op", op, "--runs", "1"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    rows = ordered_rows(r.stdout)
    assert rows
    for row in rows:
        d = dict(row)
        assert [k for k, _ in row] == OPS[want] and d["op"] == want
        if d["winner"] == "SKIPPED":  # the LUT entry's shape gate (M < 512), reported as the reference does
            assert d.get("variant") == "LUT_mu4" and d["M"] < 512, d
            continue
        assert d["speedup"] > 0
        timed = [v for k, v in row if k.endswith("median_us")]
        assert timed and all(v > 0 for v in timed), d
