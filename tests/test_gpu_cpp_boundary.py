"""The library's C++ boundary on the GPU: tests/cpp/boundary_test (built by
__graft_entry__.build()) calls the ggml hooks through include/iq4xs_ggml_custom.cuh
with ggml's own types, restating the patch's mmq.cu / mmvq.cu hook conditions,
and the standalone API through the reference's own forward declarations of its
mangled C++ names.  Its outputs are compared here with the oracle on the same
seeded inputs: Q8_1 blocks, the dequantiser and the FP64 comparator bit for
bit, the GEMV / GEMM outputs within rel-L2 1e-4 of the reference semantics."""
import os
import subprocess

import numpy as np
import pytest

from oracle.oracle import LAYOUT_KM, LAYOUT_MK, compute_metrics

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "_build", "boundary_test")


def test_cpp_boundary(orc, tmp_path):
    assert os.path.exists(BIN), f"{BIN} is missing: run __graft_entry__.build()"
    K, N, M = 5120, 333, 64
    W = orc.gen_weights(K, N, seed=91)
    x = orc.gen_activations(K, seed=92)
    X = orc.gen_activations(K * M, seed=93, outliers=True).reshape(M, K)
    (tmp_path / "meta.txt").write_text(f"{K} {N} {M}\n")
    W.tofile(tmp_path / "W.bin")
    x.tofile(tmp_path / "x.bin")
    X.tofile(tmp_path / "X_mk.bin")
    np.ascontiguousarray(X.T).tofile(tmp_path / "X_km.bin")
    print(f"[cpp-boundary] K={K} N={N} M={M}", flush=True)
    r = subprocess.run([BIN, str(tmp_path)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stderr
    codes = dict(line.rsplit(" ", 1) for line in r.stdout.splitlines() if not line.startswith("boundary_test"))
    assert codes["mmvq_hook_taken"] == "1" and codes["mmq_hook_taken"] == "1"
    assert codes["gemv_can_handle_M2"] == "0" and codes["mmvq_hook_fusion_falls_back"] == "0"
    assert codes["gemm_iq4xs_lut_gpu"] == "9"  # the reference's LUT shape gate (M < 512)

    load = lambda name, dt=np.float32: np.fromfile(tmp_path / name, dtype=dt)
    AQ1 = orc.quantize_q8_1(x)
    assert np.array_equal(load("q8_1.bin", np.uint8), AQ1)
    y_sem = orc.gemv_semantics(W, AQ1, K, N)
    for name in ("gemv_hook.bin", "stock_dp4a_gemv.bin", "gfx1100_dp4a_gemv.bin"):
        m = compute_metrics(y_sem, load(name))
        assert m["rel_l2"] <= 1e-4 and not m["bad"], (name, m)
    # the FP64 comparator reproduces the reference's CPU oracle bit for bit
    assert np.array_equal(load("stock_fp64_gemv.bin").view(np.uint32), orc.gemv_fp64(W, x, K, N).view(np.uint32))
    AQ = orc.quantize_q8_1_batched(X, K, M, LAYOUT_MK)
    assert np.array_equal(AQ, orc.quantize_q8_1_batched(np.ascontiguousarray(X.T), K, M, LAYOUT_KM))
    Y_sem = orc.gemm_semantics(W, AQ, K, N, M)  # [N, M]
    m = compute_metrics(Y_sem.T, load("gemm_hook.bin").reshape(M, N))
    assert m["rel_l2"] <= 1e-4 and not m["bad"], ("gemm_hook", m)
    for name in ("stock_dp4a_gemm.bin", "wmma_stream_gemm.bin"):
        m = compute_metrics(Y_sem, load(name).reshape(N, M))
        assert m["rel_l2"] <= 1e-4 and not m["bad"], (name, m)
    dq = load("dequant.bin")
    assert np.array_equal(dq.view(np.uint32), orc.dequant(W, K, N).ravel().view(np.uint32))
