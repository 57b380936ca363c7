"""GPU parity of iq4xs_mul_mat_q8_1_group: several matrices against one
quantised activation set in one launch.  Every output must be bit-identical
to iq4xs_mul_mat_q8_1 on its own matrix (itself held to the oracle in
test_gpu_parity.py) -- including GEMM groups whose tile size differs from
the single call's, which holds because both GEMM kernels compute each output
in the same order with the same scale tiles -- and one small case is
checked against the oracle directly."""
import numpy as np
import pytest

from oracle.oracle import LAYOUT_KM, LAYOUT_MK, compute_metrics

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    torch.cuda.set_device(0)
    return torch.device("cuda:0")


GROUP_CASES = [  # K, Ns, M, layout
    (5120, (8192, 1024, 1024), 1, LAYOUT_MK),     # q, k, v of a decode step
    (5120, (17408, 17408), 1, LAYOUT_MK),         # gate, up
    (2048, (7, 130, 1, 64), 3, LAYOUT_KM),        # ragged last tiles, N = 1
    (17408, (5120, 96), 8, LAYOUT_MK),            # matrix-core GEMV for the wide one, dot4 for the other
    (5120, (8192, 1024, 1024), 6, LAYOUT_KM),
    (5120, (17408, 17408), 8, LAYOUT_MK),         # gate/up: one matrix-core launch (8 waves each)
    (5120, (17408, 17408), 4, LAYOUT_KM),
    (5120, (8192, 4096, 1024), 7, LAYOUT_MK),     # two matrix-core matrices (16 waves) share a launch
    (5120, (8192, 1024, 1024), 8, LAYOUT_MK),     # at 8 columns the narrow k/v join q's launch
    (5120, (17408, 8192, 2048, 512), 5, LAYOUT_KM),  # 8- and 16-wave launches, one tile launch
    (2048, (2048 + 7, 4096 + 31), 8, LAYOUT_MK),  # ragged last row blocks in a shared launch
    (8192, (5120,), 2, LAYOUT_KM),
    (1024, (40, 33, 9), 2, LAYOUT_MK),            # K < 2048: one launch per matrix
    (2048, (300, 64), 20, LAYOUT_MK),             # M > 8: one GEMM launch
    (5120, (8192, 1024, 1024), 512, LAYOUT_MK),   # q/k/v: the planner sees 80 row tiles, k alone 8
    (5120, (17408, 17408), 512, LAYOUT_KM),       # gate/up: a bulk of whole rounds and a tail segment
    (8192, (130, 4000, 64), 200, LAYOUT_MK),      # ragged tiles in every matrix
    # 271 row tiles on 256 CUs: the planner's tail segment lies in the second matrix
    # (token-major outputs, ragged rows)
    (256, (128 * 200, 128 * 70 + 5), 100, LAYOUT_KM),
]


@pytest.mark.parametrize("K,Ns,M,layout", GROUP_CASES)
def test_group_matches_separate_calls(pkg, orc, dev, K, Ns, M, layout):
    print(f"group K={K} Ns={Ns} M={M} layout={layout}", flush=True)
    Ws = [pkg.synthetic_weights(K, N, seed=500 + i, device=dev) for i, N in enumerate(Ns)]
    X = pkg.synthetic_activations(K * M, seed=77, outliers=True, device=dev)
    ws = pkg.quantize_q8_1(X, K, M, layout)
    outs = pkg.mul_mat_q8_1_group(Ws, ws, K, list(Ns), M, layout)
    for i, (W, N) in enumerate(zip(Ws, Ns)):
        ref = pkg.mul_mat_q8_1(W, ws, K, N, M, layout)
        a, b = outs[i].cpu().numpy(), ref.cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (K, Ns, M, i)


def test_group_against_oracle(pkg, orc, dev):
    K, Ns, M = 2048, (48, 17, 130), 2
    Wn = [orc.gen_weights(K, N, seed=900 + i) for i, N in enumerate(Ns)]
    X = orc.gen_activations(K * M, seed=31, outliers=True)
    AQ = orc.quantize_q8_1_batched(X, K, M, LAYOUT_MK)
    ws = pkg.quantize_q8_1(torch.from_numpy(X).to(dev), K, M, LAYOUT_MK)
    outs = pkg.mul_mat_q8_1_group([torch.from_numpy(W).to(dev) for W in Wn], ws, K, list(Ns), M, LAYOUT_MK)
    for W, N, Y in zip(Wn, Ns, outs):
        m = compute_metrics(orc.gemm_semantics(W, AQ, K, N, M).T, Y.cpu().numpy())
        assert m["rel_l2"] <= 1e-4 and not m["bad"], (N, m)


def test_group_rejects_bad_arguments(pkg, dev):
    import ctypes

    L = pkg.lib()
    s = torch.cuda.current_stream().cuda_stream
    K, M = 2048, 1
    W = pkg.synthetic_weights(K, 16, seed=1, device=dev)
    Y = torch.empty(16, device=dev)
    ws = pkg.workspace(K, M, dev)
    P = ctypes.c_void_p * 5
    N5 = (ctypes.c_int64 * 5)(16, 16, 16, 16, 16)
    wp, yp = P(*([W.data_ptr()] * 5)), P(*([Y.data_ptr()] * 5))
    inv = pkg.ERROR_INVALID_VALUE
    for count in (0, 5):
        assert L.iq4xs_mul_mat_q8_1_group(count, wp, yp, N5, ws.data_ptr(), K, M, LAYOUT_MK, s) == inv
    bad_w = P(W.data_ptr(), None, W.data_ptr(), W.data_ptr(), W.data_ptr())
    assert L.iq4xs_mul_mat_q8_1_group(2, bad_w, yp, N5, ws.data_ptr(), K, M, LAYOUT_MK, s) == inv
    n0 = (ctypes.c_int64 * 5)(16, 0, 16, 16, 16)
    assert L.iq4xs_mul_mat_q8_1_group(2, wp, yp, n0, ws.data_ptr(), K, M, LAYOUT_MK, s) == inv
    assert L.iq4xs_mul_mat_q8_1_group(1, wp, yp, N5, ws.data_ptr(), K + 32, M, LAYOUT_MK, s) == inv
    torch.cuda.synchronize()
