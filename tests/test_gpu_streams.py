"""Calls are stateless and stream-ordered -- the reference's convention: one
host thread per stream, every launcher takes a hipStream_t
(real_stock_dp4a_comparator.hip:480-486).  The same work issued on two
streams at once, interleaved call by call, gives results bit-identical to a
serial run.  Both streams keep the default priority."""
import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    torch.cuda.set_device(0)
    return torch.device("cuda:0")


# K, N, M: bs=1 fused, bs=1 K > the fused bound, the matrix-core GEMV, both GEMM kernels
CASES = [(5120, 1024, 1), (17408, 640, 1), (5120, 2048, 6), (2048, 300, 64), (1024, 128 * 150, 130)]


def run_all(pkg, L, Ws, Xs, Ys, wss, streams):
    """Issue every case's iq4xs_mul_mat, alternating the streams call by call."""
    for i, ((K, N, M), W, X, Y, ws) in enumerate(zip(CASES, Ws, Xs, Ys, wss)):
        s = streams[i % len(streams)]
        L.check("iq4xs_mul_mat", W.data_ptr(), X.data_ptr(), Y.data_ptr(), K, N, M, pkg.LAYOUT_MK, ws.data_ptr(),
                ws.numel(), s.cuda_stream)


def test_two_streams_match_serial(pkg, dev):
    L = pkg.lib()
    Ws = [pkg.synthetic_weights(K, N, seed=40 + i, device=dev) for i, (K, N, M) in enumerate(CASES)]
    Xs = [pkg.synthetic_activations(K * M, seed=60 + i, outliers=True, device=dev) for i, (K, N, M) in enumerate(CASES)]
    ref = [torch.empty((M, N), device=dev) for (K, N, M) in CASES]
    wss = [torch.empty(L.iq4xs_workspace_bytes(K, M), dtype=torch.uint8, device=dev) for (K, N, M) in CASES]
    main = torch.cuda.current_stream()
    run_all(pkg, L, Ws, Xs, ref, wss, [main])
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()  # default priority
    for rep in range(3):
        outs = [torch.full((M, N), float("nan"), device=dev) for (K, N, M) in CASES]
        ws2 = [torch.empty_like(w) for w in wss]  # each stream's calls own their workspace
        torch.cuda.synchronize()
        run_all(pkg, L, Ws, Xs, outs, ws2, [s1, s2])
        torch.cuda.synchronize()
        for (K, N, M), a, b in zip(CASES, outs, ref):
            assert np.array_equal(a.cpu().numpy().view(np.uint32), b.cpu().numpy().view(np.uint32)), (rep, K, N, M)


def test_group_on_two_streams(pkg, dev):
    """Two grouped launches (GEMV and GEMM) in flight on different streams."""
    L = pkg.lib()
    K = 5120
    Ns = (2048, 512, 512)
    Ws = [pkg.synthetic_weights(K, N, seed=80 + i, device=dev) for i, N in enumerate(Ns)]
    P = ctypes.c_void_p * 3
    res = {}
    for M in (1, 96):
        X = pkg.synthetic_activations(K * M, seed=90 + M, device=dev)
        ws = pkg.quantize_q8_1(X, K, M)
        res[M] = (ws, [pkg.mul_mat_q8_1(W, ws, K, N, M) for W, N in zip(Ws, Ns)])
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = {M: [torch.empty((M, N), device=dev) for N in Ns] for M in res}
    for M, s in ((1, s1), (96, s2)):
        ws = res[M][0]
        L.check("iq4xs_mul_mat_q8_1_group", 3, P(*[W.data_ptr() for W in Ws]), P(*[y.data_ptr() for y in outs[M]]),
                (ctypes.c_int64 * 3)(*Ns), ws.data_ptr(), K, M, pkg.LAYOUT_MK, s.cuda_stream)
    torch.cuda.synchronize()
    for M in res:
        for a, b in zip(outs[M], res[M][1]):
            assert torch.equal(a.view(torch.int32), b.view(torch.int32)), M
