"""GPU parity of the fused producers (iq4xs_rms_norm_q8_1, iq4xs_swiglu_q8_1)
through the C ABI: the Q8_1 blocks they write, and the residual sum h, are
compared bit for bit with the CPU oracle on the same seeded inputs; a
producer -> GEMV chain is held to the path's output tolerances."""
import numpy as np
import pytest

from oracle.oracle import compute_metrics

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    torch.cuda.set_device(0)
    return torch.device("cuda:0")


def D(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def blocks(pkg, ws, K, M):
    return pkg.q8_1_blocks(ws, K, M).cpu().numpy().ravel()


def activations(orc, n, seed, scale=1.0):
    return (orc.gen_activations(n, seed, outliers=True) * np.float32(scale)).astype(np.float32)


RMS_CASES = [  # K, M, residual, H mode, gain, magnitude (K > 32768 takes the kernel's global re-read path)
    (32, 1, False, None, False, 1.0),
    (5120, 1, True, "separate", True, 1.0),
    (5120, 3, True, "x", True, 1e-3),
    (5120 + 96, 2, True, "r", False, 1.0),
    (8192, 5, False, "separate", True, 30.0),
    (17408, 2, True, None, True, 1.0),
    (8192 + 32, 2, True, "x", True, 1.0),
    (32768 + 32, 2, True, "x", True, 1.0),
    (32768, 1, True, None, True, 1.0),
    (1024, 64, True, "x", True, 1.0),
]


@pytest.mark.parametrize("K,M,res,hmode,gain,mag", RMS_CASES)
def test_rms_norm_q8_1_bit_exact(pkg, orc, dev, K, M, res, hmode, gain, mag):
    print(f"rms_norm_q8_1 K={K} M={M} res={res} H={hmode} gain={gain} mag={mag}", flush=True)
    X = activations(orc, K * M, 1000 + K + M, mag)
    R = activations(orc, K * M, 2000 + K + M, mag) if res else None
    g = (np.random.default_rng(K).random(K) * 2).astype(np.float32) if gain else None
    Xd, Rd = D(X, dev), (D(R, dev) if res else None)
    gd = D(g, dev) if gain else None
    Hd = {"separate": torch.empty(M * K, device=dev), "x": Xd, "r": Rd, None: None}[hmode]
    ws = pkg.rms_norm_q8_1(Xd, K, M, residual=Rd, out_h=Hd, gamma=gd, eps=1e-6)
    H_ref, _, Q_ref = orc.rms_norm_q8_1(X, K, M, R=R, gamma=g, eps=1e-6)
    assert np.array_equal(blocks(pkg, ws, K, M), Q_ref)
    if Hd is not None:
        assert np.array_equal(Hd.cpu().numpy().ravel().view(np.uint32), H_ref.ravel().view(np.uint32))
    if hmode != "x":
        assert np.array_equal(Xd.cpu().numpy().ravel(), X)  # input untouched


def test_rms_norm_zero_row_and_constant_row(pkg, orc, dev):
    K, M = 2048, 2
    X = np.zeros(K * M, np.float32)
    X[K:] = 0.5
    ws = pkg.rms_norm_q8_1(D(X, dev), K, M, eps=1e-6)
    _, _, Q_ref = orc.rms_norm_q8_1(X, K, M, eps=1e-6)
    assert np.array_equal(blocks(pkg, ws, K, M), Q_ref)


SWIGLU_CASES = [(32, 1), (17408, 1), (1024 + 96, 4), (17408, 3), (5120, 33)]


@pytest.mark.parametrize("K,M", SWIGLU_CASES)
def test_swiglu_q8_1_bit_exact(pkg, orc, dev, K, M):
    print(f"swiglu_q8_1 K={K} M={M}", flush=True)
    rng = np.random.default_rng(K * 7 + M)
    G = (rng.standard_normal(K * M) * 6).astype(np.float32)
    G[: min(16, K * M)] = np.float32([0, -90, 90, -87.5, 88.8, -20, 20, 1e-6, -1e-6, 3.5, -3.5, 50, -50, 1e3,
                                      -1e3, 0.5])[: min(16, K * M)]
    U = activations(orc, K * M, 3000 + K + M)
    ws = pkg.swiglu_q8_1(D(G, dev), D(U, dev), K, M)
    _, Q_ref = orc.swiglu_q8_1(G, U, K, M)
    assert np.array_equal(blocks(pkg, ws, K, M), Q_ref)


def test_producer_feeds_gemv_and_gemm(pkg, orc, dev):
    """rms norm -> Q8_1 -> GEMV (M=1) and GEMM (M=24): the workspace a producer
    writes is consumed as is; outputs meet the path's tolerances."""
    for K, N, M in ((5120, 256, 1), (5120, 192, 24)):
        X = activations(orc, K * M, 4000 + M)
        W = orc.gen_weights(K, N, seed=40 + M)
        ws = pkg.rms_norm_q8_1(D(X, dev), K, M, eps=1e-6)
        Y = pkg.mul_mat_q8_1(torch.from_numpy(W).to(dev), ws, K, N, M).cpu().numpy()
        _, _, AQ = orc.rms_norm_q8_1(X, K, M, eps=1e-6)
        Y_sem = orc.gemm_semantics(W, AQ, K, N, M).T
        m = compute_metrics(Y_sem, Y)
        assert m["rel_l2"] <= 1e-4 and not m["bad"], (K, N, M, m)


def test_rms_norm_workspace_next_to_its_inputs(pkg, orc, dev):
    """Arguments packed into one buffer -- workspace first, then X, R and H,
    each directly after the previous one -- are accepted and computed as
    when apart."""
    K, M = 1024, 2
    wsb = pkg.lib().iq4xs_workspace_bytes(K, M)
    ws_span = (wsb + 255) // 256 * 256
    buf = torch.zeros(ws_span + 3 * K * M * 4, dtype=torch.uint8, device=dev)
    ws = buf[:wsb]
    f = buf[ws_span:].view(torch.float32)
    X = activations(orc, K * M, 71)
    R = activations(orc, K * M, 72)
    f[:K * M] = D(X, dev)
    f[K * M:2 * K * M] = D(R, dev)
    Xd, Rd, Hd = f[:K * M], f[K * M:2 * K * M], f[2 * K * M:]
    pkg.rms_norm_q8_1(Xd, K, M, residual=Rd, out_h=Hd, eps=1e-6, ws=ws)
    H_ref, _, Q_ref = orc.rms_norm_q8_1(X, K, M, R=R, eps=1e-6)
    assert np.array_equal(blocks(pkg, ws, K, M), Q_ref)
    assert np.array_equal(Hd.cpu().numpy().view(np.uint32), H_ref.ravel().view(np.uint32))


def test_producers_reject_bad_arguments(pkg, dev):
    L = pkg.lib()
    s = torch.cuda.current_stream().cuda_stream
    K, M = 1024, 2
    X = torch.zeros(K * M + 64, device=dev)
    ws = pkg.workspace(K, M, dev)
    inv = pkg.ERROR_INVALID_VALUE
    n = ws.numel()
    assert L.iq4xs_rms_norm_q8_1(X.data_ptr(), None, None, None, -1.0, K, M, ws.data_ptr(), n, s) == inv
    assert L.iq4xs_rms_norm_q8_1(X.data_ptr(), None, None, None, float("nan"), K, M, ws.data_ptr(), n, s) == inv
    assert L.iq4xs_rms_norm_q8_1(X.data_ptr() + 4, None, None, None, 1e-6, K, M, ws.data_ptr(), n, s) == inv
    assert L.iq4xs_rms_norm_q8_1(X.data_ptr(), None, X.data_ptr() + 64, None, 1e-6, K, M, ws.data_ptr(), n,
                                 s) == inv  # H overlaps X without being X
    assert L.iq4xs_rms_norm_q8_1(X.data_ptr(), None, None, None, 1e-6, K + 16, M, ws.data_ptr(), n, s) == inv
    assert L.iq4xs_rms_norm_q8_1(X.data_ptr(), None, None, None, 1e-6, K, M, ws.data_ptr(), n - 1, s) == inv
    assert L.iq4xs_rms_norm_q8_1(X.data_ptr(), None, None, None, 1e-6, K, 1, X.data_ptr() + 4096 - 256, n,
                                 s) == inv  # workspace overlaps X's last bytes
    assert L.iq4xs_swiglu_q8_1(X.data_ptr(), None, K, M, ws.data_ptr(), n, s) == inv
    assert L.iq4xs_swiglu_q8_1(X.data_ptr(), X.data_ptr(), K, 0, ws.data_ptr(), n, s) == inv
    torch.cuda.synchronize()
