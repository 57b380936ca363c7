"""iq4xs_rms_norm_mul_mat_group: the RMS norm of one column fused into the
prologue of a grouped bs=1 GEMV.  Its outputs (every Y[i], and H) must be
bit-identical to iq4xs_rms_norm_q8_1 followed by iq4xs_mul_mat_q8_1_group,
both held to the oracle elsewhere (test_gpu_producers.py, test_gpu_grouped.py);
the fused kernel runs the producer's own reduction order (rms_device.h)."""
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


def bits(t):
    return t.contiguous().cpu().numpy().view(np.uint32)


CASES = [  # K, Ns, residual, gain, write H
    (5120, (8192, 1024, 1024), True, True, True),    # q, k, v after the attention norm
    (5120, (17408, 17408), True, True, True),        # gate, up after the FFN norm
    (5120, (7, 130, 1), True, True, False),          # ragged last tiles, N = 1
    (2048, (300, 64), False, True, True),            # smallest K the tile kernel takes; no residual
    (8192, (5120,), True, False, True),              # no gain
    (4096, (2048, 33, 96, 4000), False, False, False),
]


@pytest.mark.parametrize("K,Ns,res,gain,write_h", CASES)
def test_fused_matches_two_calls(pkg, dev, K, Ns, res, gain, write_h):
    print(f"rms-fused K={K} Ns={Ns} res={res} gain={gain} H={write_h}", flush=True)
    g = torch.Generator().manual_seed(K + len(Ns))
    X = (torch.randn(K, generator=g) * 3.0).to(dev)
    R = (torch.randn(K, generator=g) * 0.5).to(dev) if res else None
    gamma = (torch.rand(K, generator=g) + 0.5).to(dev) if gain else None
    Ws = [pkg.synthetic_weights(K, N, seed=700 + i, device=dev) for i, N in enumerate(Ns)]
    eps = 1e-6
    H_ref = torch.empty(K, device=dev) if write_h else None
    ws = pkg.rms_norm_q8_1(X, K, 1, residual=R, out_h=H_ref, gamma=gamma, eps=eps)
    ref = pkg.mul_mat_q8_1_group(Ws, ws, K, list(Ns), 1)
    H = torch.full((K,), float("nan"), device=dev) if write_h else None
    for rep in range(2):  # twice: no state carried between calls
        outs = pkg.rms_norm_mul_mat_group(Ws, X, K, list(Ns), residual=R, out_h=H, gamma=gamma, eps=eps)
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(outs, ref)):
            assert np.array_equal(bits(a), bits(b).ravel()), (rep, i)
        if write_h:
            assert np.array_equal(bits(H), bits(H_ref)), rep


def test_fused_rejects(pkg, dev):
    L = pkg.lib()
    s = torch.cuda.current_stream().cuda_stream
    K, N = 5120, 64
    W = pkg.synthetic_weights(K, N, seed=1, device=dev)
    X = torch.randn(2 * K, device=dev)
    Y = torch.empty(N, device=dev)
    P1 = ctypes.c_void_p * 1
    wp, yp, nn = P1(W.data_ptr()), P1(Y.data_ptr()), (ctypes.c_int64 * 1)(N)
    inv, nsup = pkg.ERROR_INVALID_VALUE, pkg.ERROR_NOT_SUPPORTED
    f = L.iq4xs_rms_norm_mul_mat_group
    assert f(0, wp, yp, nn, X.data_ptr(), None, None, None, 1e-6, K, s) == inv
    assert f(5, wp, yp, nn, X.data_ptr(), None, None, None, 1e-6, K, s) == inv
    assert f(1, wp, yp, nn, None, None, None, None, 1e-6, K, s) == inv
    assert f(1, wp, yp, nn, X.data_ptr(), None, None, None, -1.0, K, s) == inv
    assert f(1, wp, yp, nn, X.data_ptr(), None, None, None, 1e-6, K + 32, s) == inv
    # in place (H = X) and overlapping outputs are refused: workgroup 0 writes H while others read X
    assert f(1, wp, yp, nn, X.data_ptr(), None, X.data_ptr(), None, 1e-6, K, s) == inv
    assert f(1, wp, yp, nn, X.data_ptr(), None, X.data_ptr() + 4 * K - 16, None, 1e-6, K, s) == inv
    yx = P1(X.data_ptr() + 4 * 16)
    assert f(1, wp, yx, nn, X.data_ptr(), None, None, None, 1e-6, K, s) == inv
    assert f(1, wp, yp, nn, X.data_ptr() + 4, None, None, None, 1e-6, K, s) == inv  # unaligned X
    assert f(1, wp, yp, nn, X.data_ptr(), None, None, X.data_ptr() + 4 * K + 4, 1e-6, K, s) == inv  # unaligned gamma
    # shapes the fused prologue does not take
    Ws = pkg.synthetic_weights(1024, N, seed=2, device=dev)
    assert f(1, P1(Ws.data_ptr()), yp, nn, X.data_ptr(), None, None, None, 1e-6, 1024, s) == nsup
    # past one pass-1 batch of the norm (K > 8192): the first K above the bound, the
    # largest multiple of 256 that an earlier four-round batch took, and one beyond
    for Kb in (8448, 16384, 16640):
        Xb = torch.randn(Kb, device=dev)
        Wb = pkg.synthetic_weights(Kb, N, seed=3, device=dev)
        assert f(1, P1(Wb.data_ptr()), yp, nn, Xb.data_ptr(), None, None, None, 1e-6, Kb, s) == nsup, Kb
    torch.cuda.synchronize()


@pytest.mark.parametrize("K", [8448, 16384])
def test_two_call_path_past_fused_bound(pkg, orc, dev, K):
    """Where the fused kernel refuses (K past one pass-1 batch), the two calls it
    stands for -- the rms producer and the grouped GEMV -- still meet the oracle:
    Q8_1 blocks and h bit for bit, outputs within the path's tolerance."""
    from oracle.oracle import compute_metrics

    print(f"rms two-call K={K}", flush=True)
    N = 96
    rng = np.random.default_rng(K)
    x = (rng.standard_normal(K) * 3.0).astype(np.float32)
    r = (rng.standard_normal(K) * 0.5).astype(np.float32)
    gamma = (rng.random(K) + 0.5).astype(np.float32)
    h_ref, _, blocks_ref = orc.rms_norm_q8_1(x, K, 1, R=r, gamma=gamma, eps=1e-6)
    W = orc.gen_weights(K, N, seed=K + 1)
    Xd, Rd, Gd = (torch.from_numpy(a).to(dev) for a in (x, r, gamma))
    H = torch.empty(K, device=dev)
    ws = pkg.rms_norm_q8_1(Xd, K, 1, residual=Rd, out_h=H, gamma=Gd, eps=1e-6)
    (y,) = pkg.mul_mat_q8_1_group([torch.from_numpy(W).to(dev)], ws, K, [N], 1)
    torch.cuda.synchronize()
    assert np.array_equal(pkg.q8_1_blocks(ws, K, 1).cpu().numpy().ravel(), blocks_ref)
    assert np.array_equal(H.cpu().numpy().view(np.uint32), h_ref.ravel().view(np.uint32))
    m = compute_metrics(orc.gemv_semantics(W, blocks_ref, K, N), y.cpu().numpy().ravel())
    assert m["rel_l2"] <= 1e-4 and not m["bad"], m


# iq4xs_rms_norm_mul_mat_swiglu: the norm, the gate/up pair (each workgroup
# owns the same rows of both) and S = silu(gate) * up in its epilogue.
SWIGLU_CASES = [  # K, N, residual, gain, write H
    (5120, 17408, True, True, True),    # the FFN's gate/up after its norm: 68 rows per workgroup
    (8192, 5120, True, False, True),
    (2048, 1000, False, True, False),
    (4096, 97, False, False, False),    # one row per workgroup
]


@pytest.mark.parametrize("K,N,res,gain,write_h", SWIGLU_CASES)
def test_swiglu_pair_matches_group_and_producer(pkg, orc, dev, K, N, res, gain, write_h):
    """gate, up and H bit-identical to the rms-fused group call on (gate, up);
    S bit-identical to the oracle's silu(gate) * up in fp32; and, where N is a
    whole number of Q8_1 blocks, Q8_1(S) bit-identical to the SwiGLU producer
    on the group call's gate and up."""
    print(f"rms-swiglu K={K} N={N} res={res} gain={gain} H={write_h}", flush=True)
    g = torch.Generator().manual_seed(K + N)
    X = (torch.randn(K, generator=g) * 3.0).to(dev)
    R = (torch.randn(K, generator=g) * 0.5).to(dev) if res else None
    gamma = (torch.rand(K, generator=g) + 0.5).to(dev) if gain else None
    Wg = pkg.synthetic_weights(K, N, seed=900, device=dev)
    Wu = pkg.synthetic_weights(K, N, seed=901, device=dev)
    eps = 1e-6
    H_ref = torch.empty(K, device=dev) if write_h else None
    gate_ref, up_ref = pkg.rms_norm_mul_mat_group([Wg, Wu], X, K, [N, N], residual=R, out_h=H_ref, gamma=gamma,
                                                  eps=eps)
    torch.cuda.synchronize()
    gn, un = gate_ref.cpu().numpy(), up_ref.cpu().numpy()
    S_ref = (orc.silu(gn) * un).astype(np.float32)
    for rep in range(2):  # twice: no state carried between calls
        H = torch.full((K,), float("nan"), device=dev) if write_h else None
        S, gate, up = pkg.rms_norm_mul_mat_swiglu(Wg, Wu, X, K, N, residual=R, out_h=H, gamma=gamma, eps=eps)
        torch.cuda.synchronize()
        assert np.array_equal(bits(gate), bits(gate_ref)), rep
        assert np.array_equal(bits(up), bits(up_ref)), rep
        assert np.array_equal(bits(S), S_ref.view(np.uint32)), rep
        if write_h:
            assert np.array_equal(bits(H), bits(H_ref)), rep
    S2, g2, u2 = pkg.rms_norm_mul_mat_swiglu(Wg, Wu, X, K, N, residual=R, gamma=gamma, eps=eps, keep_gate_up=False)
    torch.cuda.synchronize()
    assert g2 is None and u2 is None and np.array_equal(bits(S2), bits(S))
    if N % 32 == 0:
        ws_p = pkg.swiglu_q8_1(gate_ref, up_ref, N, 1)
        ws_s = pkg.quantize_q8_1(S, N, 1)
        assert np.array_equal(pkg.q8_1_blocks(ws_s, N, 1).cpu().numpy(), pkg.q8_1_blocks(ws_p, N, 1).cpu().numpy())


def test_swiglu_pair_rejects(pkg, dev):
    L = pkg.lib()
    s = torch.cuda.current_stream().cuda_stream
    K, N = 5120, 64
    Wg = pkg.synthetic_weights(K, N, seed=1, device=dev)
    Wu = pkg.synthetic_weights(K, N, seed=2, device=dev)
    X = torch.randn(2 * K, device=dev)
    S = torch.empty(N, device=dev)
    Yg, Yu = torch.empty(N, device=dev), torch.empty(N, device=dev)
    inv, nsup = pkg.ERROR_INVALID_VALUE, pkg.ERROR_NOT_SUPPORTED
    f = L.iq4xs_rms_norm_mul_mat_swiglu
    x, w, u = X.data_ptr(), Wg.data_ptr(), Wu.data_ptr()
    assert f(w, u, N, x, None, None, None, 1e-6, K, Yg.data_ptr(), Yu.data_ptr(), None, s) == inv  # no S
    assert f(None, u, N, x, None, None, None, 1e-6, K, None, None, S.data_ptr(), s) == inv
    assert f(w, u, 0, x, None, None, None, 1e-6, K, None, None, S.data_ptr(), s) == inv
    assert f(w, u, N, x, None, None, None, -1.0, K, None, None, S.data_ptr(), s) == inv
    assert f(w, u, N, x + 4, None, None, None, 1e-6, K, None, None, S.data_ptr(), s) == inv  # unaligned X
    assert f(w, u, N, x, None, x, None, 1e-6, K, None, None, S.data_ptr(), s) == inv  # H = X
    assert f(w, u, N, x, None, None, None, 1e-6, K, Yg.data_ptr(), None, Yg.data_ptr(), s) == inv  # S = Y_gate
    assert f(w, u, N, x, None, None, None, 1e-6, K, None, None, x + 64, s) == inv  # S inside X
    # N = 17 at K = 5120: no divisor of N makes whole steps (20 super-blocks per row, steps of 8)
    W17 = pkg.synthetic_weights(K, 17, seed=3, device=dev)
    assert f(W17.data_ptr(), W17.data_ptr(), 17, x, None, None, None, 1e-6, K, None, None, S.data_ptr(), s) == nsup
    X16 = torch.randn(16640, device=dev)  # K past one pass-1 batch (X sized for it, so nothing overlaps)
    assert f(w, u, N, X16.data_ptr(), None, None, None, 1e-6, 16640, None, None, S.data_ptr(), s) == nsup
    torch.cuda.synchronize()
