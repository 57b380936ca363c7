"""iq4xs_mul_mat_noalloc: the allocation-free form of iq4xs_mul_mat, whose Q8_1
workspace is the library's static device scratch.  Through the C ABI, each call
must equal iq4xs_mul_mat (same kernels, caller workspace) bit for bit; two
calls in a row, the second on a smaller input, so a stale larger workspace in
the shared scratch would show; and sizes past the scratch are refused before
anything is launched."""
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


# (K, N, M, layout): the GEMM path (M > 8, workspace), the GEMV past the fused
# bound (K > 8192, workspace), the small-batch GEMV, then a single column the
# fused GEMV takes (no workspace)
SEQUENCES = [
    [(5120, 1024, 96, 1), (5120, 1024, 24, 1)],
    [(17408, 640, 8, 0), (17408, 640, 1, 1)],
    [(8192, 512, 300, 0), (2048, 300, 5, 1), (4096, 200, 1, 1)],
]


@pytest.mark.parametrize("seq", SEQUENCES)
def test_noalloc_matches_mul_mat(pkg, dev, seq):
    L = pkg.lib()
    s = torch.cuda.current_stream().cuda_stream
    for call, (K, N, M, layout) in enumerate(seq):
        print(f"[noalloc] call {call}: K={K} N={N} M={M} layout={layout}", flush=True)
        W = pkg.synthetic_weights(K, N, seed=K + N + call, device=dev)
        X = pkg.synthetic_activations(K * M, seed=M + call, outliers=True, device=dev)
        shape = (M, N) if layout == pkg.LAYOUT_MK else (N, M)
        Y = torch.full(shape, float("nan"), device=dev)
        L.check("iq4xs_mul_mat_noalloc", W.data_ptr(), X.data_ptr(), Y.data_ptr(), K, N, M, layout, s)
        ref = pkg.mul_mat(W, X, K, N, M, layout)
        torch.cuda.synchronize()
        assert np.array_equal(bits(Y), bits(ref)), (call, K, N, M)
        assert bool(torch.isfinite(Y).all())


def test_noalloc_refuses_sizes_past_the_scratch(pkg, dev):
    L = pkg.lib()
    s = torch.cuda.current_stream().cuda_stream
    K, N = 17408, 64
    limit = 128 << 20
    M_over = 2500  # 17408 * 2500 * 3.125 bytes > 128 MiB
    assert L.iq4xs_workspace_bytes(K, M_over) > limit >= L.iq4xs_workspace_bytes(K, 2400)
    W = torch.zeros(N * K // 256 * 136, dtype=torch.uint8, device=dev)
    X = torch.zeros(16, device=dev)  # never read: the call is refused before any launch
    Y = torch.full((4,), 7.0, device=dev)
    assert L.iq4xs_mul_mat_noalloc(W.data_ptr(), X.data_ptr(), Y.data_ptr(), K, N, M_over, pkg.LAYOUT_MK, s) == \
        pkg.ERROR_INVALID_VALUE
    assert L.iq4xs_mul_mat_noalloc(W.data_ptr(), None, Y.data_ptr(), K, N, 1, pkg.LAYOUT_MK, s) == \
        pkg.ERROR_INVALID_VALUE
    torch.cuda.synchronize()
    assert bool((Y == 7.0).all())
