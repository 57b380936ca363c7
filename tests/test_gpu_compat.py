"""The rest of the reference's standalone entry points, through the C ABI:
its FP64 comparators against the reference's own CPU FP64 outputs (golden,
bit for bit) and the oracle's restatement of the gfx1100 order, its
prequantised cooperative GEMV on the 64-byte padded Q8_1 layout, and the
WMMA / tiled / LUT GEMM names, which run the Q8_1 GEMM."""
import ctypes

import numpy as np
import pytest

from oracle.oracle import LAYOUT_KM, compute_metrics

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    torch.cuda.set_device(0)
    return torch.device("cuda:0")


def D(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def stream():
    return torch.cuda.current_stream().cuda_stream


def bits(t):
    return t.cpu().numpy().view(np.uint32)


GEMV_GOLDEN = ("gemv_512x48", "gemv_768x8_odd_superblocks", "gemv_1024x16_outliers")
GEMM_GOLDEN = ("gemm_256x8x5", "gemm_512x16x8")


def test_fp64_comparators_match_reference_cpu_outputs(pkg, orc, golden, dev):
    L = pkg.lib()
    for name in GEMV_GOLDEN:
        W, x, y_ref = golden[name + ".W"], golden[name + ".x"], golden[name + ".y"].astype(np.float32)
        K, N = (int(v) for v in golden[name + ".shape"][:2])
        # device copies are held in names: a temporary freed after data_ptr()
        # would be handed to the next allocation before the kernel reads it
        Wd, xd, y = D(W, dev), D(x, dev), torch.empty(N, device=dev)
        L.check("gemv_iq4xs_stock_gpu", Wd.data_ptr(), xd.data_ptr(), y.data_ptr(), K, N, stream())
        assert np.array_equal(bits(y), y_ref.view(np.uint32)), name
        L.check("gemv_iq4xs_gfx1100_gpu", Wd.data_ptr(), xd.data_ptr(), y.data_ptr(), K, N, stream())
        assert np.array_equal(bits(y), orc.gemv_fp64_by_subblock(W, x, K, N).view(np.uint32)), name
    for name in GEMM_GOLDEN:
        W, X, Y_ref = golden[name + ".W"], golden[name + ".X_km"], golden[name + ".Y"].astype(np.float32)
        K, N, M = (int(v) for v in golden[name + ".shape"][:3])
        Wd, Xd, Y = D(W, dev), D(X, dev), torch.empty(N * M, device=dev)
        L.check("gemm_iq4xs_stock_gpu", Wd.data_ptr(), Xd.data_ptr(), Y.data_ptr(), K, N, M, stream())
        assert np.array_equal(bits(Y), Y_ref.ravel().view(np.uint32)), name


def test_fp64_comparators_larger_shape(pkg, orc, dev):
    K, N = 5120, 300
    W = orc.gen_weights(K, N, seed=17)
    x = orc.gen_activations(K, seed=18, outliers=True)
    Wd, xd, y = D(W, dev), D(x, dev), torch.empty(N, device=dev)
    pkg.lib().check("gemv_iq4xs_stock_gpu", Wd.data_ptr(), xd.data_ptr(), y.data_ptr(), K, N, stream())
    assert np.array_equal(bits(y), orc.gemv_fp64(W, x, K, N).view(np.uint32))


def test_prequantized_coop_layout(pkg, orc, dev):
    """64-byte blocks (ds at 0, codes at 16..47) give exactly the GEMV of the
    same codes through the planar workspace."""
    L = pkg.lib()
    for K, N in ((2048, 96), (5120, 1024)):
        x = orc.gen_activations(K, seed=K, outliers=True)
        AQ = orc.quantize_q8_1(x).reshape(K // 32, 36)   # 36-byte blocks: ds, then 32 codes
        coop = np.zeros((K // 32, 64), np.uint8)
        coop[:, 0:4] = AQ[:, 0:4]
        coop[:, 16:48] = AQ[:, 4:36]
        coop[:, 4:16] = 0xA5   # padding is never read
        coop[:, 48:64] = 0x5A
        W, cd = D(orc.gen_weights(K, N, seed=3), dev), D(coop, dev)
        y = torch.empty(N, device=dev)
        L.check("gemv_iq4xs_dp4a_gfx1100_prequantized_gpu", W.data_ptr(), cd.data_ptr(), y.data_ptr(), K, N,
                stream())
        ws = pkg.quantize_q8_1(D(x, dev), K, 1)
        ref = pkg.mul_mat_q8_1(W, ws, K, N, 1)
        assert np.array_equal(bits(y), bits(ref).ravel()), (K, N)


GEMM_NAMES = ("gemm_iq4xs_wmma_stream_gpu", "gemm_iq4xs_wmma_p4_xor_gpu", "gemm_iq4xs_wmma_64x64_gpu",
              "gemm_iq4xs_stream_tiled_gpu", "gemm_iq4xs_wmma_gpu", "gemm_iq4xs_tiled_gpu")


def test_gemm_family_and_gemv_aliases(pkg, orc, dev):
    L = pkg.lib()
    K, N, M = 512, 64, 512
    W = D(orc.gen_weights(K, N, seed=21), dev)
    X = D(orc.gen_activations(K * M, seed=22).reshape(K, M), dev)   # [K][M]
    ref = torch.empty(N * M, device=dev)
    L.check("gemm_iq4xs_stock_dp4a_gpu", W.data_ptr(), X.data_ptr(), ref.data_ptr(), K, N, M, stream())
    for name in GEMM_NAMES:
        Y = torch.empty(N * M, device=dev)
        L.check(name, W.data_ptr(), X.data_ptr(), Y.data_ptr(), K, N, M, stream())
        assert np.array_equal(bits(Y), bits(ref)), name
    Y = torch.empty(N * M, device=dev)
    lut = torch.zeros(16, dtype=torch.float16, device=dev)
    L.check("gemm_iq4xs_lut_gpu", W.data_ptr(), lut.data_ptr(), X.data_ptr(), Y.data_ptr(), K, N, M, stream())
    assert np.array_equal(bits(Y), bits(ref))
    # the LUT gate of the reference: M < 512 (or unaligned shapes) is refused
    assert L.gemm_iq4xs_lut_gpu(W.data_ptr(), lut.data_ptr(), X.data_ptr(), Y.data_ptr(), K, N, 256,
                                stream()) == pkg.ERROR_INVALID_CONFIG
    assert L.gemm_iq4xs_lut_gpu(W.data_ptr(), lut.data_ptr(), X.data_ptr(), Y.data_ptr(), K, N - 8, M,
                                stream()) == pkg.ERROR_INVALID_CONFIG
    # the GEMV name of the cooperative kernel is the same path as the stock one
    x = D(orc.gen_activations(K, seed=23), dev)
    y1, y2 = torch.empty(N, device=dev), torch.empty(N, device=dev)
    L.check("gemv_iq4xs_dp4a_gfx1100_gpu", W.data_ptr(), x.data_ptr(), y1.data_ptr(), K, N, stream())
    L.check("gemv_iq4xs_stock_dp4a_gpu", W.data_ptr(), x.data_ptr(), y2.data_ptr(), K, N, stream())
    assert np.array_equal(bits(y1), bits(y2))
    m = compute_metrics(orc.gemm_semantics(orc.gen_weights(K, N, seed=21), orc.quantize_q8_1_batched(
        X.cpu().numpy(), K, M, LAYOUT_KM), K, N, M).ravel(), ref.cpu().numpy())
    assert m["rel_l2"] <= 1e-4, m
