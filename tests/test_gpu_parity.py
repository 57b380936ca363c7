"""GPU parity tests: every call goes through the C ABI of libiq4xs_mi355x.so
and is compared with the CPU oracle on the same seeded inputs.

Bars (from the path's contract):
  * Q8_1 blocks and per-32-element int32 sub-block sums: bit-exact;
  * fp32 outputs: relative L2 <= 1e-4 against the reference kernel semantics
    (oracle gemv/gemm_semantics), cosine >= 0.99999 against the FP64 oracle
    evaluated on the dequantised Q8_1 activations x_hat.
"""
import numpy as np
import pytest

from oracle.oracle import BLOCK_Q8_1, LAYOUT_KM, LAYOUT_MK, compute_metrics

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

REL_L2_TOL = 1e-4
COS_TOL = 0.99999

CONFIG1 = {  # K -> N of the 27B-class decode projections
    "q_proj": (5120, 8192), "k_proj": (5120, 1024), "v_proj": (5120, 1024), "o_proj": (8192, 5120),
    "gate_proj": (5120, 17408), "up_proj": (5120, 17408), "down_proj": (17408, 5120),
}


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    torch.cuda.set_device(0)
    return torch.device("cuda:0")


def D(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def stream():
    return torch.cuda.current_stream().cuda_stream


def check_outputs(orc, W, AQ, Y_gpu_mn, K, N, M, label):
    """Y_gpu_mn: numpy [M, N]."""
    Y_sem = orc.gemm_semantics(W, AQ, K, N, M).T
    m = compute_metrics(Y_sem, Y_gpu_mn)
    assert m["rel_l2"] <= REL_L2_TOL and not m["bad"], (label, m)
    xhat = orc.dequant_q8_1(AQ).reshape(M, K)
    Y64 = orc.gemm_fp64(W, np.ascontiguousarray(xhat.T), K, N, M, nthreads=8).T
    m64 = compute_metrics(Y64, Y_gpu_mn)
    assert m64["cosine"] >= COS_TOL, (label, m64)
    return m, m64


# ------------------------------------------------------------------ building blocks
def test_probe_mfma_layout(pkg, dev):
    rng = np.random.default_rng(0)
    A = rng.integers(-128, 128, (32, 32), dtype=np.int8)
    B = rng.integers(-128, 128, (32, 32), dtype=np.int8)
    C = torch.zeros((32, 32), dtype=torch.int32, device=dev)
    Ad, Bd = D(A, dev), D(B, dev)  # keep both alive until the kernel has run
    pkg.lib().check("iq4xs_probe_mfma_i8", Ad.data_ptr(), Bd.data_ptr(), C.data_ptr(), stream())
    torch.cuda.synchronize()
    assert np.array_equal(C.cpu().numpy(), A.astype(np.int32) @ B.astype(np.int32).T)


def test_synthetic_weights_match_oracle(pkg, orc, dev):
    W = pkg.synthetic_weights(4096, 48, seed=42, device=dev).cpu().numpy()
    assert np.array_equal(W, orc.gen_weights(4096, 48, seed=42))
    part = pkg.synthetic_weights(256, 7, seed=42, first_block=123, device=dev).cpu().numpy()
    assert np.array_equal(part, W[123 * 136:130 * 136])


def test_synthetic_activations_distribution(pkg, dev):
    x = pkg.synthetic_activations(1 << 20, seed=5, device=dev).cpu().numpy()
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    xo = pkg.synthetic_activations(1 << 20, seed=5, outliers=True, device=dev).cpu().numpy()
    assert 0.008 < np.mean(xo != x) < 0.012


@pytest.mark.parametrize("K,M,layout,outliers", [
    (256, 1, LAYOUT_MK, False), (5120, 1, LAYOUT_MK, False), (17408, 1, LAYOUT_MK, True),
    (5120, 8, LAYOUT_MK, True), (1024, 37, LAYOUT_KM, False), (2048, 512, LAYOUT_MK, True),
    (512, 300, LAYOUT_KM, True)])
def test_q8_1_blocks_bit_exact(pkg, orc, dev, K, M, layout, outliers):
    X = orc.gen_activations(K * M, seed=K + M, outliers=outliers)
    X = X.reshape(M, K) if layout == LAYOUT_MK else X.reshape(K, M)
    ref = orc.quantize_q8_1_batched(X, K, M, layout)
    ws = pkg.quantize_q8_1(D(X, dev), K, M, layout)
    got = pkg.q8_1_blocks(ws, K, M).cpu().numpy().ravel()
    assert np.array_equal(got, ref)


def test_q8_1_reference_entry_points(pkg, orc, dev):
    L = pkg.lib()
    K, M = 1024, 6
    x = orc.gen_activations(K, seed=1, outliers=True)
    y = torch.zeros(K // 32 * 36, dtype=torch.uint8, device=dev)
    xd = D(x, dev)
    L.check("quantize_row_q8_1_gpu", xd.data_ptr(), y.data_ptr(), K, stream())
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), orc.quantize_q8_1(x))
    X = orc.gen_activations(K * M, seed=2).reshape(K, M)
    Y = torch.zeros(M * K // 32 * 36, dtype=torch.uint8, device=dev)
    Xd = D(X, dev)
    L.check("quantize_row_q8_1_batched_gpu", Xd.data_ptr(), Y.data_ptr(), K, M, stream())
    torch.cuda.synchronize()
    assert np.array_equal(Y.cpu().numpy(), orc.quantize_q8_1_batched(X, K, M, LAYOUT_KM))


def test_q8_1_special_blocks(pkg, orc, dev):
    blocks = []
    blocks.append(np.zeros(32, np.float32))                                   # all zero
    b = np.zeros(32, np.float32); b[5] = 3.0; blocks.append(b)                # single nonzero
    b = np.zeros(32, np.float32); b[0] = 127.0
    b[1:9] = [2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 3.5, 126.5]; blocks.append(b)  # exact .5 ties
    b = np.zeros(32, np.float32); b[0] = 2.0**24; b[16] = -(2.0**24 - 1); b[1] = 0.75; blocks.append(b)  # tree order
    b = np.zeros(32, np.float32); b[0] = 1.0; b[1] = -0.0; blocks.append(b)   # -0.0
    b = np.full(32, 1e-30, np.float32); blocks.append(b)                      # d underflows fp16
    b = np.full(32, -7e4, np.float32); blocks.append(b)                       # sum overflows fp16
    x = np.concatenate(blocks + [np.zeros(32 * (8 - len(blocks)), np.float32)])
    ws = pkg.quantize_q8_1(D(x, dev), 256, 1, LAYOUT_MK)
    got = pkg.q8_1_blocks(ws, 256, 1).cpu().numpy().ravel()
    assert np.array_equal(got, orc.quantize_q8_1(x))


def rounding_boundary_blocks(n_blocks: int, seed: int) -> np.ndarray:
    """Blocks whose x/d sit on or within a few ulp-scale offsets of half
    integers (the quantiser's reciprocal fast path must hand those to the
    exact division), plus blocks of fp32 denormals and mixed magnitudes."""
    rng = np.random.default_rng(seed)
    out = np.zeros((n_blocks, 32), np.float32)
    offs = np.array([0.0, 2.0**-22, -2.0**-22, 2.0**-16, -2.0**-16, 2.0**-14, -2.0**-14,
                     2.0**-13, -2.0**-13, 2.0**-10, -2.0**-10])
    for b in range(n_blocks):
        kind = b % 4
        if kind == 3:  # denormal block (d stays > 0)
            out[b] = (rng.standard_normal(32) * 1e-39).astype(np.float32)
            continue
        amax = np.float32(10.0 ** rng.uniform(-6, 4))
        d = np.float32(amax / np.float32(127.0))
        k = rng.integers(-127, 127, 32)
        x = (k + 0.5 + rng.choice(offs, 32)) * np.float64(d)
        if kind == 1:
            x *= rng.choice([1.0, 1e-3], 32)  # mixed magnitudes inside one block
        out[b] = x.astype(np.float32)
        out[b, rng.integers(32)] = amax * rng.choice([-1.0, 1.0])
    return out.ravel()


def test_q8_1_rounding_boundaries(pkg, orc, dev):
    K = 256 * 64
    x = rounding_boundary_blocks(K // 32, seed=11)
    ref = orc.quantize_q8_1(x)
    ws = pkg.quantize_q8_1(D(x, dev), K, 1, LAYOUT_MK)
    got = pkg.q8_1_blocks(ws, K, 1).cpu().numpy().ravel()
    assert np.array_equal(got, ref)
    X = x.reshape(8, K // 8)
    ws = pkg.quantize_q8_1(D(np.ascontiguousarray(X.T), dev), K // 8, 8, LAYOUT_KM)
    got = pkg.q8_1_blocks(ws, K // 8, 8).cpu().numpy().ravel()
    assert np.array_equal(got, orc.quantize_q8_1_batched(X, K // 8, 8, LAYOUT_MK))


# ------------------------------------------------------------------ dequantiser
def test_dequant_bit_exact(pkg, orc, golden, dev):
    """dequant_iq4xs_gpu == the reference's CPU dequantiser bit for bit: its
    own outputs (golden fixtures from the compiled ref_cpu.cpp), the KAT
    blocks' hand values, and the oracle on a large random matrix."""
    import json, os
    L = pkg.lib()
    for name in ("gemv_512x48", "gemv_768x8_odd_superblocks", "gemm_256x8x5"):
        W = golden[name + ".W"]
        want = golden[name + ".dequant"].ravel()
        got = pkg.dequant(D(W, dev), W.size // 136).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32)), name
    with open(os.path.join(os.path.dirname(__file__), "golden", "iq4xs_kat_blocks.json")) as f:
        kat = json.load(f)
    for case in kat["cases"]:
        W = np.frombuffer(bytes.fromhex(case["raw_hex"]), np.uint8).copy()
        got = pkg.dequant(D(W, dev), case["n_blocks"]).cpu().numpy().reshape(case["n_blocks"], 256)
        for blk, elem, value in case["hand_values"]:
            assert got[int(blk), int(elem)] == np.float32(value), (case["name"], blk, elem)
    K, N = 5120, 333
    W = orc.gen_weights(K, N, seed=77)
    got = pkg.dequant(D(W, dev), N * K // 256).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), orc.dequant(W, K, N).ravel().view(np.uint32))
    Wd, y = D(W, dev), torch.zeros(256, device=dev)
    assert L.dequant_iq4xs_gpu(Wd.data_ptr(), y.data_ptr(), 1, 48, stream()) == pkg.ERROR_INVALID_VALUE
    # warp_size 32 selects the same kernel; an empty matrix writes nothing
    got32 = torch.full((256,), -1.0, device=dev)
    assert L.dequant_iq4xs_gpu(Wd.data_ptr(), got32.data_ptr(), 1, 32, stream()) == 0
    assert L.dequant_iq4xs_gpu(Wd.data_ptr(), y.data_ptr(), 0, 64, stream()) == 0
    torch.cuda.synchronize()
    assert np.array_equal(got32.cpu().numpy().view(np.uint32), orc.dequant(W, K, N).ravel()[:256].view(np.uint32))
    assert not y.any()


# ------------------------------------------------------------------ GEMV / GEMM kernels
GEMV_CASES = [(256, 1, 1), (768, 7, 1), (1024, 64, 1), (5120, 333, 1), (4096, 4096, 1),
              (768, 9, 2), (1280, 65, 3), (2048, 130, 4), (256, 5, 5), (5120, 100, 6), (512, 77, 7),
              (8192, 96, 8), (17408, 40, 8),
              # N >= 2048 and M >= 5: the matrix-core GEMV (ragged last 32-row block; fewer
              # super-blocks than waves; long K; 16- and 8-wave workgroups)
              (2048, 2048 + 33, 6), (768, 2051, 7), (5120, 2048, 8), (17408, 2080, 7), (5120, 8192, 5),
              (2048, 17408, 5), (5120, 2048 + 5, 4),
              # from M = 8 also narrow matrices (N >= 1024), at least 8 rows per workgroup
              (5120, 1024, 8), (2048, 1024 + 17, 8), (768, 1500, 8)]


@pytest.mark.parametrize("K,N,M", GEMV_CASES)
def test_gemv_sums_and_outputs(pkg, orc, dev, K, N, M):
    W = orc.gen_weights(K, N, seed=1000 + K + N)
    X = orc.gen_activations(K * M, seed=2000 + M, outliers=(M > 1)).reshape(M, K)
    AQ = orc.quantize_q8_1_batched(X, K, M, LAYOUT_MK)
    Wd = D(W, dev)
    ws = pkg.quantize_q8_1(D(X, dev), K, M, LAYOUT_MK)
    S, Y = pkg.subblock_sums(Wd, ws, K, N, M, pkg.PATH_GEMV)
    Y2 = pkg.mul_mat_q8_1(Wd, ws, K, N, M, LAYOUT_MK, pkg.PATH_GEMV)
    torch.cuda.synchronize()
    assert np.array_equal(S.cpu().numpy(), orc.subblock_sums(W, AQ, K, N, M))
    check_outputs(orc, W, AQ, Y.cpu().numpy(), K, N, M, "gemv+dbg")
    assert torch.equal(Y, Y2)  # the debug store does not change the arithmetic


FUSED_CASES = [(256, 1, 1, LAYOUT_MK), (5120, 333, 1, LAYOUT_MK), (8192, 333, 1, LAYOUT_MK), (17408, 40, 1, LAYOUT_MK),
               (768, 9, 2, LAYOUT_KM), (2048, 130, 4, LAYOUT_MK), (5120, 100, 6, LAYOUT_KM),
               (8192, 96, 7, LAYOUT_MK), (5120, 64, 8, LAYOUT_KM)]


@pytest.mark.parametrize("K,N,M,layout", FUSED_CASES)
def test_fused_quantize_gemv(pkg, orc, dev, K, N, M, layout):
    """One-launch path (Q8_1 quantisation in the GEMV prologue) against the
    two-launch path: the same codes, d and int32 sub-block sums always; for a
    single column the same kernel, hence bit-identical outputs; for several
    columns the two-launch path runs the matrix-core GEMV, whose fp32
    summation order differs (held to the path's tolerance instead)."""
    W = orc.gen_weights(K, N, seed=5000 + K + N)
    X = orc.gen_activations(K * M, seed=6000 + M, outliers=True).reshape(M, K)
    if M == 1 and K == 5120:
        X = rounding_boundary_blocks(K // 32, seed=12).reshape(1, K)
    AQ = orc.quantize_q8_1_batched(X, K, M, LAYOUT_MK)
    Wd = D(W, dev)
    Xd = D(X if layout == LAYOUT_MK else X.T, dev)
    Yf, Sf = pkg.mul_mat_fused(Wd, Xd, K, N, M, layout, sums=True)
    ws = pkg.quantize_q8_1(Xd, K, M, layout)
    Yp = pkg.mul_mat_q8_1(Wd, ws, K, N, M, layout, pkg.PATH_GEMV)
    torch.cuda.synchronize()
    assert np.array_equal(Sf.cpu().numpy(), orc.subblock_sums(W, AQ, K, N, M))
    if M == 1:
        assert torch.equal(Yf, Yp)
        assert torch.equal(pkg.mul_mat_fused(Wd, Xd, K, N, M, layout), Yp)  # without the debug store
    else:
        m = compute_metrics(Yp.cpu().numpy(), Yf.cpu().numpy())
        assert m["rel_l2"] <= REL_L2_TOL and not m["bad"], m
    Ymn = Yf.cpu().numpy() if layout == LAYOUT_MK else Yf.cpu().numpy().T
    check_outputs(orc, W, AQ, Ymn, K, N, M, "fused")


@pytest.mark.parametrize("K,N", [(5120, 333), (17408, 40), (20480, 17)])
def test_fused_single_column_unaligned_x(pkg, orc, dev, K, N):
    """A single column whose fp32 activations start 4 bytes past a 16-byte
    boundary takes the per-element prologue loads instead of the 16-byte
    vector loads; both must give the two-launch path's bits."""
    W = orc.gen_weights(K, N, seed=5100 + K + N)
    X = orc.gen_activations(K, seed=6100, outliers=True).reshape(1, K)
    AQ = orc.quantize_q8_1_batched(X, K, 1, LAYOUT_MK)
    Wd = D(W, dev)
    buf = torch.zeros(K + 4, dtype=torch.float32, device=dev)
    buf[1:K + 1] = D(X.reshape(K), dev)
    Xu = buf[1:K + 1]
    assert Xu.data_ptr() % 16 == 4
    Yd, Sf = pkg.mul_mat_fused(Wd, Xu, K, N, 1, LAYOUT_MK, sums=True)  # the debug-store instance
    Yf = pkg.mul_mat_fused(Wd, Xu, K, N, 1, LAYOUT_MK)                   # per-element loads
    Ya = pkg.mul_mat_fused(Wd, D(X, dev), K, N, 1, LAYOUT_MK)            # 16-byte loads
    Yp = pkg.mul_mat_q8_1(Wd, pkg.quantize_q8_1(D(X, dev), K, 1, LAYOUT_MK), K, N, 1, LAYOUT_MK, pkg.PATH_GEMV)
    # the public entry: an aligned column fuses up to K = 20480, an unaligned one
    # up to K = 8192 (past it: quantiser launch + GEMV); the same bits either way
    Ym = pkg.mul_mat(Wd, D(X, dev), K, N, 1, LAYOUT_MK)
    Ymu = pkg.mul_mat(Wd, Xu, K, N, 1, LAYOUT_MK)
    torch.cuda.synchronize()
    assert np.array_equal(Sf.cpu().numpy(), orc.subblock_sums(W, AQ, K, N, 1))
    assert torch.equal(Yd, Yp) and torch.equal(Yf, Yp) and torch.equal(Ya, Yp)
    assert torch.equal(Ym, Yp) and torch.equal(Ymu, Yp)
    check_outputs(orc, W, AQ, Yf.cpu().numpy(), K, N, 1, "fused-unaligned")


def test_fused_rejects_oversized_activations(pkg, dev):
    K, N, M = 17408, 64, 8  # 8 x 17408 codes exceed the on-chip activation buffer
    W = torch.zeros(N * K // 256 * 136, dtype=torch.uint8, device=dev)
    X = torch.zeros((M, K), dtype=torch.float32, device=dev)
    with pytest.raises(pkg.Iq4xsError) as e:
        pkg.mul_mat_fused(W, X, K, N, M)
    assert e.value.code == pkg.ERROR_NOT_SUPPORTED
    with pytest.raises(pkg.Iq4xsError) as e:
        pkg.mul_mat_fused(W, X, K, N, 9)
    assert e.value.code == pkg.ERROR_NOT_SUPPORTED


GEMM_CASES = [(256, 64, 64), (256, 1, 1), (512, 100, 20), (768, 130, 65), (1024, 64, 128),
              (2048, 200, 100), (512, 64, 512), (256, 300, 9),
              # more row tiles than CUs: one super-block per row; then an odd super-block count
              # with ragged rows and tokens
              (256, 128 * 148, 64), (768, 128 * 145 + 33, 33),
              # more than one round of 128-row tiles on 256 CUs with a short last round: the round
              # planner gives the tail smaller token tiles (the debug export keeps one segment of
              # full tiles, so the equality with it below pins every plan bit for bit)
              (256, 128 * 276 + 5, 100), (256, 128 * 68 + 7, 512)]


@pytest.mark.parametrize("K,N,M", GEMM_CASES)
def test_gemm_sums_and_outputs(pkg, orc, dev, K, N, M):
    W = orc.gen_weights(K, N, seed=3000 + K + N)
    X = orc.gen_activations(K * M, seed=4000 + M, outliers=True).reshape(M, K)
    AQ = orc.quantize_q8_1_batched(X, K, M, LAYOUT_MK)
    Wd = D(W, dev)
    ws = pkg.quantize_q8_1(D(X, dev), K, M, LAYOUT_MK)
    S, Y = pkg.subblock_sums(Wd, ws, K, N, M, pkg.PATH_GEMM)
    Y2 = pkg.mul_mat_q8_1(Wd, ws, K, N, M, LAYOUT_MK, pkg.PATH_GEMM)
    Ykm = pkg.mul_mat_q8_1(Wd, ws, K, N, M, LAYOUT_KM, pkg.PATH_GEMM)
    torch.cuda.synchronize()
    assert np.array_equal(S.cpu().numpy(), orc.subblock_sums(W, AQ, K, N, M))
    check_outputs(orc, W, AQ, Y.cpu().numpy(), K, N, M, "gemm+dbg")
    assert torch.equal(Y, Y2)
    assert torch.equal(Ykm.T, Y2)


# fp16 super-block scales at the edges of the format: zero, the smallest subnormal, the
# smallest normal, one, the largest finite, and negatives of some (bit patterns)
EXTREME_D = np.array([0x0000, 0x0001, 0x0400, 0x3C00, 0x7BFF, 0x8400, 0x8001, 0xFBFF], np.uint16)


# N, M: bs=1 tile GEMV, matrix-core GEMV (M = 4, 8), the GEMM on one and on many row tiles
@pytest.mark.parametrize("N,M", [(2051, 1), (2051, 4), (2051, 8), (2051, 100), (128 * 145 + 3, 64)])
def test_extreme_weight_scales(pkg, orc, dev, N, M):
    """Each kernel family on weights whose fp16 d spans zero, subnormals and the largest
    finite values: the sub-block sums stay bit-exact and the outputs match the reference
    semantics."""
    K = 2048
    W = orc.gen_weights(K, N, seed=77)
    blocks = W.reshape(-1, 136)
    d = np.resize(EXTREME_D, blocks.shape[0])
    blocks[:, 0] = (d & 0xFF).astype(np.uint8)
    blocks[:, 1] = (d >> 8).astype(np.uint8)
    X = orc.gen_activations(K * M, seed=78, outliers=True).reshape(M, K)
    AQ = orc.quantize_q8_1_batched(X, K, M, LAYOUT_MK)
    Wd = D(W, dev)
    ws = pkg.quantize_q8_1(D(X, dev), K, M, LAYOUT_MK)
    S, Y = pkg.subblock_sums(Wd, ws, K, N, M, pkg.PATH_GEMV if M <= 8 else pkg.PATH_GEMM)
    Y2 = pkg.mul_mat_q8_1(Wd, ws, K, N, M, LAYOUT_MK)  # path AUTO: the same kernel
    torch.cuda.synchronize()
    assert np.array_equal(S.cpu().numpy(), orc.subblock_sums(W, AQ, K, N, M))
    assert torch.equal(Y, Y2)
    assert bool(torch.isfinite(Y).all())
    check_outputs(orc, W, AQ, Y.cpu().numpy(), K, N, M, f"extreme d, M={M}")

def test_gemv_and_gemm_paths_agree(pkg, orc, dev):
    K, N, M = 2048, 256, 8
    W = D(orc.gen_weights(K, N, seed=5), dev)
    X = D(orc.gen_activations(K * M, seed=6).reshape(M, K), dev)
    ws = pkg.quantize_q8_1(X, K, M)
    S1, Y1 = pkg.subblock_sums(W, ws, K, N, M, pkg.PATH_GEMV)
    S2, Y2 = pkg.subblock_sums(W, ws, K, N, M, pkg.PATH_GEMM)
    torch.cuda.synchronize()
    assert torch.equal(S1, S2)
    assert compute_metrics(Y1.cpu().numpy(), Y2.cpu().numpy())["rel_l2"] < 1e-6


# ------------------------------------------------------------------ reference entry points
def test_reference_entry_points(pkg, orc, dev):
    L = pkg.lib()
    K, N = 5120, 160
    W = orc.gen_weights(K, N, seed=77)
    x = orc.gen_activations(K, seed=78)
    AQ = orc.quantize_q8_1(x)
    y_sem = orc.gemv_semantics(W, AQ, K, N)
    Wd, xd = D(W, dev), D(x, dev)
    for fn in ("gemv_iq4xs_stock_dp4a_gpu", "gemv_iq4xs_dp4a_coop_gpu", "custom_gemv_iq4xs_dispatch"):
        y = torch.full((N,), float("nan"), device=dev)
        L.check(fn, Wd.data_ptr(), xd.data_ptr(), y.data_ptr(), K, N, stream())
        torch.cuda.synchronize()
        assert compute_metrics(y_sem, y.cpu().numpy())["rel_l2"] <= REL_L2_TOL, fn
    # standalone GEMM: X[k*M+m] -> Y[n*M+m] (real_stock_dp4a_comparator.hip:505-512)
    for M in (4, 96):
        X_km = orc.gen_activations(K * M, seed=79 + M).reshape(K, M)
        AQm = orc.quantize_q8_1_batched(X_km, K, M, LAYOUT_KM)
        Y_sem = orc.gemm_semantics(W, AQm, K, N, M)          # [N, M]
        Y = torch.full((N, M), float("nan"), device=dev)
        Xkm_d, Xmk_d = D(X_km, dev), D(X_km.T, dev)
        L.check("gemm_iq4xs_stock_dp4a_gpu", Wd.data_ptr(), Xkm_d.data_ptr(), Y.data_ptr(), K, N, M, stream())
        # ggml: X[m*K+k] -> Y[m*N+n] (patch:117,129)
        Yg = torch.full((M, N), float("nan"), device=dev)
        L.check("custom_gemm_iq4xs_dispatch", Wd.data_ptr(), Xmk_d.data_ptr(), Yg.data_ptr(), K, N, M,
                stream())
        torch.cuda.synchronize()
        assert compute_metrics(Y_sem, Y.cpu().numpy())["rel_l2"] <= REL_L2_TOL
        assert compute_metrics(Y_sem.T, Yg.cpu().numpy())["rel_l2"] <= REL_L2_TOL


def test_invalid_arguments_on_gpu(pkg, dev):
    L = pkg.lib()
    W = torch.zeros(136 * 4, dtype=torch.uint8, device=dev)
    x = torch.zeros(256, device=dev)
    y = torch.zeros(4, device=dev)
    assert L.gemv_iq4xs_stock_dp4a_gpu(W.data_ptr(), x.data_ptr(), y.data_ptr(), 255, 4, stream()) == 1
    assert L.iq4xs_mul_mat_q8_1(W.data_ptr(), x.data_ptr() + 4, y.data_ptr(), 256, 4, 1, LAYOUT_MK, -1,
                                stream()) == 1  # misaligned workspace
    assert L.iq4xs_mul_mat_q8_1(W.data_ptr(), x.data_ptr(), y.data_ptr(), 256, 4, 9, LAYOUT_MK, pkg.PATH_GEMV,
                                stream()) == 1  # GEMV serves at most 8 columns


# ------------------------------------------------------------------ full-size shapes
@pytest.mark.parametrize("proj", list(CONFIG1))
def test_config1_gemv_bs1_full_size(pkg, orc, dev, proj):
    K, N = CONFIG1[proj]
    W = pkg.synthetic_weights(K, N, seed=42, device=dev)
    x = orc.gen_activations(K, seed=43)
    y = pkg.mul_mat(W, D(x, dev), K, N, 1)
    torch.cuda.synchronize()
    Wh = W.cpu().numpy()
    AQ = orc.quantize_q8_1(x)
    y_sem = orc.gemv_semantics(Wh, AQ, K, N)
    m = compute_metrics(y_sem, y.cpu().numpy().ravel())
    assert m["rel_l2"] <= REL_L2_TOL, m
    y_hat = orc.gemv_fp64(Wh, orc.dequant_q8_1(AQ), K, N)
    assert compute_metrics(y_hat, y.cpu().numpy().ravel())["cosine"] >= COS_TOL


def sampled_rows(W, N, rows):
    """Rows `rows` of a device weight matrix [N][K/256 blocks], gathered on the device."""
    idx = torch.from_numpy(np.asarray(rows, np.int64)).to(W.device)
    return W.view(N, -1)[idx].cpu().numpy().ravel()


@pytest.mark.parametrize("M", [2, 4, 8])
@pytest.mark.parametrize("proj", list(CONFIG1))
def test_config2_small_batch_full_size(pkg, orc, dev, proj, M):
    """Every config-1 projection at bs = 2, 4, 8 with 1 % x20 outlier activations,
    through iq4xs_mul_mat (quantiser + the small-batch GEMV the shape routes to: the
    dot4 tile kernel, or the matrix-core GEMV for M >= 4 and N >= 2048)."""
    print(f"config2 {proj} M={M}", flush=True)
    K, N = CONFIG1[proj]
    W = pkg.synthetic_weights(K, N, seed=44, device=dev)
    X = orc.gen_activations(K * M, seed=45 + M, outliers=True).reshape(M, K)
    Xd = D(X, dev)
    ws = pkg.workspace(K, M, dev)
    Y = pkg.mul_mat(W, Xd, K, N, M, ws=ws)
    torch.cuda.synchronize()
    AQ = orc.quantize_q8_1_batched(X, K, M, LAYOUT_MK)
    assert np.array_equal(pkg.q8_1_blocks(ws, K, M).cpu().numpy().ravel(), AQ)
    rows = np.sort(np.random.default_rng(M).choice(N, 256, replace=False))
    Y_sem = orc.gemm_semantics(sampled_rows(W, N, rows), AQ, K, len(rows), M).T
    m = compute_metrics(Y_sem, Y.cpu().numpy()[:, rows])
    assert m["rel_l2"] <= REL_L2_TOL and not m["bad"], m


def dequantised_activations_km(pkg, ws, K, M):
    """x_hat = d * q of every Q8_1 block (exact in fp32), as X[k*M + m] on the device."""
    blk = pkg.q8_1_blocks(ws, K, M)
    d = blk[:, 0:2].contiguous().view(torch.float16).float()            # [M*K/32, 1]
    q = blk[:, 4:].contiguous().view(torch.int8).float()                # [M*K/32, 32]
    return (q * d).reshape(M, K).T.contiguous()


@pytest.mark.parametrize("M", [512, 2048])
@pytest.mark.parametrize("proj", list(CONFIG1))
def test_config3_prefill_gemm_full_size(pkg, orc, dev, proj, M):
    """Every config-1 projection at M = 512 and 2048, through the plans the round planner
    picks for these shapes (bulk and tail segments, 64-row tiles for k/v at M = 512).
    * Sampled rows, the first and last included, against the CPU oracle's reference kernel
      semantics (rel-L2 1e-4).
    * Every output against the reference's FP64 comparator (gemm_iq4xs_stock_gpu, pinned bit
      for bit to ref_cpu.cpp by the golden outputs) evaluated on the dequantised activations
      x_hat: the two differ by fp32 rounding only, so each weight row and each token is held
      to rel-L2 1e-4 on its own -- a wrong tile, segment or row anywhere fails -- and the
      whole output to cosine 0.99999."""
    print(f"config3 {proj} M={M}", flush=True)
    K, N = CONFIG1[proj]
    W = pkg.synthetic_weights(K, N, seed=46, device=dev)
    X = pkg.synthetic_activations(K * M, seed=47, device=dev)
    ws = pkg.quantize_q8_1(X, K, M)
    Y = pkg.mul_mat_q8_1(W, ws, K, N, M)
    torch.cuda.synchronize()
    AQ = pkg.q8_1_blocks(ws, K, M).cpu().numpy().ravel()
    assert np.array_equal(AQ, orc.quantize_q8_1_batched(X.cpu().numpy(), K, M, LAYOUT_MK))
    rng = np.random.default_rng(M + N)
    rows = np.unique(np.concatenate([[0, N - 1], rng.choice(N, 10, replace=False)]))
    Y_sem = orc.gemm_semantics(sampled_rows(W, N, rows), AQ, K, len(rows), M).T
    m = compute_metrics(Y_sem, Y.cpu().numpy()[:, rows])
    assert m["rel_l2"] <= REL_L2_TOL and not m["bad"], m
    # every output against FP64 on x_hat
    Y64 = torch.full((N, M), float("nan"), device=dev)
    xhat = dequantised_activations_km(pkg, ws, K, M)
    pkg.lib().check("gemm_iq4xs_stock_gpu", W.data_ptr(), xhat.data_ptr(), Y64.data_ptr(), K, N, M, stream())
    torch.cuda.synchronize()
    a, b = Y64.T.double(), Y.double()                                    # [M, N]
    assert bool(torch.isfinite(b).all()) and bool(torch.isfinite(a).all())
    err = (a - b).square()
    per_row = (err.sum(0) / a.square().sum(0)).sqrt()                   # each weight row n
    per_tok = (err.sum(1) / a.square().sum(1)).sqrt()                   # each token m
    assert float(per_row.max()) <= REL_L2_TOL, ("row", int(per_row.argmax()), float(per_row.max()))
    assert float(per_tok.max()) <= REL_L2_TOL, ("token", int(per_tok.argmax()), float(per_tok.max()))
    cos = float((a * b).sum() / (a.norm() * b.norm()))
    assert cos >= COS_TOL, cos


def test_deterministic_replay(pkg, dev):
    K, N, M = 5120, 1024, 64
    W = pkg.synthetic_weights(K, N, seed=1, device=dev)
    X = pkg.synthetic_activations(K * M, seed=2, device=dev)
    a = pkg.mul_mat(W, X, K, N, M)
    b = pkg.mul_mat(W, X, K, N, M)
    c = pkg.mul_mat(W, X[:K], K, N, 1)
    d = pkg.mul_mat(W, X[:K], K, N, 1)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(c, d)


# Non-finite fp16 super-block scales (+Inf, -Inf, NaN): every output keeps the reference's
# class (finite within tolerance, +Inf, -Inf or NaN), as the reference's product
# fp16(d_w) * fp16(d_x) * float(sumi * (ls - 32)) gives it.  So does an activation block whose
# Q8_1 scale overflows to +Inf (|x| >= 8.3e6): the GEMV paths carry it through, and the GEMM
# recomputes that token's outputs term by term (its scale MFMA would meet the Inf with the
# zero k slots of the other sub-blocks).
NONFINITE_D = np.array([0x7C00, 0xFC00, 0x7E00], np.uint16)


def check_classes(y_ref, y_gpu, label):
    ref_nan, gpu_nan = np.isnan(y_ref), np.isnan(y_gpu)
    assert np.array_equal(ref_nan, gpu_nan), f"{label}: NaN positions differ"
    for sgn in (1, -1):
        assert np.array_equal(y_ref == sgn * np.inf, y_gpu == sgn * np.inf), f"{label}: {sgn:+d} Inf positions differ"
    fin = np.isfinite(y_ref)
    assert fin.any() and (~fin).any(), label
    a, b = y_ref[fin].astype(np.float64), y_gpu[fin].astype(np.float64)
    assert np.linalg.norm(a - b) <= REL_L2_TOL * np.linalg.norm(a), label


def nonfinite_case(orc, M, inf_activation):
    K, N = 2048, 2051
    W = orc.gen_weights(K, N, seed=91)
    blocks = W.reshape(-1, 136)
    bpr = K // 256
    for j, r in enumerate(range(0, N, 37)):  # one super-block of every 37th row gets a non-finite d
        d = int(NONFINITE_D[j % 3])
        blocks[r * bpr + (j % bpr), 0] = d & 0xFF
        blocks[r * bpr + (j % bpr), 1] = d >> 8
    X = orc.gen_activations(K * M, seed=92, outliers=True).reshape(M, K)
    if inf_activation:
        X[M // 2, 300:340] = 3.0e7  # activation blocks whose fp16 d_x overflows to +Inf
    return K, N, W, X


# M: bs=1 tile GEMV, matrix-core GEMV (4, 8), fp16 matrix-core GEMM (64 one tile, 200 two token tiles)
@pytest.mark.parametrize("M", [1, 4, 8, 64, 200])
def test_nonfinite_weight_scales_keep_reference_classes(pkg, orc, dev, M):
    K, N, W, X = nonfinite_case(orc, M, inf_activation=False)
    AQ = orc.quantize_q8_1_batched(X, K, M, LAYOUT_MK)
    ws = pkg.quantize_q8_1(D(X, dev), K, M, LAYOUT_MK)
    Y = pkg.mul_mat_q8_1(D(W, dev), ws, K, N, M, LAYOUT_MK)
    torch.cuda.synchronize()
    y_ref = orc.gemm_semantics(W, AQ, K, N, M).T if M > 1 else orc.gemv_semantics(W, AQ, K, N)[None, :]
    check_classes(y_ref, Y.cpu().numpy().reshape(M, N), f"non-finite weight scales, M={M}")


# M: matrix-core GEMV (4, 8) and the GEMM (64: one token tile; 200: more than one), on
# weights that also carry non-finite scales
@pytest.mark.parametrize("M", [4, 8, 64, 200])
def test_infinite_activation_scale_keeps_reference_classes(pkg, orc, dev, M):
    print(f"Inf d_x M={M}", flush=True)
    K, N, W, X = nonfinite_case(orc, M, inf_activation=True)
    AQ = orc.quantize_q8_1_batched(X, K, M, LAYOUT_MK)
    y_ref = orc.gemm_semantics(W, AQ, K, N, M).T
    Wd, Xd = D(W, dev), D(X, dev)
    ws = pkg.quantize_q8_1(Xd, K, M, LAYOUT_MK)
    path = pkg.PATH_GEMV if M <= 8 else pkg.PATH_GEMM
    Y = pkg.mul_mat_q8_1(Wd, ws, K, N, M, LAYOUT_MK, path)
    # the ggml mmq hook (patch:299-306) on the same activations, ggml layout
    Yg = torch.full((M, N), float("nan"), device=dev)
    pkg.lib().check("custom_gemm_iq4xs_dispatch", Wd.data_ptr(), Xd.data_ptr(), Yg.data_ptr(), K, N, M, stream())
    torch.cuda.synchronize()
    check_classes(y_ref, Y.cpu().numpy().reshape(M, N), f"Inf d_x, M={M}")
    check_classes(y_ref, Yg.cpu().numpy(), f"Inf d_x through the mmq hook, M={M}")
    # the rows of the token with the infinite scale are all non-finite, the other tokens' finite
    # where the weights are
    bad = M // 2
    assert not np.isfinite(y_ref[bad]).any()
