"""Pins the CPU oracle (oracle/iq4xs_oracle.c) before it is trusted as the
checker: reference golden vectors and KATs, hand-derived known answers, and
independent numpy formulations chosen so that the plausible mistakes
(RNE instead of truncation, x*(1/d) instead of x/d, rint instead of roundf,
sequential instead of tree sums, swapped nibble halves, wrong scale bits)
each fail at least one test."""
import hashlib
import json
import os

import numpy as np
import pytest

from oracle.oracle import (BLOCK_IQ4_XS, BLOCK_Q8_1, KVALUES_IQ4NL, LAYOUT_KM, LAYOUT_MK, RefCpu, compute_metrics,
                           ref_available)

GOLDEN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ---------------------------------------------------------------- helpers
def np_trunc_fp16_bits(f):
    """Round-toward-zero binary16, built from numpy's round-to-nearest-even
    conversion plus a one-ulp correction; |x| >= 65536, Inf, NaN -> signed Inf."""
    f = np.asarray(f, dtype=np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        h = f.astype(np.float16)
    bits = h.view(np.uint16).copy()
    back = h.astype(np.float32)
    with np.errstate(invalid="ignore"):
        away = np.isfinite(f) & (np.abs(back) > np.abs(f))
    bits[away] -= 1
    sign = (f.view(np.uint32) >> 16).astype(np.uint16) & np.uint16(0x8000)
    big = ~np.isfinite(f) | (np.abs(f) >= 65536.0)
    bits[big] = sign[big] | np.uint16(0x7C00)
    return bits


def np_quant_block(x):
    """Independent numpy formulation of the reference device quantiser."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.float32(np.abs(x).max())
    s = x.copy()
    w = 16
    while w >= 1:
        s = (s[:w] + s[w:2 * w]).astype(np.float32)
        w //= 2
    d = np.float32(amax / np.float32(127.0))
    if amax == 0:
        q = np.zeros(32, np.int8)
    else:
        v = (x / d).astype(np.float32).astype(np.float64)
        q = (np.sign(v) * np.floor(np.abs(v) + 0.5)).astype(np.int8)
    ds = int(np_trunc_fp16_bits(d)) | (int(np_trunc_fp16_bits(s[0])) << 16)
    return ds, q


def decode_weights_np(W, K, N):
    """int codebook values [N, K] and 6-bit scales [N, K/32] from raw bytes."""
    B = W.view(BLOCK_IQ4_XS).reshape(N, K // 256)
    qs = B["qs"].reshape(N, K // 256, 8, 16)
    lo = KVALUES_IQ4NL[qs & 15].astype(np.int64)
    hi = KVALUES_IQ4NL[qs >> 4].astype(np.int64)
    vals = np.concatenate([lo, hi], axis=3).reshape(N, K)
    sl = B["scales_l"].astype(np.int64)  # [N, bpr, 4]
    sh = B["scales_h"].astype(np.int64)  # [N, bpr]
    ib = np.arange(8)
    ls = ((sl[:, :, ib // 2] >> (4 * (ib & 1))) & 15) | (((sh[:, :, None] >> (2 * ib)) & 3) << 4)
    d = B["d"].view(np.float16).astype(np.float64)
    return vals, ls.reshape(N, K // 32), d


def np_subblock_sums(W, AQ, K, N, M):
    vals, ls, _ = decode_weights_np(W, K, N)
    q = AQ.view(BLOCK_Q8_1).reshape(M, K // 32)["qs"].astype(np.int64)
    S = np.einsum("nkt,mkt->mnk", vals.reshape(N, K // 32, 32), q)
    return S * (ls - 32)[None]


def np_dequant64(W, K, N):
    vals, ls, d = decode_weights_np(W, K, N)
    scale = np.repeat(d, 8, axis=1) * (ls - 32)
    return vals * np.repeat(scale, 32, axis=1)


# ---------------------------------------------------------------- fp16 codecs
def test_fp16_decode_exhaustive(orc):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.fp16_to_fp32(h).view(np.uint32)
    ref = h.view(np.float16).astype(np.float32).view(np.uint32)
    nan = (h & 0x7C00) == 0x7C00
    nan &= (h & 0x3FF) != 0
    assert np.array_equal(got[~nan], ref[~nan])
    # NaN: sign | Inf exponent | payload << 13, bit for bit (block_iq4_xs.h:52-54)
    hn = h[nan].astype(np.uint32)
    expect = ((hn & 0x8000) << 16) | 0x7F800000 | ((hn & 0x3FF) << 13)
    assert np.array_equal(got[nan], expect)


def test_fp16_trunc_encode_structured(orc):
    exps = np.arange(256, dtype=np.uint32)
    mants = np.array([0, 1, 0xFFF, 0x1000, 0x1001, 0x1FFF, 0x2000, 0x2001, 0x3FFF, 0x400000, 0x7FE000,
                      0x7FEFFF, 0x7FF000, 0x7FFFFF], dtype=np.uint32)
    bits = (exps[:, None] << 23 | mants[None, :]).ravel()
    bits = np.concatenate([bits, bits | 0x80000000])
    rng = np.random.default_rng(1)
    bits = np.concatenate([bits, rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)])
    f = bits.view(np.float32)
    assert np.array_equal(orc.fp32_to_fp16_trunc(f), np_trunc_fp16_bits(f))


def test_fp16_trunc_known_answers(orc):
    cases = [
        (1.0, 0x3C00), (-1.0, 0xBC00), (0.0, 0x0000), (-0.0, 0x8000),
        (1.0009765, 0x3C00),          # just below 1 + 2^-10: truncates (RNE would give 0x3C01)
        (65519.0, 0x7BFF), (65535.0, 0x7BFF), (65536.0, 0x7C00),
        (2.0**-24, 0x0001), (2.0**-25, 0x0000), (1.5 * 2.0**-24, 0x0001),
        (float("inf"), 0x7C00), (float("-inf"), 0xFC00), (float("nan"), 0x7C00),
    ]
    for v, want in cases:
        assert int(orc.fp32_to_fp16_trunc(np.array([v], np.float32))[0]) == want, v


# ---------------------------------------------------------------- format KATs
def test_kat_blocks_sha256_and_values(orc):
    with open(os.path.join(GOLDEN_DIR, "iq4xs_kat_blocks.json")) as f:
        kat = json.load(f)
    assert len(kat["cases"]) == 5
    for case in kat["cases"]:
        raw = bytes.fromhex(case["raw_hex"])
        assert hashlib.sha256(raw).hexdigest() == case["raw_sha256_reference"], case["name"]
        W = np.frombuffer(raw, np.uint8).copy()
        n = case["n_blocks"]
        deq = orc.dequant(W, 256, n)
        for blk, elem, value in case["hand_values"]:
            assert deq[int(blk), int(elem)] == np.float32(value), (case["name"], blk, elem)
        # the FP64 GEMV on one-hot activations reproduces each column of the dequantised block
        for blk, elem, value in case["hand_values"]:
            x = np.zeros(256, np.float32)
            x[int(elem)] = 1.0
            y = orc.gemv_fp64(W, x, 256, n)
            assert y[int(blk)] == np.float32(value)


def test_block_layout_scale_bits(orc):
    rng = np.random.default_rng(3)
    W = rng.integers(0, 256, 136 * 64, dtype=np.uint8)
    _, ls_np, _ = decode_weights_np(W, 256 * 8, 8)
    blocks = W.view(BLOCK_IQ4_XS)
    for b in range(64):
        for ib in range(8):
            assert orc.lib.orc_subblock_scale(W.ctypes.data + 136 * b, ib) == ls_np.reshape(-1, 8)[b, ib]
    assert blocks.itemsize == 136


# ---------------------------------------------------------------- Q8_1
def q8(orc, x):
    y = orc.quantize_q8_1(np.asarray(x, np.float32)).view(BLOCK_Q8_1)
    return int(y["ds"][0]), y["qs"][0].copy()


def test_q8_1_zero_block(orc):
    ds, q = q8(orc, np.zeros(32))
    assert ds == 0 and not q.any()


def test_q8_1_single_nonzero(orc):
    x = np.zeros(32, np.float32)
    x[5] = 3.0
    ds, q = q8(orc, x)
    assert q[5] == 127 and np.count_nonzero(q) == 1
    assert ds >> 16 == 0x4200  # sum 3.0
    assert ds & 0xFFFF == int(np_trunc_fp16_bits(np.float32(3.0) / np.float32(127.0)))
    x[5] = -2.5
    ds, q = q8(orc, x)
    assert q[5] == -127 and ds >> 16 == 0xC100


def test_q8_1_ties_round_half_away(orc):
    # amax 127 -> d = 1 exactly, so x/d = x; roundf sends .5 away from zero (rint would not)
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:9] = [2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 3.5, 126.5]
    _, q = q8(orc, x)
    assert list(q[:9]) == [127, 3, -3, 1, -1, 2, -2, 4, 127]


def test_q8_1_negative_zero(orc):
    x = np.zeros(32, np.float32)
    x[0] = 1.0
    x[1] = -0.0
    ds, q = q8(orc, x)
    assert q[1] == 0 and q[0] == 127


def test_q8_1_tree_sum_order(orc):
    # tree: (x0 + x16) = 1 exactly, then + 0.75 -> 1.75; a sequential sum
    # absorbs 0.75 into 2^24 first and ends at 1.0
    x = np.zeros(32, np.float32)
    x[0] = 2.0**24
    x[16] = -(2.0**24 - 1)
    x[1] = 0.75
    ds, q = q8(orc, x)
    assert ds >> 16 == 0x3F00      # trunc-fp16(1.75)
    assert ds & 0xFFFF == 0x7C00   # d = 2^24/127 overflows fp16 -> Inf
    assert q[0] == 127 and q[16] == -127 and q[1] == 0


def test_q8_1_division_not_reciprocal(orc):
    """A block where roundf(x*(1/d)) != roundf(x/d): pins true division."""
    rng = np.random.default_rng(11)

    def rnd(v):
        v = v.astype(np.float32).astype(np.float64)
        return np.sign(v) * np.floor(np.abs(v) + 0.5)

    found = 0
    for _ in range(4000):
        amax = np.float32(rng.uniform(0.5, 4.0))
        d = np.float32(amax / np.float32(127.0))
        k = rng.integers(1, 126)
        x0 = np.float32((k + 0.5) * np.float64(d))  # near a .5 quotient boundary
        cand = np.nextafter(x0, np.float32(np.inf) if rng.random() < 0.5 else np.float32(0), dtype=np.float32)
        for xv in (x0, cand):
            x = np.zeros(32, np.float32)
            x[0] = amax
            x[1] = xv
            if rnd(x / d)[1] != rnd(x * (np.float32(1.0) / d))[1]:
                _, q = q8(orc, x)
                assert q[1] == rnd(x / d)[1]
                found += 1
    assert found >= 3


@pytest.mark.parametrize("outliers", [False, True])
def test_q8_1_brute_force_vs_numpy(orc, outliers):
    x = orc.gen_activations(32 * 512, seed=5, outliers=outliers)
    y = orc.quantize_q8_1(x).view(BLOCK_Q8_1)
    for b in range(512):
        ds, q = np_quant_block(x[32 * b:32 * b + 32])
        assert int(y["ds"][b]) == ds and np.array_equal(y["qs"][b], q), b


def test_q8_1_batched_layouts(orc):
    K, M = 256, 5
    X = orc.gen_activations(K * M, seed=9).reshape(M, K)
    rows = np.concatenate([orc.quantize_q8_1(X[m]) for m in range(M)])
    assert np.array_equal(orc.quantize_q8_1_batched(X, K, M, LAYOUT_MK), rows)
    assert np.array_equal(orc.quantize_q8_1_batched(np.ascontiguousarray(X.T), K, M, LAYOUT_KM), rows)


# ---------------------------------------------------------------- integer sums
@pytest.mark.parametrize("K,N,M", [(256, 3, 1), (768, 5, 3), (1024, 4, 2)])
def test_subblock_sums_brute_force(orc, K, N, M):
    W = orc.gen_weights(K, N, seed=K + N)
    AQ = orc.quantize_q8_1_batched(orc.gen_activations(K * M, seed=M, outliers=True), K, M, LAYOUT_MK)
    assert np.array_equal(orc.subblock_sums(W, AQ, K, N, M), np_subblock_sums(W, AQ, K, N, M))


def test_subblock_sums_extremes(orc):
    # all codes 0 (kv -127) against all activations -127 with ls = 0 -> -32:
    # 32 * 16129 * -32 = -16516096, the most negative sum
    W = np.zeros(136, np.uint8)
    W[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    x = np.full(256, -1.0, np.float32)
    AQ = orc.quantize_q8_1(x)
    S = orc.subblock_sums(W, AQ, 256, 1, 1)
    assert np.all(S == 32 * 127 * 127 * -32)


# ---------------------------------------------------------------- FP64 oracle vs reference golden
GOLDEN_CASES = ["gemv_512x48", "gemv_1024x16_outliers", "gemv_768x8_odd_superblocks", "gemm_512x16x8",
                "gemm_256x8x5"]


@pytest.mark.parametrize("name", GOLDEN_CASES)
def test_fp64_oracle_matches_reference_golden(orc, golden, name):
    K, N, M = (int(v) for v in golden[f"{name}.shape"])
    W = golden[f"{name}.W"]
    assert np.array_equal(W, orc.gen_weights(K, N, seed={"gemv_512x48": 101, "gemv_1024x16_outliers": 102,
                                                          "gemv_768x8_odd_superblocks": 103, "gemm_512x16x8": 104,
                                                          "gemm_256x8x5": 105}[name]))
    if M == 1:
        y = orc.gemv_fp64(W, golden[f"{name}.x"], K, N)
        assert np.array_equal(y.view(np.uint32), golden[f"{name}.y"].view(np.uint32))
    else:
        Y = orc.gemm_fp64(W, golden[f"{name}.X_km"], K, N, M, nthreads=2)
        assert np.array_equal(Y.view(np.uint32), golden[f"{name}.Y"].view(np.uint32))
    assert np.array_equal(orc.dequant(W, K, N), golden[f"{name}.dequant"])


@pytest.mark.skipif(not ref_available(), reason="reference not mounted (oracle/_ref not built)")
def test_fp64_oracle_matches_reference_live(orc):
    ref = RefCpu()
    for K, N, seed in [(1280, 24, 1), (2048, 9, 2)]:
        W = orc.gen_weights(K, N, seed)
        x = orc.gen_activations(K, seed, outliers=True)
        assert np.array_equal(orc.gemv_fp64(W, x, K, N), ref.gemv_fp64(W, x, K, N))


def test_fp64_oracle_vs_numpy_float64(orc):
    K, N = 1536, 32
    W = orc.gen_weights(K, N, seed=21)
    x = orc.gen_activations(K, seed=22)
    ref = (np_dequant64(W, K, N) @ x.astype(np.float64)).astype(np.float32)
    y = orc.gemv_fp64(W, x, K, N)
    assert np.max(np.abs(y - ref) / np.maximum(np.abs(ref), 1e-3)) < 1e-6


# ---------------------------------------------------------------- reference kernel semantics model
def test_semantics_gemv_vs_fp64_on_dequantised_activations(orc):
    K, N = 5120, 64
    W = orc.gen_weights(K, N, seed=31)
    x = orc.gen_activations(K, seed=32)
    AQ = orc.quantize_q8_1(x)
    y = orc.gemv_semantics(W, AQ, K, N)
    y_hat = orc.gemv_fp64(W, orc.dequant_q8_1(AQ), K, N)
    m = compute_metrics(y_hat, y)
    assert m["cosine"] >= 0.99999 and m["rel_l2"] < 1e-5
    # on raw x a Q8_1 path sits near 0.999986 (kernels/matmul_iq4xs/BASELINE_DP4A.md:30)
    m_raw = compute_metrics(orc.gemv_fp64(W, x, K, N), y)
    assert 0.9999 < m_raw["cosine"] < 0.999999


def test_semantics_gemm_and_gemv_agree(orc):
    K, N = 1024, 16
    W = orc.gen_weights(K, N, seed=41)
    AQ = orc.quantize_q8_1(orc.gen_activations(K, seed=42))
    a = orc.gemv_semantics(W, AQ, K, N)
    b = orc.gemm_semantics(W, AQ, K, N, 1)[:, 0]
    assert compute_metrics(a, b)["rel_l2"] < 1e-6


def test_semantics_terms_are_exact_products(orc):
    """One sub-block: the semantics model returns fp16(d_w)*fp16(d_x)*sumi
    rounded once (the exact terms are checked through orc_subblock_sums)."""
    W = orc.gen_weights(256, 1, seed=51)
    W[8 + 16:] = 0x88  # sub-blocks 1..7: every code 8 (kvalue +1)
    blk = W.view(BLOCK_IQ4_XS)
    blk["scales_l"][0] = [0x00, 0x00, 0x00, 0x00]
    blk["scales_h"][0] = 2  # sub-block 0: ls = 0 | 2<<4 = 32 -> factor 0; sub-blocks 1..7: ls = 0 -> -32
    x = orc.gen_activations(256, seed=52)
    AQ = orc.quantize_q8_1(x)
    S = orc.subblock_sums(W, AQ, 256, 1, 1)[0, 0]
    dw = np.float32(blk["d"].view(np.float16)[0])
    dx = AQ.view(BLOCK_Q8_1)["ds"].astype(np.uint32) & 0xFFFF
    dx = dx.astype(np.uint16).view(np.float16).astype(np.float32)
    terms = [(np.float32(dw * dx[k]) * np.float32(S[k])).astype(np.float32) for k in range(8)]
    assert S[0] == 0  # scale 32 -> factor 0
    y = orc.gemm_semantics(W, AQ, 256, 1, 1)[0, 0]
    acc = np.float32(0)
    for t in terms:
        acc = np.float32(acc + t)
    assert y == acc


# ---------------------------------------------------------------- generator
def test_generator_distribution(orc):
    K, N = 4096, 64
    W = orc.gen_weights(K, N, seed=42)
    vals, ls, d = decode_weights_np(W, K, N)
    assert d.min() >= 0.00499 and d.max() < 0.02
    counts = np.bincount(ls.ravel(), minlength=64)
    assert counts.min() > 60 and counts.max() < 200
    codes = np.concatenate([W.view(BLOCK_IQ4_XS)["qs"].ravel() & 15, W.view(BLOCK_IQ4_XS)["qs"].ravel() >> 4])
    freq = np.bincount(codes, minlength=16) / codes.size
    assert np.all(np.abs(freq - 1 / 16) < 0.01)
    # counter-based: block i of a matrix == block first_block + i generated alone
    part = orc.gen_weights(256, 5, seed=42, first_block=77)
    assert np.array_equal(part, W[77 * 136:82 * 136])


def test_generator_activations(orc):
    x = orc.gen_activations(200000, seed=3)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01
    xo = orc.gen_activations(200000, seed=3, outliers=True)
    frac = np.mean(xo != x)
    assert 0.008 < frac < 0.012
    assert np.allclose(xo[xo != x], 20 * x[xo != x])


def test_compute_metrics():
    r = np.array([1.0, -2.0, 3.0], np.float32)
    m = compute_metrics(r, r)
    assert m["cosine"] == pytest.approx(1.0) and m["max_abs"] == 0 and m["pass"]
    m = compute_metrics(r, -r)
    assert m["cosine"] == pytest.approx(-1.0) and not m["pass"]
    assert compute_metrics(r, np.array([1, -2, np.nan], np.float32))["bad"]


# ---------------------------------------------------------------- dequant mutation control
def dequant_gate(ref, got):
    """Acceptance gate of the reference's dequant harness
    (kernels/demo_iq4xs_dequant/test_compare.cpp:76-111): max_abs < 1e-5,
    mean_abs < 1e-6, cosine >= 0.99999, no NaN/Inf."""
    ref = ref.astype(np.float64).ravel()
    got = got.astype(np.float64).ravel()
    diff = np.abs(ref - got)
    denom = np.linalg.norm(ref) * np.linalg.norm(got)
    cos = float(ref @ got / denom) if denom > 1e-12 else 1.0
    return bool(np.isfinite(got).all() and diff.max() < 1e-5 and diff.mean() < 1e-6 and cos >= 0.99999)


def np_dequant_fp32(W, K, N, mutate=None):
    """fp32 dequant in the reference's operation order (dl = d*(ls-32) in fp32,
    then dl*kv), optionally with the reference's planted bugs
    (kernels/demo_iq4xs_dequant/impl_broken.hip:33-46): 'scale' builds ls with
    hi << 3, 'swap' swaps the nibbles."""
    B = W.view(BLOCK_IQ4_XS).reshape(N, K // 256)
    qs = B["qs"].reshape(N, K // 256, 8, 16)
    lo_n, hi_n = (qs >> 4, qs & 15) if mutate == "swap" else (qs & 15, qs >> 4)
    vals = np.concatenate([KVALUES_IQ4NL[lo_n], KVALUES_IQ4NL[hi_n]], axis=3).astype(np.float32)
    sl = B["scales_l"].astype(np.int64)
    sh = B["scales_h"].astype(np.int64)
    ib = np.arange(8)
    shift = 3 if mutate == "scale" else 4
    ls = ((sl[:, :, ib // 2] >> (4 * (ib & 1))) & 15) | (((sh[:, :, None] >> (2 * ib)) & 3) << shift)
    d = B["d"].view(np.float16).astype(np.float32)
    dl = (d[:, :, None] * (ls.astype(np.float32) - np.float32(32.0))).astype(np.float32)
    return (dl[:, :, :, None] * vals).astype(np.float32).reshape(N, K)


def test_dequant_mutation_control(orc, golden):
    """The comparison discriminates: the oracle and the fp32 restatement
    match the reference's own dequant outputs bit for bit, while each of the
    reference's planted bugs, applied to the restatement, fails the
    reference's gate (the mistakes are planted here on the CPU, never in a
    GPU kernel)."""
    for name in ("gemv_512x48", "gemm_256x8x5"):
        W = golden[name + ".W"]
        K, N = (int(v) for v in golden[name + ".shape"][:2])
        ref = golden[name + ".dequant"].astype(np.float32).reshape(N, K)
        assert np.array_equal(orc.dequant(W, K, N).view(np.uint32), ref.view(np.uint32))
        assert np.array_equal(np_dequant_fp32(W, K, N).view(np.uint32), ref.view(np.uint32))
        assert dequant_gate(ref, np_dequant_fp32(W, K, N))
        for bug in ("scale", "swap"):
            assert not dequant_gate(ref, np_dequant_fp32(W, K, N, mutate=bug)), (name, bug)


def test_fp64_by_subblock_order(orc, golden):
    """The gfx1100 FP64 order (8 per-sub-block partials, then added) holds the
    same products as ref_cpu.cpp in another order: against the reference's
    own FP64 outputs it may differ by the final float rounding only, and
    against numpy float64 it is exact to 1e-12."""
    for name in ("gemv_512x48", "gemv_768x8_odd_superblocks", "gemv_1024x16_outliers"):
        W, x, y_ref = golden[name + ".W"], golden[name + ".x"], golden[name + ".y"].astype(np.float32)
        K, N = (int(v) for v in golden[name + ".shape"][:2])
        y = orc.gemv_fp64_by_subblock(W, x, K, N)
        ulp = np.abs(y.astype(np.float64) - y_ref.astype(np.float64)) / np.spacing(np.abs(y_ref)).astype(np.float64)
        assert ulp.max() <= 1.0, (name, ulp.max())
        y64 = np_dequant64(W, K, N) @ x.astype(np.float64)
        assert np.allclose(y, y64, rtol=1e-6, atol=1e-6)


def test_fp64_by_subblock_order_is_distinguishable(orc):
    """A cancellation that only the per-sub-block order survives: every weight
    is exactly 1 (d = 1.0, ls = 33, code 8 -> +1), and x holds +2^80 at
    (super-block 0, sub-block 0), 1 at (0, 1) and -2^80 at (1, 0).  The
    sequential order of ref_cpu.cpp adds 1 to 2^80 (lost) and ends at 0; the
    gfx1100 order cancels sub-block 0's partial first and ends at 1."""
    K, N = 512, 2
    blk = np.zeros(136, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[2:4] = (0xAA, 0xAA)          # hi bits 2 for every sub-block
    blk[4:8] = 0x11                  # lo bits 1 for every sub-block -> ls = 33
    blk[8:] = 0x88                   # both nibbles code 8 -> kvalue +1
    W = np.tile(blk, K // 256 * N)
    x = np.zeros(K, np.float32)
    x[0], x[32], x[256] = 2.0 ** 80, 1.0, -(2.0 ** 80)
    assert np.array_equal(orc.gemv_fp64(W, x, K, N), np.zeros(N, np.float32))
    assert np.array_equal(orc.gemv_fp64_by_subblock(W, x, K, N), np.ones(N, np.float32))


@pytest.mark.parametrize("K,N,threads", [(256, 5, 1), (768, 37, 4), (5120, 64, 3), (2048, 1, 8)])
def test_host_int8_path_equals_kernel_semantics(orc, K, N, threads):
    """The host int8 timing path (byte-shuffle decode, 16-bit products, eight
    sub-blocks reduced together, OpenMP rows) gives exactly the kernel
    semantics on the quantised activations, for any thread count."""
    W = orc.gen_weights(K, N, seed=K + N)
    x = orc.gen_activations(K, seed=N, outliers=True)
    want = orc.gemv_semantics(W, orc.quantize_q8_1(x), K, N)
    got = orc.gemv_q8_1_host(W, x, K, N, threads)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
