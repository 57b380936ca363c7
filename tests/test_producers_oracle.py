"""Pins the oracle's fused producers (orc_exp_cw, orc_silu, orc_rms_norm_q8_1,
orc_swiglu_q8_1) before they are trusted as the checker of the device
kernels.  These ops have no counterpart in the reference's kernels, so they
are pinned by mathematics: error bounds against float64 evaluations, closed
forms, and the already-pinned quantiser applied to the values they return.
The plausible mistakes -- a dropped or wrong Taylor term, a wrong ln2 split,
the sign of silu's exponent, eps dropped or added after the square root, a
divisor of K-1, the residual or gain left out -- each fail one of them."""
import math

import numpy as np
import pytest

from oracle.oracle import BLOCK_Q8_1


def ulps(got, ref64):
    """|got - ref| in units of the float32 spacing at ref."""
    ref32 = np.abs(ref64).astype(np.float32)
    return np.abs(got.astype(np.float64) - ref64) / np.spacing(ref32).astype(np.float64)


def test_exp_error_bound_dense_sweep(orc):
    x = np.linspace(-87.0, 88.7, 400001).astype(np.float32)
    e = orc.exp_cw(x)
    err = ulps(e, np.exp(x.astype(np.float64)))
    assert err.max() <= 1.0, err.max()
    assert err.mean() <= 0.35


def test_exp_special_values(orc):
    assert orc.exp_cw(np.float32([0.0]))[0] == 1.0
    assert orc.exp_cw(np.float32([1.0]))[0] == np.float32(math.e)
    assert orc.exp_cw(np.float32([-1.0]))[0] == np.float32(1.0 / math.e)
    big = orc.exp_cw(np.float32([88.72284, 89.0, 1e30, np.inf]))
    assert np.all(np.isposinf(big))
    # inputs below -87 are raised to -87: the result stays normal
    low = orc.exp_cw(np.float32([-87.0, -88.0, -1e30, -np.inf]))
    assert np.all(low == low[0]) and low[0] >= np.finfo(np.float32).tiny
    assert np.isnan(orc.exp_cw(np.float32([np.nan]))[0])
    # near multiples of ln2 the reduction must pick n = k and land on ~2^k
    for k in (-120, -100, -10, 1, 10, 100, 127):
        x = np.float32(k * math.log(2.0))
        assert ulps(orc.exp_cw(np.float32([x])), np.exp(np.float64(x)))[0] <= 1.0, k


def test_silu_error_bound(orc):
    x = np.concatenate([np.linspace(-60, 100, 200001), np.float32([-1e-30, 1e-30, 1e-3, -1e-3])]).astype(np.float32)
    s = orc.silu(x)
    x64 = x.astype(np.float64)
    ref = x64 / (1.0 + np.exp(-x64))
    err = ulps(s, ref)
    assert err.max() <= 4.0, err.max()
    assert orc.silu(np.float32([0.0]))[0] == 0.0
    assert orc.silu(np.float32([100.0]))[0] == 100.0
    big_neg = orc.silu(np.float32([-100.0]))[0]
    assert big_neg == 0.0 and np.signbit(big_neg)


def test_swiglu_values_and_blocks(orc):
    rng = np.random.default_rng(5)
    K, M = 1024, 3
    G = (rng.standard_normal(K * M) * 4).astype(np.float32)
    G[:8] = [0.0, -90.0, 90.0, -20.0, 20.0, 1e-6, -1e-6, 3.5]
    U = rng.standard_normal(K * M).astype(np.float32)
    Y, Q = orc.swiglu_q8_1(G, U, K, M)
    g64 = G.astype(np.float64)
    ref = g64 / (1.0 + np.exp(-g64)) * U.astype(np.float64)
    keep = np.abs(ref) > 1e-30
    assert ulps(Y.ravel()[keep], ref[keep]).max() <= 5.0
    assert np.array_equal(Q, orc.quantize_q8_1(Y.ravel()))


def rms_reference64(X, R, gamma, eps, K, M):
    h = X.reshape(M, K) if R is None else (X.reshape(M, K) + R.reshape(M, K)).astype(np.float32)
    h64 = h.astype(np.float64)
    ms = np.array([math.fsum(v) for v in h64 * h64]) / K
    y = h64 / np.sqrt(ms + np.float64(np.float32(eps)))[:, None]
    if gamma is not None:
        y = y * gamma.astype(np.float64)[None, :]
    return h, y


@pytest.mark.parametrize("K,M,res,gain,scale", [(1024, 2, False, False, 1.0), (5120, 3, True, True, 1.0),
                                                (5120 + 96, 2, True, False, 1.0), (288, 4, False, True, 1e-3),
                                                (5120, 2, True, True, 1e-3)])
def test_rms_norm_vs_float64(orc, K, M, res, gain, scale):
    """Small-magnitude rows (scale 1e-3: mean square ~ eps) make eps matter."""
    rng = np.random.default_rng(K + M)
    X = (rng.standard_normal(K * M) * scale).astype(np.float32)
    R = (rng.standard_normal(K * M) * scale).astype(np.float32) if res else None
    g = (rng.random(K) * 2).astype(np.float32) if gain else None
    H, Y, Q = orc.rms_norm_q8_1(X, K, M, R=R, gamma=g, eps=1e-6)
    h_ref, y_ref = rms_reference64(X, R, g, 1e-6, K, M)
    assert np.array_equal(H, h_ref)
    rel = np.abs(Y.astype(np.float64) - y_ref) / np.maximum(np.abs(y_ref), 1e-30)
    assert rel.max() <= 2.0 ** -21, rel.max()
    assert np.array_equal(Q, orc.quantize_q8_1(Y.ravel()))


def test_rms_norm_eps_and_divisor_are_visible(orc):
    """At mean square ~ eps the tolerance above separates the right formula
    from eps dropped (x2 in the mean) and from K-1 as divisor."""
    K = 1024
    x = np.full(K, 1e-3, np.float32)
    _, Y, _ = orc.rms_norm_q8_1(x, K, 1, eps=1e-6)
    right = 1e-3 / math.sqrt(float(np.float32(1e-3)) ** 2 + float(np.float32(1e-6)))
    assert Y[0, 0] == pytest.approx(right, rel=2 ** -21)
    assert abs(Y[0, 0] - 1.0) > 0.2                                     # eps dropped would give 1
    wrong_div = 1e-3 / math.sqrt(float(np.float32(1e-3)) ** 2 * K / (K - 1) + 1e-6)
    assert abs(Y[0, 0] - wrong_div) / right > 2 ** -21


def test_rms_norm_closed_forms(orc):
    K = 2048
    # constant row 0.5, eps 0: mean 0.25 exactly, scale 2, y == 1; Q8_1 codes all 127
    _, Y, Q = orc.rms_norm_q8_1(np.full(K, 0.5, np.float32), K, 1, eps=0.0)
    assert np.all(Y == 1.0)
    b = Q.view(BLOCK_Q8_1)
    assert np.all(b["qs"] == 127)
    # one nonzero element a: y = sign(a) * sqrt(K) (to rounding), all else 0
    x = np.zeros(K, np.float32)
    x[77] = -3.0
    _, Y, _ = orc.rms_norm_q8_1(x, K, 1, eps=0.0)
    assert Y[0, 77] == pytest.approx(-math.sqrt(K), rel=2 ** -22)
    assert np.count_nonzero(Y) == 1
    # gain multiplies after the normalisation, element by element
    g = np.arange(K, dtype=np.float32)
    _, Yg, _ = orc.rms_norm_q8_1(np.full(K, 0.5, np.float32), K, 1, gamma=g, eps=0.0)
    assert np.array_equal(Yg[0], g)
    # residual: X + R is what gets normalised, and what H returns
    H, Y1, _ = orc.rms_norm_q8_1(np.full(K, 0.25, np.float32), K, 1, R=np.full(K, 0.25, np.float32), eps=0.0)
    assert np.all(H == 0.5) and np.all(Y1 == 1.0)
