"""ctypes binding of the CPU oracle (liboracle_iq4xs.so) and of the compiled
reference FP64 oracle (_ref/libref_cpu.so, built from the reference's
kernels/matmul_iq4xs/ref_cpu.cpp where the reference is mounted).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product package.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_iq4xs.so")
REF_LIB_PATH = os.path.join(HERE, "_ref", "libref_cpu.so")

QK_K = 256
QK8_1 = 32
BLOCK_BYTES = 136
Q8_1_BYTES = 36
LAYOUT_KM = 0
LAYOUT_MK = 1

# numpy views of the two block formats (byte-exact with the C structs)
BLOCK_IQ4_XS = np.dtype([("d", "<u2"), ("scales_h", "<u2"), ("scales_l", "u1", (4,)), ("qs", "u1", (128,))])
BLOCK_Q8_1 = np.dtype([("ds", "<u4"), ("qs", "i1", (32,))])
assert BLOCK_IQ4_XS.itemsize == BLOCK_BYTES and BLOCK_Q8_1.itemsize == Q8_1_BYTES

KVALUES_IQ4NL = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], dtype=np.int8)

_P = ctypes.c_void_p
_I64 = ctypes.c_int64


def build() -> None:
    """Compile liboracle_iq4xs.so (and the reference oracle where mounted)."""
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)
    if os.path.isdir("/root/reference/kernels"):
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


class Oracle:
    def __init__(self, path: str = LIB_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        lib = ctypes.CDLL(path)
        sig = {
            "orc_fp16_to_fp32": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_fp32_to_fp16_trunc": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_fp16_to_fp32_array": (None, [_P, _P, ctypes.c_size_t]),
            "orc_fp32_to_fp16_trunc_array": (None, [_P, _P, ctypes.c_size_t]),
            "orc_subblock_scale": (ctypes.c_int, [_P, ctypes.c_int]),
            "orc_quantize_q8_1": (None, [_P, _P, _I64]),
            "orc_quantize_q8_1_batched": (None, [_P, _P, _I64, _I64, ctypes.c_int]),
            "orc_dequant_q8_1": (None, [_P, _P, _I64]),
            "orc_subblock_sumi": (ctypes.c_int32, [_P, _P, ctypes.c_int]),
            "orc_subblock_sums": (None, [_P, _P, _P, _I64, _I64, _I64]),
            "orc_gemv_semantics": (None, [_P, _P, _P, _I64, _I64]),
            "orc_gemm_semantics": (None, [_P, _P, _P, _I64, _I64, _I64]),
            "orc_gemv_fp64": (None, [_P, _P, _P, _I64, _I64]),
            "orc_gemm_fp64": (None, [_P, _P, _P, _I64, _I64, _I64, ctypes.c_int]),
            "orc_dequant": (None, [_P, _P, _I64, _I64]),
            "orc_gemv_fp64_by_subblock": (None, [_P, _P, _P, _I64, _I64]),
            "orc_gemv_q8_1_host": (None, [_P, _P, _P, _I64, _I64, ctypes.c_int]),
            "orc_exp_cw": (ctypes.c_float, [ctypes.c_float]),
            "orc_silu": (ctypes.c_float, [ctypes.c_float]),
            "orc_swiglu_q8_1": (None, [_P, _P, _I64, _I64, _P, _P]),
            "orc_rms_norm_q8_1": (None, [_P, _P, _P, _P, ctypes.c_float, _I64, _I64, _P, _P]),
            "orc_gen_weights": (None, [_P, _I64, ctypes.c_uint64, _I64]),
            "orc_gen_activations": (None, [_P, _I64, ctypes.c_uint64, ctypes.c_int]),
        }
        for name, (res, args) in sig.items():
            f = getattr(lib, name)
            f.restype = res
            f.argtypes = args
        self.lib = lib

    # --- scalar codecs -------------------------------------------------
    def fp16_to_fp32(self, h: np.ndarray) -> np.ndarray:
        h = np.ascontiguousarray(h, dtype=np.uint16)
        out = np.empty(h.shape, np.float32)
        self.lib.orc_fp16_to_fp32_array(_ptr(h), _ptr(out), h.size)
        return out

    def fp32_to_fp16_trunc(self, f: np.ndarray) -> np.ndarray:
        f = np.ascontiguousarray(f, dtype=np.float32)
        out = np.empty(f.shape, np.uint16)
        self.lib.orc_fp32_to_fp16_trunc_array(_ptr(f), _ptr(out), f.size)
        return out

    # --- inputs --------------------------------------------------------
    def gen_weights(self, K: int, N: int, seed: int, first_block: int = 0) -> np.ndarray:
        """Seeded IQ4_XS matrix [N][K/256] as raw 136-byte blocks (uint8 array)."""
        nblk = N * (K // QK_K)
        W = np.empty(nblk * BLOCK_BYTES, np.uint8)
        self.lib.orc_gen_weights(_ptr(W), nblk, seed, first_block)
        return W

    def gen_activations(self, n: int, seed: int, outliers: bool = False) -> np.ndarray:
        x = np.empty(n, np.float32)
        self.lib.orc_gen_activations(_ptr(x), n, seed, int(outliers))
        return x

    # --- Q8_1 ----------------------------------------------------------
    def quantize_q8_1(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        K = x.size
        y = np.zeros((K // QK8_1) * Q8_1_BYTES, np.uint8)
        self.lib.orc_quantize_q8_1(_ptr(x), _ptr(y), K)
        return y

    def quantize_q8_1_batched(self, X: np.ndarray, K: int, M: int, layout: int) -> np.ndarray:
        X = np.ascontiguousarray(X, dtype=np.float32)
        assert X.size == K * M
        Y = np.zeros(M * (K // QK8_1) * Q8_1_BYTES, np.uint8)
        self.lib.orc_quantize_q8_1_batched(_ptr(X), _ptr(Y), K, M, layout)
        return Y

    def dequant_q8_1(self, AQ: np.ndarray) -> np.ndarray:
        nb = AQ.size // Q8_1_BYTES
        out = np.empty(nb * QK8_1, np.float32)
        self.lib.orc_dequant_q8_1(_ptr(np.ascontiguousarray(AQ)), _ptr(out), nb)
        return out

    # --- fused producers -> Q8_1 ---------------------------------------
    def exp_cw(self, x: np.ndarray) -> np.ndarray:
        f = self.lib.orc_exp_cw
        return np.array([f(float(v)) for v in np.asarray(x, np.float32).ravel()], np.float32)

    def silu(self, x: np.ndarray) -> np.ndarray:
        f = self.lib.orc_silu
        return np.array([f(float(v)) for v in np.asarray(x, np.float32).ravel()], np.float32)

    def swiglu_q8_1(self, G: np.ndarray, U: np.ndarray, K: int, M: int):
        """(y [M][K] float32, Q8_1 blocks of y as bytes)."""
        G = np.ascontiguousarray(G, dtype=np.float32)
        U = np.ascontiguousarray(U, dtype=np.float32)
        assert G.size == U.size == K * M
        Y = np.empty((M, K), np.float32)
        Q = np.zeros(M * (K // QK8_1) * Q8_1_BYTES, np.uint8)
        self.lib.orc_swiglu_q8_1(_ptr(G), _ptr(U), K, M, _ptr(Y), _ptr(Q))
        return Y, Q

    def rms_norm_q8_1(self, X: np.ndarray, K: int, M: int, R=None, gamma=None, eps: float = 1e-6):
        """(h = X + R [M][K], y [M][K], Q8_1 blocks of y as bytes)."""
        X = np.ascontiguousarray(X, dtype=np.float32)
        assert X.size == K * M
        H = np.empty((M, K), np.float32)
        Y = np.empty((M, K), np.float32)
        Q = np.zeros(M * (K // QK8_1) * Q8_1_BYTES, np.uint8)
        Rp = None if R is None else np.ascontiguousarray(R, dtype=np.float32)
        Gp = None if gamma is None else np.ascontiguousarray(gamma, dtype=np.float32)
        self.lib.orc_rms_norm_q8_1(_ptr(X), None if Rp is None else _ptr(Rp), _ptr(H),
                                   None if Gp is None else _ptr(Gp), eps, K, M, _ptr(Y), _ptr(Q))
        return H, Y, Q

    # --- integer sums and outputs -------------------------------------
    def subblock_sums(self, W: np.ndarray, AQ: np.ndarray, K: int, N: int, M: int) -> np.ndarray:
        S = np.empty((M, N, K // QK8_1), np.int32)
        self.lib.orc_subblock_sums(_ptr(W), _ptr(AQ), _ptr(S), K, N, M)
        return S

    def gemv_semantics(self, W: np.ndarray, AQ: np.ndarray, K: int, N: int) -> np.ndarray:
        y = np.empty(N, np.float32)
        self.lib.orc_gemv_semantics(_ptr(W), _ptr(AQ), _ptr(y), K, N)
        return y

    def gemm_semantics(self, W: np.ndarray, AQ: np.ndarray, K: int, N: int, M: int) -> np.ndarray:
        """Y[n, m] (row-major [N, M]) in the reference GEMM kernel's order."""
        Y = np.empty((N, M), np.float32)
        self.lib.orc_gemm_semantics(_ptr(W), _ptr(AQ), _ptr(Y), K, N, M)
        return Y

    def gemv_q8_1_host(self, W: np.ndarray, x: np.ndarray, K: int, N: int, nthreads: int = 1) -> np.ndarray:
        """Host int8 path (quantise + GEMV) on nthreads threads; equals
        gemv_semantics(W, quantize_q8_1(x)) bit for bit."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(N, np.float32)
        self.lib.orc_gemv_q8_1_host(_ptr(W), _ptr(x), _ptr(y), K, N, nthreads)
        return y

    def gemv_fp64(self, W: np.ndarray, x: np.ndarray, K: int, N: int) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(N, np.float32)
        self.lib.orc_gemv_fp64(_ptr(W), _ptr(x), _ptr(y), K, N)
        return y

    def gemm_fp64(self, W: np.ndarray, X_km: np.ndarray, K: int, N: int, M: int, nthreads: int = 1) -> np.ndarray:
        """X_km is [K, M] (X[k*M+m]); returns Y [N, M]."""
        X_km = np.ascontiguousarray(X_km, dtype=np.float32)
        Y = np.empty((N, M), np.float32)
        self.lib.orc_gemm_fp64(_ptr(W), _ptr(X_km), _ptr(Y), K, N, M, nthreads)
        return Y

    def gemv_fp64_by_subblock(self, W: np.ndarray, x: np.ndarray, K: int, N: int) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(N, np.float32)
        self.lib.orc_gemv_fp64_by_subblock(_ptr(W), _ptr(x), _ptr(y), K, N)
        return y

    def dequant(self, W: np.ndarray, K: int, N: int) -> np.ndarray:
        out = np.empty((N, K), np.float32)
        self.lib.orc_dequant(_ptr(W), _ptr(out), K, N)
        return out


class RefCpu:
    """The reference's own ref_cpu.cpp, compiled unchanged into _ref/libref_cpu.so."""

    def __init__(self, path: str = REF_LIB_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        lib = ctypes.CDLL(path)
        self.gemv = lib._Z18gemv_iq4xs_cpu_refPK12block_iq4_xsPKfPfll
        self.gemv.restype = None
        self.gemv.argtypes = [_P, _P, _P, _I64, _I64]
        self.gemm = lib._Z18gemm_iq4xs_cpu_refPK12block_iq4_xsPKfPflll
        self.gemm.restype = None
        self.gemm.argtypes = [_P, _P, _P, _I64, _I64, _I64]
        self.deq = lib._Z21dequant_mat_iq4xs_cpuPK12block_iq4_xsPfll
        self.deq.restype = None
        self.deq.argtypes = [_P, _P, _I64, _I64]

    def gemv_fp64(self, W, x, K, N):
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(N, np.float32)
        self.gemv(_ptr(W), _ptr(x), _ptr(y), K, N)
        return y

    def gemm_fp64(self, W, X_km, K, N, M):
        X_km = np.ascontiguousarray(X_km, dtype=np.float32)
        Y = np.empty((N, M), np.float32)
        self.gemm(_ptr(W), _ptr(X_km), _ptr(Y), K, N, M)
        return Y

    def dequant(self, W, K, N):
        out = np.empty((N, K), np.float32)
        self.deq(_ptr(W), _ptr(out), K, N)
        return out


def ref_available() -> bool:
    return os.path.exists(REF_LIB_PATH)


# --- metrics (kernels/common/matmul_test_util.h:22-47) -----------------
def compute_metrics(ref: np.ndarray, got: np.ndarray) -> dict:
    r = np.asarray(ref, dtype=np.float64).ravel()
    g = np.asarray(got, dtype=np.float64).ravel()
    bad = bool(np.any(~np.isfinite(r)) or np.any(~np.isfinite(g)))
    d = np.abs(r - g)
    mask = np.abs(r) > 1e-3
    max_rel = float(np.max(d[mask] / np.abs(r[mask]))) if mask.any() else 0.0
    nr, ng = float(np.sqrt(np.dot(r, r))), float(np.sqrt(np.dot(g, g)))
    denom = nr * ng
    if denom > 1e-12:
        cos = float(np.dot(r, g) / denom)
    else:
        cos = 1.0 if (nr * nr < 1e-12 and ng * ng < 1e-12) else 0.0
    rel_l2 = float(np.sqrt(np.dot(r - g, r - g)) / nr) if nr > 0 else float(np.sqrt(np.dot(g, g)))
    return {
        "max_abs": float(d.max()) if d.size else 0.0,
        "mean_abs": float(d.mean()) if d.size else 0.0,
        "max_rel": max_rel,
        "cosine": cos,
        "rel_l2": rel_l2,
        "bad": bad,
        "pass": (not bad) and cos >= 0.999,
    }
