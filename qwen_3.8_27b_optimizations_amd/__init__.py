"""Python side of the MI355X IQ4_XS mul_mat library.

Loads libiq4xs_mi355x.so (built in this directory by `make`) through ctypes
and exposes the C ABI of include/iq4xs_mi355x.h.  Two layers:

* `Lib` -- one method per extern "C" entry point, raw device pointers (ints)
  and a stream handle; this is the boundary the parity tests call.
* torch helpers (`mul_mat`, `quantize_q8_1`, ...) that take torch tensors on a
  ROCm device, allocate outputs/workspace and pass the current stream.

There is no fallback: if the shared library or a GPU is missing, the calls
raise.  The directory name contains a dot, so load it with
`load_package()` from __graft_entry__ or importlib, not a plain import.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_NAME = "libiq4xs_mi355x.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)

SUCCESS = 0
ERROR_INVALID_VALUE = 1
ERROR_INVALID_CONFIG = 9
ERROR_NOT_SUPPORTED = 801

QK_K = 256
QK8_1 = 32
BLOCK_BYTES = 136
Q8_1_BLOCK_BYTES = 36
GGML_TYPE_IQ4_XS = 23
LAYOUT_KM = 0
LAYOUT_MK = 1
PATH_AUTO = -1
PATH_GEMV = 0
PATH_GEMM = 1
GEMV_MAX_COLS = 8

# (restype, argtypes) of every exported symbol, in header order
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int
SIGNATURES = {
    "quantize_row_q8_1_gpu": (_INT, [_P, _P, _I64, _P]),
    "quantize_row_q8_1_batched_gpu": (_INT, [_P, _P, _I64, _I64, _P]),
    "gemv_iq4xs_stock_dp4a_gpu": (_INT, [_P, _P, _P, _I64, _I64, _P]),
    "gemv_iq4xs_dp4a_coop_gpu": (_INT, [_P, _P, _P, _I64, _I64, _P]),
    "gemm_iq4xs_stock_dp4a_gpu": (_INT, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "dequant_iq4xs_gpu": (_INT, [_P, _P, _I64, _INT, _P]),
    "gemv_iq4xs_dp4a_gfx1100_gpu": (_INT, [_P, _P, _P, _I64, _I64, _P]),
    "gemv_iq4xs_dp4a_gfx1100_prequantized_gpu": (_INT, [_P, _P, _P, _I64, _I64, _P]),
    "gemv_iq4xs_stock_gpu": (_INT, [_P, _P, _P, _I64, _I64, _P]),
    "gemm_iq4xs_stock_gpu": (_INT, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "gemv_iq4xs_gfx1100_gpu": (_INT, [_P, _P, _P, _I64, _I64, _P]),
    "gemm_iq4xs_wmma_stream_gpu": (_INT, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "gemm_iq4xs_wmma_p4_xor_gpu": (_INT, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "gemm_iq4xs_wmma_64x64_gpu": (_INT, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "gemm_iq4xs_stream_tiled_gpu": (_INT, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "gemm_iq4xs_wmma_gpu": (_INT, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "gemm_iq4xs_tiled_gpu": (_INT, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "gemm_iq4xs_lut_gpu": (_INT, [_P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "custom_gemv_iq4xs_can_handle": (ctypes.c_bool, [_I64, _I64, _I64, _INT]),
    "custom_gemv_iq4xs_dispatch": (_INT, [_P, _P, _P, _I64, _I64, _P]),
    "custom_gemm_iq4xs_can_handle": (ctypes.c_bool, [_I64, _I64, _I64, _INT]),
    "custom_gemm_iq4xs_dispatch": (_INT, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "iq4xs_workspace_bytes": (ctypes.c_size_t, [_I64, _I64]),
    "iq4xs_quantize_q8_1": (_INT, [_P, _I64, _I64, _INT, _P, ctypes.c_size_t, _P]),
    "iq4xs_mul_mat_q8_1": (_INT, [_P, _P, _P, _I64, _I64, _I64, _INT, _INT, _P]),
    "iq4xs_mul_mat": (_INT, [_P, _P, _P, _I64, _I64, _I64, _INT, _P, ctypes.c_size_t, _P]),
    "iq4xs_mul_mat_noalloc": (_INT, [_P, _P, _P, _I64, _I64, _I64, _INT, _P]),
    "iq4xs_mul_mat_fused": (_INT, [_P, _P, _P, _I64, _I64, _I64, _INT, _P, _P]),
    "iq4xs_mul_mat_q8_1_group": (_INT, [_INT, _P, _P, _P, _P, _I64, _I64, _INT, _P]),
    "iq4xs_rms_norm_q8_1": (_INT, [_P, _P, _P, _P, ctypes.c_float, _I64, _I64, _P, ctypes.c_size_t, _P]),
    "iq4xs_swiglu_q8_1": (_INT, [_P, _P, _I64, _I64, _P, ctypes.c_size_t, _P]),
    "iq4xs_rms_norm_mul_mat_group": (_INT, [_INT, _P, _P, _P, _P, _P, _P, _P, ctypes.c_float, _I64, _P]),
    "iq4xs_rms_norm_mul_mat_swiglu": (_INT, [_P, _P, _I64, _P, _P, _P, _P, ctypes.c_float, _I64, _P, _P, _P, _P]),
    "iq4xs_q8_1_to_blocks": (_INT, [_P, _P, _I64, _I64, _P]),
    "iq4xs_subblock_sums": (_INT, [_P, _P, _P, _P, _I64, _I64, _I64, _INT, _P]),
    "iq4xs_probe_mfma_i8": (_INT, [_P, _P, _P, _P]),
    "iq4xs_fill_synthetic_weights": (_INT, [_P, _I64, ctypes.c_uint64, _I64, _P]),
    "iq4xs_fill_synthetic_activations": (_INT, [_P, _I64, ctypes.c_uint64, _INT, _P]),
    "iq4xs_version": (ctypes.c_char_p, []),
}


class Iq4xsError(RuntimeError):
    def __init__(self, fn: str, code: int):
        super().__init__(f"{fn} returned hipError {code}")
        self.code = code


class Lib:
    """The C ABI, one attribute per entry point."""

    def __init__(self, path: str = LIB_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(
                f"{path} is missing: build it with `make -C {HERE}` (or __graft_entry__.build())")
        self.path = path
        self.cdll = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(self.cdll, name)
            fn.restype = res
            fn.argtypes = args
            setattr(self, name, fn)

    def check(self, name: str, *args) -> None:
        code = getattr(self, name)(*args)
        if code != SUCCESS:
            raise Iq4xsError(name, code)


_LIB: Lib | None = None


def lib() -> Lib:
    global _LIB
    if _LIB is None:
        _LIB = Lib()
    return _LIB


# ---------------------------------------------------------------------------
# torch helpers (device memory and streams only)

def _torch():
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("no ROCm GPU visible: the IQ4_XS kernels have no CPU path")
    return torch


def _stream(torch) -> int:
    return torch.cuda.current_stream().cuda_stream


def _check_weights(W, K: int, N: int) -> None:
    if W.dtype.itemsize != 1 or W.numel() != N * (K // QK_K) * BLOCK_BYTES or not W.is_contiguous():
        raise ValueError("W must be a contiguous byte tensor of N*(K/256)*136 bytes")


def workspace(K: int, M: int, device=None):
    torch = _torch()
    nbytes = lib().iq4xs_workspace_bytes(K, M)
    if nbytes == 0:
        raise ValueError("bad workspace shape")
    return torch.empty(nbytes, dtype=torch.uint8, device=device or "cuda")


def quantize_q8_1(X, K: int, M: int, layout: int = LAYOUT_MK, ws=None):
    """fp32 activations -> planar Q8_1 workspace (uint8 tensor)."""
    torch = _torch()
    ws = workspace(K, M, X.device) if ws is None else ws
    lib().check("iq4xs_quantize_q8_1", X.data_ptr(), K, M, layout, ws.data_ptr(), ws.numel(), _stream(torch))
    return ws


def rms_norm_q8_1(X, K: int, M: int, residual=None, out_h=None, gamma=None, eps: float = 1e-6, ws=None):
    """h = X (+ residual) -> planar Q8_1 of (h / rms(h)) * gamma.

    out_h receives h when given (it may be X or residual itself: the in-place
    residual add).  Returns the workspace."""
    torch = _torch()
    ws = workspace(K, M, X.device) if ws is None else ws
    ptr = lambda t: None if t is None else t.data_ptr()
    lib().check("iq4xs_rms_norm_q8_1", X.data_ptr(), ptr(residual), ptr(out_h), ptr(gamma), eps, K, M,
                ws.data_ptr(), ws.numel(), _stream(torch))
    return ws


def swiglu_q8_1(G, U, K: int, M: int, ws=None):
    """planar Q8_1 of silu(G) * U; returns the workspace."""
    torch = _torch()
    ws = workspace(K, M, G.device) if ws is None else ws
    lib().check("iq4xs_swiglu_q8_1", G.data_ptr(), U.data_ptr(), K, M, ws.data_ptr(), ws.numel(), _stream(torch))
    return ws


def rms_norm_mul_mat_group(Ws, X, K: int, Ns, residual=None, out_h=None, gamma=None, eps: float = 1e-6, outs=None):
    """RMS norm of one column (h = X + residual, written to out_h) fused into one grouped bs=1 GEMV:
    [W_i * Q8_1((h * scale) * gamma)], bit-identical to rms_norm_q8_1 followed by mul_mat_q8_1_group."""
    torch = _torch()
    n = len(Ws)
    if outs is None:
        outs = [torch.empty(N, dtype=torch.float32, device=X.device) for N in Ns]
    for W, N in zip(Ws, Ns):
        _check_weights(W, K, N)
    wp = (ctypes.c_void_p * n)(*[W.data_ptr() for W in Ws])
    yp = (ctypes.c_void_p * n)(*[y.data_ptr() for y in outs])
    nn = (ctypes.c_int64 * n)(*Ns)
    ptr = lambda t: t.data_ptr() if t is not None else None
    lib().check("iq4xs_rms_norm_mul_mat_group", n, wp, yp, nn, X.data_ptr(), ptr(residual), ptr(out_h), ptr(gamma),
                eps, K, _stream(torch))
    return outs


def rms_norm_mul_mat_swiglu(W_gate, W_up, X, K: int, N: int, residual=None, out_h=None, gamma=None,
                            eps: float = 1e-6, gate_out=None, up_out=None, keep_gate_up: bool = True, out=None):
    """RMS norm + gate/up GEMVs + SwiGLU in one bs=1 launch: returns (S, gate, up) with S = silu(gate) * up
    (fp32, the SwiGLU producer's arithmetic); gate/up bit-identical to rms_norm_mul_mat_group on the pair.
    With keep_gate_up=False gate and up are not written (None is returned for them)."""
    torch = _torch()
    _check_weights(W_gate, K, N)
    _check_weights(W_up, K, N)
    new = lambda: torch.empty(N, dtype=torch.float32, device=X.device)
    S = new() if out is None else out
    g = (new() if gate_out is None else gate_out) if keep_gate_up else None
    u = (new() if up_out is None else up_out) if keep_gate_up else None
    ptr = lambda t: t.data_ptr() if t is not None else None
    lib().check("iq4xs_rms_norm_mul_mat_swiglu", W_gate.data_ptr(), W_up.data_ptr(), N, X.data_ptr(), ptr(residual),
                ptr(out_h), ptr(gamma), eps, K, ptr(g), ptr(u), S.data_ptr(), _stream(torch))
    return S, g, u


def q8_1_blocks(ws, K: int, M: int):
    """Planar workspace -> [M*K/32, 36] uint8 tensor of ggml Q8_1 blocks."""
    torch = _torch()
    out = torch.empty((M * (K // QK8_1), Q8_1_BLOCK_BYTES), dtype=torch.uint8, device=ws.device)
    lib().check("iq4xs_q8_1_to_blocks", ws.data_ptr(), out.data_ptr(), K, M, _stream(torch))
    return out


def mul_mat_q8_1(W, ws, K: int, N: int, M: int, layout: int = LAYOUT_MK, path: int = PATH_AUTO, out=None):
    torch = _torch()
    _check_weights(W, K, N)
    if out is None:
        shape = (M, N) if layout == LAYOUT_MK else (N, M)
        out = torch.empty(shape, dtype=torch.float32, device=W.device)
    lib().check("iq4xs_mul_mat_q8_1", W.data_ptr(), ws.data_ptr(), out.data_ptr(), K, N, M, layout, path,
                _stream(torch))
    return out


def mul_mat_q8_1_group(Ws, ws, K: int, Ns, M: int, layout: int = LAYOUT_MK, outs=None):
    """[W_i * dequant(ws)] for up to 4 matrices sharing the activations, in one launch (the GEMV for
    M <= 8, the GEMM above); each output bit-identical to mul_mat_q8_1 on its own matrix."""
    torch = _torch()
    n = len(Ws)
    if not 1 <= n <= 4 or len(Ns) != n:
        raise ValueError("1 to 4 matrices, one N each")
    for W, N in zip(Ws, Ns):
        _check_weights(W, K, N)
    if outs is None:
        outs = [torch.empty((M, N) if layout == LAYOUT_MK else (N, M), dtype=torch.float32, device=Ws[0].device)
                for N in Ns]
    arr_p = ctypes.c_void_p * n
    wp = arr_p(*[W.data_ptr() for W in Ws])
    yp = arr_p(*[Y.data_ptr() for Y in outs])
    nn = (ctypes.c_int64 * n)(*Ns)
    lib().check("iq4xs_mul_mat_q8_1_group", n, wp, yp, nn, ws.data_ptr(), K, M, layout, _stream(torch))
    return outs


def mul_mat(W, X, K: int, N: int, M: int, layout: int = LAYOUT_MK, ws=None, out=None):
    """Y = W * X with X quantised to Q8_1 on the fly (explicit workspace, no allocation in the library)."""
    torch = _torch()
    _check_weights(W, K, N)
    ws = workspace(K, M, W.device) if ws is None else ws
    if out is None:
        shape = (M, N) if layout == LAYOUT_MK else (N, M)
        out = torch.empty(shape, dtype=torch.float32, device=W.device)
    lib().check("iq4xs_mul_mat", W.data_ptr(), X.data_ptr(), out.data_ptr(), K, N, M, layout, ws.data_ptr(),
                ws.numel(), _stream(torch))
    return out


def mul_mat_fused(W, X, K: int, N: int, M: int, layout: int = LAYOUT_MK, out=None, sums: bool = False):
    """Y = W * X for M <= 8 with the Q8_1 quantisation inside the GEMV kernel.

    Raises Iq4xsError with code ERROR_NOT_SUPPORTED when M*K is too large for
    the fused kernel.  With sums=True also returns S[M, N, K/32] (int32)."""
    torch = _torch()
    _check_weights(W, K, N)
    if out is None:
        shape = (M, N) if layout == LAYOUT_MK else (N, M)
        out = torch.empty(shape, dtype=torch.float32, device=W.device)
    S = torch.empty((M, N, K // QK8_1), dtype=torch.int32, device=W.device) if sums else None
    lib().check("iq4xs_mul_mat_fused", W.data_ptr(), X.data_ptr(), out.data_ptr(), K, N, M, layout,
                S.data_ptr() if sums else None, _stream(torch))
    return (out, S) if sums else out


def subblock_sums(W, ws, K: int, N: int, M: int, path: int):
    """(S[M, N, K/32] int32, Y[M, N] fp32) from the production kernel `path`."""
    torch = _torch()
    S = torch.empty((M, N, K // QK8_1), dtype=torch.int32, device=W.device)
    Y = torch.empty((M, N), dtype=torch.float32, device=W.device)
    lib().check("iq4xs_subblock_sums", W.data_ptr(), ws.data_ptr(), S.data_ptr(), Y.data_ptr(), K, N, M, path,
                _stream(torch))
    return S, Y


def dequant(W, n_blocks: int, out=None):
    """IQ4_XS super-blocks -> fp32 weights [n_blocks * 256]."""
    torch = _torch()
    if W.dtype.itemsize != 1 or W.numel() < n_blocks * BLOCK_BYTES:
        raise ValueError("W must hold n_blocks * 136 bytes")
    out = torch.empty(n_blocks * QK_K, dtype=torch.float32, device=W.device) if out is None else out
    lib().check("dequant_iq4xs_gpu", W.data_ptr(), out.data_ptr(), n_blocks, 64, _stream(torch))
    return out


def synthetic_weights(K: int, N: int, seed: int, first_block: int = 0, device=None):
    torch = _torch()
    nblk = N * (K // QK_K)
    W = torch.empty(nblk * BLOCK_BYTES, dtype=torch.uint8, device=device or "cuda")
    lib().check("iq4xs_fill_synthetic_weights", W.data_ptr(), nblk, seed, first_block, _stream(torch))
    return W


def synthetic_activations(n: int, seed: int, outliers: bool = False, device=None):
    torch = _torch()
    x = torch.empty(n, dtype=torch.float32, device=device or "cuda")
    lib().check("iq4xs_fill_synthetic_activations", x.data_ptr(), n, seed, int(outliers), _stream(torch))
    return x
