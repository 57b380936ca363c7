"""C ABI checks that need no GPU: the library loads, exports exactly what
include/iq4xs_mi355x.h declares, and its host-side logic (shape gates,
workspace sizing, argument validation) behaves like the reference launchers.
Calls here either touch no device or are rejected before any launch."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "iq4xs_mi355x.h")


@pytest.fixture(scope="module")
def L(pkg):
    if not os.path.exists(pkg.LIB_PATH):
        subprocess.run(["make", "-s", "-j8", "-C", os.path.dirname(pkg.LIB_PATH)], check=True)
    return pkg.lib()


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w]*\s*\**\s+(\w+)\s*\(", text, flags=re.M)


def test_header_declares_the_boundary():
    names = header_functions()
    for must in ["quantize_row_q8_1_gpu", "quantize_row_q8_1_batched_gpu", "gemv_iq4xs_stock_dp4a_gpu",
                 "gemm_iq4xs_stock_dp4a_gpu", "gemv_iq4xs_dp4a_coop_gpu", "custom_gemv_iq4xs_can_handle",
                 "custom_gemv_iq4xs_dispatch", "custom_gemm_iq4xs_can_handle", "custom_gemm_iq4xs_dispatch"]:
        assert must in names


def test_library_exports_every_declared_symbol(L, pkg):
    names = header_functions()
    assert len(names) >= 19
    out = subprocess.run(["nm", "-D", "--defined-only", L.path], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    # the Python mirror binds exactly the declared set
    assert set(pkg.SIGNATURES) == set(names)
    for n in names:
        assert getattr(L.cdll, n) is not None


def test_version(L):
    assert b"gfx950" in L.iq4xs_version()


def test_can_handle_gates(L, pkg):
    T = pkg.GGML_TYPE_IQ4_XS
    g, m = L.custom_gemv_iq4xs_can_handle, L.custom_gemm_iq4xs_can_handle
    # the config shapes the reference's whitelist (patch:274-277) refused are served
    for K, N in [(5120, 8192), (5120, 1024), (8192, 5120), (5120, 17408), (17408, 5120), (4096, 4096)]:
        assert g(K, N, 1, T) and m(K, N, 512, T)
    # the GEMV dispatch has no M argument: one column only, as the reference's gate (patch:274-277)
    assert g(5120, 8192, 1, T) and not g(5120, 8192, 2, T) and not g(5120, 8192, 8, T)
    assert not g(5120, 8192, 9, T) and m(5120, 8192, 2, T) and m(5120, 8192, 8, T)
    assert not g(5120, 8192, 1, T + 1) and not m(5120, 8192, 512, 0)
    assert not g(5000, 8192, 1, T) and not m(5000, 64, 16, T)   # K % 256 != 0
    assert not g(0, 8, 1, T) and not g(256, 0, 1, T) and not m(256, 8, 0, T)
    assert m(256, 1, 1, T)


def test_workspace_bytes(L):
    """codes int8 [M][K], then ds uint32 [M][K/32], then the fp16 code pairs [M][K]
    (2 bytes per code), each part at a 256-byte boundary."""
    K, M = 5120, 512
    qs = K * M
    ds_off = (qs + 255) // 256 * 256
    hq_off = (ds_off + M * (K // 32) * 4 + 255) // 256 * 256
    assert L.iq4xs_workspace_bytes(K, M) == hq_off + 2 * K * M
    assert L.iq4xs_workspace_bytes(256, 1) == 256 + 256 + 512
    assert L.iq4xs_workspace_bytes(0, 1) == 0 and L.iq4xs_workspace_bytes(100, 1) == 0
    # past the kernels' index range, as every entry point refuses (no wrapped size)
    assert L.iq4xs_workspace_bytes(1 << 31, 1) == 0 and L.iq4xs_workspace_bytes(256, 1 << 31) == 0
    assert L.iq4xs_workspace_bytes((1 << 31) - 32, 1) > 0


FAKE = ctypes.c_void_p(0x100000)  # never dereferenced: every call below fails validation


def test_invalid_arguments_rejected_before_launch(L, pkg):
    E = pkg.ERROR_INVALID_VALUE
    assert L.gemv_iq4xs_stock_dp4a_gpu(None, FAKE, FAKE, 256, 4, None) == E
    assert L.gemv_iq4xs_stock_dp4a_gpu(FAKE, FAKE, FAKE, 300, 4, None) == E
    assert L.gemv_iq4xs_stock_dp4a_gpu(FAKE, FAKE, FAKE, 256, 0, None) == E
    assert L.gemv_iq4xs_dp4a_coop_gpu(FAKE, None, FAKE, 256, 4, None) == E
    assert L.gemm_iq4xs_stock_dp4a_gpu(FAKE, FAKE, FAKE, 256, 4, 0, None) == E
    assert L.gemm_iq4xs_stock_dp4a_gpu(FAKE, FAKE, None, 256, 4, 4, None) == E
    assert L.custom_gemv_iq4xs_dispatch(FAKE, FAKE, FAKE, -256, 4, None) == E
    assert L.custom_gemm_iq4xs_dispatch(FAKE, FAKE, FAKE, 256, 4, -1, None) == E
    assert L.quantize_row_q8_1_gpu(FAKE, FAKE, 33, None) == E
    assert L.quantize_row_q8_1_batched_gpu(FAKE, FAKE, 64, 0, None) == E
    ws_small = L.iq4xs_workspace_bytes(256, 2) - 1
    assert L.iq4xs_quantize_q8_1(FAKE, 256, 2, pkg.LAYOUT_MK, FAKE, ws_small, None) == E
    assert L.iq4xs_quantize_q8_1(FAKE, 256, 2, 7, FAKE, 1 << 20, None) == E
    assert L.iq4xs_quantize_q8_1(FAKE, 256, 2, pkg.LAYOUT_MK, ctypes.c_void_p(0x100010), 1 << 20, None) == E
    assert L.iq4xs_mul_mat_q8_1(FAKE, FAKE, FAKE, 256, 4, 2, 5, pkg.PATH_AUTO, None) == E
    assert L.iq4xs_mul_mat(FAKE, FAKE, FAKE, 256, 4, 2, pkg.LAYOUT_MK, None, 1 << 20, None) == E
    assert L.iq4xs_subblock_sums(FAKE, FAKE, None, FAKE, 256, 4, 2, pkg.PATH_GEMV, None) == E
    assert L.iq4xs_subblock_sums(FAKE, FAKE, FAKE, FAKE, 256, 4, 2, 3, None) == E
    assert L.iq4xs_probe_mfma_i8(None, FAKE, FAKE, None) == E
    assert L.iq4xs_fill_synthetic_weights(FAKE, 0, 1, 0, None) == E
    assert L.iq4xs_fill_synthetic_activations(None, 10, 1, 0, None) == E
    assert L.gemv_iq4xs_dp4a_gfx1100_gpu(FAKE, FAKE, None, 256, 4, None) == E
    assert L.gemv_iq4xs_dp4a_gfx1100_prequantized_gpu(FAKE, None, FAKE, 256, 4, None) == E
    assert L.gemv_iq4xs_dp4a_gfx1100_prequantized_gpu(FAKE, ctypes.c_void_p(0x100008), FAKE, 256, 4, None) == E
    assert L.gemv_iq4xs_stock_gpu(FAKE, FAKE, FAKE, 100, 4, None) == E
    assert L.gemv_iq4xs_gfx1100_gpu(FAKE, FAKE, FAKE, 256, 0, None) == E
    assert L.gemm_iq4xs_stock_gpu(FAKE, FAKE, FAKE, 256, 4, 0, None) == E
    for name in ("gemm_iq4xs_wmma_stream_gpu", "gemm_iq4xs_wmma_p4_xor_gpu", "gemm_iq4xs_wmma_64x64_gpu",
                 "gemm_iq4xs_stream_tiled_gpu", "gemm_iq4xs_wmma_gpu", "gemm_iq4xs_tiled_gpu"):
        assert getattr(L, name)(FAKE, FAKE, FAKE, 300, 4, 4, None) == E, name
    assert L.gemm_iq4xs_lut_gpu(FAKE, FAKE, None, FAKE, 256, 64, 512, None) == E
    # the reference's LUT shape gate: refused before any launch
    assert L.gemm_iq4xs_lut_gpu(FAKE, FAKE, FAKE, FAKE, 256, 64, 256, None) == pkg.ERROR_INVALID_CONFIG


def test_product_package_has_no_oracle_dependency():
    """The product must never route through the checker."""
    pkg_dir = os.path.join(ROOT, "qwen_3.8_27b_optimizations_amd")
    for dirpath, _, files in os.walk(pkg_dir):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp", "Makefile")):
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in text.replace("oracle is", ""), os.path.join(dirpath, f)
    out = subprocess.run(["ldd", os.path.join(pkg_dir, "libiq4xs_mi355x.so")], capture_output=True, text=True)
    assert "oracle" not in out.stdout


REFERENCE_CPP_API = {  # the reference's own C++ signatures (include/iq4xs_reference_api.hpp cites each)
    "quantize_row_q8_1_gpu(float const*, block_q8_1_real*, long, ihipStream_t*)",
    "quantize_row_q8_1_batched_gpu(float const*, block_q8_1_real*, long, long, ihipStream_t*)",
    "gemv_iq4xs_stock_dp4a_gpu(block_iq4_xs const*, float const*, float*, long, long, ihipStream_t*)",
    "gemm_iq4xs_stock_dp4a_gpu(block_iq4_xs const*, float const*, float*, long, long, long, ihipStream_t*)",
    "gemv_iq4xs_dp4a_gfx1100_prequantized_gpu(block_iq4_xs const*, block_q8_1_coop const*, float*, long, long, "
    "ihipStream_t*)",
    "gemv_iq4xs_dp4a_gfx1100_gpu(block_iq4_xs const*, float const*, float*, long, long, ihipStream_t*)",
    "gemv_iq4xs_stock_gpu(block_iq4_xs const*, float const*, float*, long, long, ihipStream_t*)",
    "gemm_iq4xs_stock_gpu(block_iq4_xs const*, float const*, float*, long, long, long, ihipStream_t*)",
    "gemv_iq4xs_gfx1100_gpu(block_iq4_xs const*, float const*, float*, long, long, ihipStream_t*)",
    "gemm_iq4xs_wmma_stream_gpu(block_iq4_xs const*, float const*, float*, long, long, long, ihipStream_t*)",
    "gemm_iq4xs_wmma_p4_xor_gpu(block_iq4_xs const*, float const*, float*, long, long, long, ihipStream_t*)",
    "gemm_iq4xs_wmma_64x64_gpu(block_iq4_xs const*, float const*, float*, long, long, long, ihipStream_t*)",
    "gemm_iq4xs_stream_tiled_gpu(block_iq4_xs const*, float const*, float*, long, long, long, ihipStream_t*)",
    "gemm_iq4xs_wmma_gpu(block_iq4_xs const*, float const*, float*, long, long, long, ihipStream_t*)",
    "gemm_iq4xs_tiled_gpu(block_iq4_xs const*, float const*, float*, long, long, long, ihipStream_t*)",
    "dequant_iq4xs_gpu(block_iq4_xs const*, float*, long, int, ihipStream_t*)",
}
# _Float16 in the LUT entry's signature: its mangled name, which binutils' demangler may not expand
LUT_MANGLED = "_Z18gemm_iq4xs_lut_gpuPK12block_iq4_xsPKDF16_PKfPflllP12ihipStream_t"


def test_library_exports_the_reference_cpp_api(L):
    """The reference's tests and benches forward-declare these mangled names
    (test_real_stock_compare.cpp:12-13, bench_gemm_wmma.cpp:23-28): the library
    defines each with exactly that signature, so they link unchanged."""
    out = subprocess.run(["nm", "-DC", "--defined-only", L.path], capture_output=True, text=True, check=True).stdout
    defined = {line.split(" ", 2)[2] for line in out.splitlines() if " T " in line}
    missing = sorted(REFERENCE_CPP_API - defined)
    assert not missing, missing
    raw = subprocess.run(["nm", "-D", "--defined-only", L.path], capture_output=True, text=True, check=True).stdout
    assert LUT_MANGLED in raw or any(s.startswith("gemm_iq4xs_lut_gpu(block_iq4_xs const*, _Float16 const*")
                                     for s in defined)


def test_cpp_boundary_binary_links_the_reference_names():
    """tests/cpp/boundary_test (built by __graft_entry__.build()) calls the hooks through
    include/iq4xs_ggml_custom.cuh and the standalone API through the reference's own
    declarations: the only library symbols it needs are the C hooks and those C++ names."""
    binary = os.path.join(ROOT, "tests", "cpp", "_build", "boundary_test")
    if not os.path.exists(binary):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "tests", "cpp")], check=True)
    out = subprocess.run(["nm", "-C", "--undefined-only", binary], capture_output=True, text=True, check=True).stdout
    und = {line.split(" U ", 1)[1].strip() for line in out.splitlines() if " U " in line}
    for hook in ("custom_gemv_iq4xs_can_handle", "custom_gemv_iq4xs_dispatch", "custom_gemm_iq4xs_can_handle",
                 "custom_gemm_iq4xs_dispatch"):
        assert hook in und, hook
    called = {s for s in und if "block_iq4_xs" in s or "block_q8_1_real" in s}
    assert called and called <= REFERENCE_CPP_API | {s for s in und if s.startswith("_Z18gemm_iq4xs_lut_gpu")}, called
