// reference_api.hip -- the reference's standalone entry points with their own
// C++ signatures (declared in include/iq4xs_reference_api.hpp), so that the
// reference's tests and benches, which forward-declare these mangled names
// (test_real_stock_compare.cpp:12-13, bench_gemm_wmma.cpp:23-28), link
// against this library unchanged.  Each forwards to the C entry point of the
// same name: the block pointer becomes const void*, the stream void*.
#include "iq4xs_reference_api.hpp"

namespace {
inline void* S(hipStream_t s) { return reinterpret_cast<void*>(s); }
inline hipError_t E(int code) { return static_cast<hipError_t>(code); }
}  // namespace

hipError_t quantize_row_q8_1_gpu(const float* d_x, block_q8_1_real* d_y, int64_t K, hipStream_t stream) {
    return E(::quantize_row_q8_1_gpu(d_x, static_cast<void*>(d_y), K, S(stream)));
}

hipError_t quantize_row_q8_1_batched_gpu(const float* d_X, block_q8_1_real* d_Y, int64_t K, int64_t M,
                                         hipStream_t stream) {
    return E(::quantize_row_q8_1_batched_gpu(d_X, static_cast<void*>(d_Y), K, M, S(stream)));
}

hipError_t gemv_iq4xs_stock_dp4a_gpu(const block_iq4_xs* d_W, const float* d_x, float* d_y, int64_t K, int64_t N,
                                     hipStream_t stream) {
    return E(::gemv_iq4xs_stock_dp4a_gpu(static_cast<const void*>(d_W), d_x, d_y, K, N, S(stream)));
}

hipError_t gemm_iq4xs_stock_dp4a_gpu(const block_iq4_xs* d_W, const float* d_X, float* d_Y, int64_t K, int64_t N,
                                     int64_t M, hipStream_t stream) {
    return E(::gemm_iq4xs_stock_dp4a_gpu(static_cast<const void*>(d_W), d_X, d_Y, K, N, M, S(stream)));
}

hipError_t gemv_iq4xs_dp4a_gfx1100_prequantized_gpu(const block_iq4_xs* d_W, const block_q8_1_coop* d_AQ,
                                                    float* d_y, int64_t K, int64_t N, hipStream_t stream) {
    return E(::gemv_iq4xs_dp4a_gfx1100_prequantized_gpu(static_cast<const void*>(d_W), static_cast<const void*>(d_AQ),
                                                         d_y, K, N, S(stream)));
}

hipError_t gemv_iq4xs_dp4a_gfx1100_gpu(const block_iq4_xs* d_W, const float* d_x, float* d_y, int64_t K, int64_t N,
                                       hipStream_t stream) {
    return E(::gemv_iq4xs_dp4a_gfx1100_gpu(static_cast<const void*>(d_W), d_x, d_y, K, N, S(stream)));
}

hipError_t gemv_iq4xs_stock_gpu(const block_iq4_xs* d_W, const float* d_x, float* d_y, int64_t K, int64_t N,
                                hipStream_t stream) {
    return E(::gemv_iq4xs_stock_gpu(static_cast<const void*>(d_W), d_x, d_y, K, N, S(stream)));
}

hipError_t gemm_iq4xs_stock_gpu(const block_iq4_xs* d_W, const float* d_X, float* d_Y, int64_t K, int64_t N,
                                int64_t M, hipStream_t stream) {
    return E(::gemm_iq4xs_stock_gpu(static_cast<const void*>(d_W), d_X, d_Y, K, N, M, S(stream)));
}

hipError_t gemv_iq4xs_gfx1100_gpu(const block_iq4_xs* d_W, const float* d_x, float* d_y, int64_t K, int64_t N,
                                  hipStream_t stream) {
    return E(::gemv_iq4xs_gfx1100_gpu(static_cast<const void*>(d_W), d_x, d_y, K, N, S(stream)));
}

hipError_t gemm_iq4xs_wmma_stream_gpu(const block_iq4_xs* d_W, const float* d_X, float* d_Y, int64_t K, int64_t N,
                                      int64_t M, hipStream_t stream) {
    return E(::gemm_iq4xs_wmma_stream_gpu(static_cast<const void*>(d_W), d_X, d_Y, K, N, M, S(stream)));
}

hipError_t gemm_iq4xs_wmma_p4_xor_gpu(const block_iq4_xs* d_W, const float* d_X, float* d_Y, int64_t K, int64_t N,
                                      int64_t M, hipStream_t stream) {
    return E(::gemm_iq4xs_wmma_p4_xor_gpu(static_cast<const void*>(d_W), d_X, d_Y, K, N, M, S(stream)));
}

hipError_t gemm_iq4xs_wmma_64x64_gpu(const block_iq4_xs* d_W, const float* d_X, float* d_Y, int64_t K, int64_t N,
                                     int64_t M, hipStream_t stream) {
    return E(::gemm_iq4xs_wmma_64x64_gpu(static_cast<const void*>(d_W), d_X, d_Y, K, N, M, S(stream)));
}

hipError_t gemm_iq4xs_stream_tiled_gpu(const block_iq4_xs* d_W, const float* d_X, float* d_Y, int64_t K, int64_t N,
                                       int64_t M, hipStream_t stream) {
    return E(::gemm_iq4xs_stream_tiled_gpu(static_cast<const void*>(d_W), d_X, d_Y, K, N, M, S(stream)));
}

hipError_t gemm_iq4xs_wmma_gpu(const block_iq4_xs* d_W, const float* d_X, float* d_Y, int64_t K, int64_t N, int64_t M,
                               hipStream_t stream) {
    return E(::gemm_iq4xs_wmma_gpu(static_cast<const void*>(d_W), d_X, d_Y, K, N, M, S(stream)));
}

hipError_t gemm_iq4xs_tiled_gpu(const block_iq4_xs* d_W, const float* d_X, float* d_Y, int64_t K, int64_t N,
                                int64_t M, hipStream_t stream) {
    return E(::gemm_iq4xs_tiled_gpu(static_cast<const void*>(d_W), d_X, d_Y, K, N, M, S(stream)));
}

hipError_t gemm_iq4xs_lut_gpu(const block_iq4_xs* d_W, const _Float16* d_LUT, const float* d_X, float* d_Y, int64_t K,
                              int64_t N, int64_t M, hipStream_t s) {
    return E(::gemm_iq4xs_lut_gpu(static_cast<const void*>(d_W), static_cast<const void*>(d_LUT), d_X, d_Y, K, N, M,
                                  S(s)));
}

hipError_t dequant_iq4xs_gpu(const block_iq4_xs* d_src, float* d_dst, int64_t n_blocks, int warp_size,
                             hipStream_t stream) {
    return E(::dequant_iq4xs_gpu(static_cast<const void*>(d_src), d_dst, n_blocks, warp_size, S(stream)));
}
