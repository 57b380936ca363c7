// iq4xs_reference_api.hpp -- the reference's standalone C++ API
// (kernels/matmul_iq4xs, kernels/demo_iq4xs_dequant), with its exact
// signatures: block pointers typed as the reference's structs and hipStream_t
// streams.  The reference's tests and benches forward-declare these C++
// (mangled) names themselves, e.g. test_real_stock_compare.cpp:12-13 and
// bench_gemm_wmma.cpp:23-28; libiq4xs_mi355x.so defines every one of them
// (csrc/reference_api.hip), so those sources link against it unchanged.
// Each forwards to the C entry point of the same name in iq4xs_mi355x.h
// (overloads: the C ones take const void* and a void* stream).
//
// Including this header is optional: it gives the declarations (with the
// reference's default stream argument) to callers that do not declare them
// themselves.  The block types stay incomplete here; the reference's own
// definitions (136, 36 and 64 bytes) are the byte layouts the library reads.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "iq4xs_mi355x.h"

struct block_iq4_xs;     // kernels/common/block_iq4_xs.h:10-19
struct block_q8_1_real;  // real_stock_dp4a_comparator.hip:22-26
struct block_q8_1_coop;  // impl_gemv_dp4a_gfx1100.hip:60-66

// real_stock_dp4a_comparator.hip:266, :308, :480, :505
hipError_t quantize_row_q8_1_gpu(const float* d_x, block_q8_1_real* d_y, int64_t K, hipStream_t stream = 0);
hipError_t quantize_row_q8_1_batched_gpu(const float* d_X, block_q8_1_real* d_Y, int64_t K, int64_t M,
                                         hipStream_t stream = 0);
hipError_t gemv_iq4xs_stock_dp4a_gpu(const block_iq4_xs* d_W, const float* d_x, float* d_y, int64_t K, int64_t N,
                                     hipStream_t stream = 0);
hipError_t gemm_iq4xs_stock_dp4a_gpu(const block_iq4_xs* d_W, const float* d_X, float* d_Y, int64_t K, int64_t N,
                                     int64_t M, hipStream_t stream = 0);

// impl_gemv_dp4a_gfx1100.hip:291, :310 (its :332 gemv_iq4xs_dp4a_coop_gpu is
// already extern "C" in the reference and is the C entry point itself)
hipError_t gemv_iq4xs_dp4a_gfx1100_prequantized_gpu(const block_iq4_xs* d_W, const block_q8_1_coop* d_AQ,
                                                    float* d_y, int64_t K, int64_t N, hipStream_t stream = 0);
hipError_t gemv_iq4xs_dp4a_gfx1100_gpu(const block_iq4_xs* d_W, const float* d_x, float* d_y, int64_t K, int64_t N,
                                       hipStream_t stream = 0);

// stock_hip_comparator.hip:120, :136; impl_gemv_gfx1100.hip:99
hipError_t gemv_iq4xs_stock_gpu(const block_iq4_xs* d_W, const float* d_x, float* d_y, int64_t K, int64_t N,
                                hipStream_t stream = 0);
hipError_t gemm_iq4xs_stock_gpu(const block_iq4_xs* d_W, const float* d_X, float* d_Y, int64_t K, int64_t N,
                                int64_t M, hipStream_t stream = 0);
hipError_t gemv_iq4xs_gfx1100_gpu(const block_iq4_xs* d_W, const float* d_x, float* d_y, int64_t K, int64_t N,
                                  hipStream_t stream = 0);

// impl_gemm_wmma_stream.hip:321 (three builds of one source), :353; impl_gemm_wmma.hip:199, :229
hipError_t gemm_iq4xs_wmma_stream_gpu(const block_iq4_xs* d_W, const float* d_X, float* d_Y, int64_t K, int64_t N,
                                      int64_t M, hipStream_t stream = 0);
hipError_t gemm_iq4xs_wmma_p4_xor_gpu(const block_iq4_xs* d_W, const float* d_X, float* d_Y, int64_t K, int64_t N,
                                      int64_t M, hipStream_t stream = 0);
hipError_t gemm_iq4xs_wmma_64x64_gpu(const block_iq4_xs* d_W, const float* d_X, float* d_Y, int64_t K, int64_t N,
                                     int64_t M, hipStream_t stream = 0);
hipError_t gemm_iq4xs_stream_tiled_gpu(const block_iq4_xs* d_W, const float* d_X, float* d_Y, int64_t K, int64_t N,
                                       int64_t M, hipStream_t stream = 0);
hipError_t gemm_iq4xs_wmma_gpu(const block_iq4_xs* d_W, const float* d_X, float* d_Y, int64_t K, int64_t N, int64_t M,
                               hipStream_t stream = 0);
hipError_t gemm_iq4xs_tiled_gpu(const block_iq4_xs* d_W, const float* d_X, float* d_Y, int64_t K, int64_t N,
                                int64_t M, hipStream_t stream = 0);

// impl_gemm_lut_iq4xs.hip:138 (the codebook table is not read: IQ4_XS fixes it)
hipError_t gemm_iq4xs_lut_gpu(const block_iq4_xs* d_W, const _Float16* d_LUT, const float* d_X, float* d_Y, int64_t K,
                              int64_t N, int64_t M, hipStream_t s = 0);

// kernels/demo_iq4xs_dequant/impl.hip:51
hipError_t dequant_iq4xs_gpu(const block_iq4_xs* d_src, float* d_dst, int64_t n_blocks, int warp_size,
                             hipStream_t stream);
