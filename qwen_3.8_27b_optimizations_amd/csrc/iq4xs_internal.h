// iq4xs_internal.h -- launchers shared between the kernel files and the C ABI.
#pragma once

#include "iq4xs_device.h"

namespace iq4xs {

// The runtime's last-error slot is per thread and shared with every other HIP
// user in the process: a failure some earlier call left unread would be
// reported as this library's.  Every launcher clears it first and then reads
// its own launches' status with hipGetLastError.
inline void clear_launch_error() { (void)hipGetLastError(); }

// Compute units of the current device, queried once per device (256 when the
// query fails); launchers size their grids with it.  Safe to call from any
// host thread.
int device_cu_count();

// Activation / output layouts.
constexpr int LAYOUT_KM = 0;  // X[k*M+m], Y[n*M+m]   (standalone API)
constexpr int LAYOUT_MK = 1;  // X[m*K+k], Y[m*N+n]   (ggml src1 / dst)

// Largest column count served by the streaming GEMV; wider batches go to the
// MFMA GEMM.
constexpr int GEMV_MAX_COLS = 8;
// Largest K whose single-column fused GEMV prologue takes the 16-byte vector
// loads (16-byte aligned x): five rounds of 1024 lanes x 4 elements.
constexpr int64_t GEMV_FUSED_VEC_MAX_K = 20480;

// Planar writers fill all three parts (qs, ds, hq) when qs is non-null.
hipError_t launch_quantize(const float* X, int64_t K, int64_t M, int layout, int8_t* qs, uint32_t* ds, uint32_t* hq,
                           block_q8_1* blocks, hipStream_t stream);
hipError_t launch_planar_to_blocks(const int8_t* qs, const uint32_t* ds, int64_t K, int64_t M, block_q8_1* blocks,
                                   hipStream_t stream);

// y[c] = W x[c] for c < M <= GEMV_MAX_COLS on planar Q8_1 activations.
// Output element (m, n) goes to Y[m*ldy_m + n*ldy_n].  dbg (optional) receives
// the scaled int32 sum of every sub-block: dbg[(m*N + n)*(K/32) + kb].
hipError_t launch_gemv(const uint8_t* W, const int8_t* aqs, const uint32_t* ads, float* Y, int64_t K, int64_t N,
                       int64_t M, int64_t ldy_m, int64_t ldy_n, int32_t* dbg, hipStream_t stream);

// Small-batch GEMV on the int8 matrix cores (1 <= M <= 8, same contract as
// launch_gemv); hipErrorNotSupported when the shape does not fit its LDS.
hipError_t launch_gemv_mfma(const uint8_t* W, const int8_t* aqs, const uint32_t* ads, float* Y, int64_t K,
                            int64_t N, int64_t M, int64_t ldy_m, int64_t ldy_n, int32_t* dbg, hipStream_t stream);

// Matrices run together by one grouped GEMV launch (same K, same activations).
constexpr int GEMV_GROUP_MAX = 4;

// The matrix-core GEMV over count <= GEMV_GROUP_MAX matrices in one launch
// (Y[i] element (m, n) at Y[i][m*ldy_m[i] + n*ldy_n]); every matrix must take
// the same wave count (gemv_mfma_waves), else hipErrorNotSupported.  dbg only
// with count == 1.  Outputs are bit-identical to one launch per matrix.
hipError_t launch_gemv_mfma_group(int count, const uint8_t* const* W, float* const* Y, const int64_t* N,
                                  const int64_t* ldy_m, const int8_t* aqs, const uint32_t* ads, int64_t K,
                                  int64_t M, int64_t ldy_n, int32_t* dbg, hipStream_t stream);
// Waves per workgroup the matrix-core GEMV gives an N-row matrix (its rows'
// summation order); matrices with equal counts can share a launch.
int gemv_mfma_waves(int64_t N);

// Y[i] = W[i] x for i < count <= GEMV_GROUP_MAX, M <= GEMV_MAX_COLS columns
// of planar Q8_1 activations; Y[i] in ggml layout [M][N[i]] (layout_mk) or
// [N[i]][M].  The matrices that launch_gemv runs on the matrix cores share a
// launch per wave count, the others one tile-kernel launch (one launch per
// matrix where the tile kernel does not take the shape); outputs are
// bit-identical to launch_gemv on each matrix.
hipError_t launch_gemv_group(int count, const uint8_t* const* W, float* const* Y, const int64_t* N,
                             const int8_t* aqs, const uint32_t* ads, int64_t K, int64_t M, bool layout_mk,
                             hipStream_t stream);

// Same contract with fp32 activations quantised inside the kernel (element
// (m, k) at X[m*sc + k*sk]); hipErrorNotSupported if the shape does not fit
// the fused kernel's LDS budget (then quantise separately).
hipError_t launch_gemv_fused(const uint8_t* W, const float* X, int64_t sc, int64_t sk, float* Y, int64_t K, int64_t N,
                             int64_t M, int64_t ldy_m, int64_t ldy_n, int32_t* dbg, hipStream_t stream);

// RMS norm of one column (h = X (+ R), written to H when non-null; y = (h *
// scale) * gamma) fused into a grouped bs=1 GEMV over its Q8_1 codes;
// hipErrorNotSupported for shapes the fused prologue does not take.
hipError_t launch_gemv_rms_group(int count, const uint8_t* const* W, float* const* Y, const int64_t* N,
                                 const float* X, const float* R, float* H, const float* gamma, float eps, int64_t K,
                                 hipStream_t stream);
// RMS norm + gate/up pair + SwiGLU in one bs=1 launch (S = silu(gate) * up).
hipError_t launch_gemv_rms_swiglu(const uint8_t* Wg, const uint8_t* Wu, float* Yg, float* Yu, float* S, int64_t N,
                                  const float* X, const float* R, float* H, const float* gamma, float eps, int64_t K,
                                  hipStream_t stream);

// Same contract on the matrix-core GEMM path (any M >= 1); it also reads the
// workspace's fp16 code pairs ahq.
hipError_t launch_gemm(const uint8_t* W, const int8_t* aqs, const uint32_t* ads, const uint32_t* ahq, float* Y,
                       int64_t K, int64_t N, int64_t M, int64_t ldy_m, int64_t ldy_n, int32_t* dbg,
                       hipStream_t stream);

// Y[i] = W[i] x for i < count <= GEMV_GROUP_MAX on the matrix-core GEMM path, one
// launch; Y[i] is [M][N[i]] (layout_mk) or [N[i]][M].
hipError_t launch_gemm_group(int count, const uint8_t* const* W, float* const* Y, const int64_t* N, const int8_t* aqs,
                             const uint32_t* ads, const uint32_t* ahq, int64_t K, int64_t M, bool layout_mk,
                             hipStream_t stream);

// One v_mfma_i32_32x32x32_i8 on A[32][32], B[32][32] (k-contiguous rows) ->
// C[32][32] = A B^T, through the operand layouts the small-batch matrix-core
// GEMV uses.
hipError_t launch_probe_mfma(const int8_t* A, const int8_t* B, int32_t* C, hipStream_t stream);

// n_blocks super-blocks -> fp32 weights (256 per block, in block order).
hipError_t launch_dequant(const uint8_t* src, float* dst, int64_t n_blocks, hipStream_t stream);

// FP64 comparators in the reference's loop orders (stock: X [K][M] -> Y [N][M];
// gfx1100: one column) and the 64-byte padded Q8_1 blocks of its cooperative
// GEMV -> planar workspace (one column of nb blocks).
hipError_t launch_stock_fp64(const uint8_t* W, const float* X, float* Y, int64_t K, int64_t N, int64_t M,
                             hipStream_t stream);
hipError_t launch_gfx1100_fp64(const uint8_t* W, const float* x, float* y, int64_t K, int64_t N, hipStream_t stream);
hipError_t launch_coop_to_planar(const uint8_t* coop, int64_t nb, int8_t* qs, uint32_t* ds, uint32_t* hq,
                                 hipStream_t stream);

// Producers writing the planar Q8_1 workspace (row-major [M][K] inputs).
// rms norm: h = X (+ R) (stored to H when non-null; H may equal X or R),
// y = (h * 1/sqrt(mean(h^2) + eps)) * gamma; swiglu: y = silu(G) * U.
hipError_t launch_rms_norm_q8_1(const float* X, const float* R, float* H, const float* gamma, float eps, int64_t K,
                                int64_t M, int8_t* qs, uint32_t* ds, uint32_t* hq, hipStream_t stream);
hipError_t launch_swiglu_q8_1(const float* G, const float* U, int64_t K, int64_t M, int8_t* qs, uint32_t* ds,
                              uint32_t* hq, hipStream_t stream);

hipError_t launch_fill_weights(uint8_t* W, int64_t n_blocks, uint64_t seed, int64_t first_block,
                               hipStream_t stream);
hipError_t launch_fill_activations(float* x, int64_t n, uint64_t seed, int outliers, hipStream_t stream);

}  // namespace iq4xs
