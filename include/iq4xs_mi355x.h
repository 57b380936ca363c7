/*
 * iq4xs_mi355x.h -- C ABI of the MI355X (gfx950) IQ4_XS x Q8_1 mul_mat library
 * (libiq4xs_mi355x.so).
 *
 * Every entry point takes plain device pointers and sizes; `stream` is a
 * hipStream_t passed as void* (NULL = the default stream).  Return values are
 * hipError_t codes as int:
 *   IQ4XS_SUCCESS                 0  hipSuccess
 *   IQ4XS_ERROR_INVALID_VALUE     1  hipErrorInvalidValue  (null pointer, K <= 0,
 *                                    K % 256 != 0, N <= 0, M <= 0, bad layout,
 *                                    workspace too small)
 *   IQ4XS_ERROR_INVALID_CONFIG    9  hipErrorInvalidConfiguration (grid too large)
 *   IQ4XS_ERROR_NOT_SUPPORTED   801  hipErrorNotSupported (e.g. shape not served)
 * or any other hipError_t reported by the runtime.  Arguments are validated
 * before anything is launched; a failing call launches nothing.
 *
 * Reference citations are file:line in the reference repository; "patch"
 * means patches/0001-gfx1100-mul-mat-custom.patch.
 *
 * Data formats (byte-compatible with ggml):
 *   W     : IQ4_XS, row-major [N][K/256] blocks of 136 bytes
 *           (kernels/common/block_iq4_xs.h:10-19)
 *   Q8_1  : 36-byte blocks {uint32 ds = fp16 d | fp16 sum << 16, int8 qs[32]}
 *           (real_stock_dp4a_comparator.hip:22-26); d and sum are encoded with
 *           round-toward-zero as the reference's pack_half2 (:43-62)
 */
#ifndef IQ4XS_MI355X_H
#define IQ4XS_MI355X_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IQ4XS_SUCCESS 0
#define IQ4XS_ERROR_INVALID_VALUE 1
#define IQ4XS_ERROR_INVALID_CONFIG 9
#define IQ4XS_ERROR_NOT_SUPPORTED 801

#define IQ4XS_QK_K 256
#define IQ4XS_QK8_1 32
#define IQ4XS_BLOCK_BYTES 136
#define IQ4XS_Q8_1_BLOCK_BYTES 36
#define IQ4XS_GGML_TYPE_IQ4_XS 23 /* ggml_type value of GGML_TYPE_IQ4_XS */

/* Activation / output layouts */
#define IQ4XS_LAYOUT_KM 0 /* X[k*M + m], Y[n*M + m]  (standalone kernels/matmul_iq4xs API) */
#define IQ4XS_LAYOUT_MK 1 /* X[m*K + k], Y[m*N + n]  (ggml src1 / dst)                    */

/* Kernel selection for iq4xs_mul_mat_q8_1 / iq4xs_subblock_sums */
#define IQ4XS_PATH_AUTO -1 /* streaming GEMV for M <= 8, matrix-core GEMM above */
#define IQ4XS_PATH_GEMV 0  /* streaming GEMV (M <= 8 only)                   */
#define IQ4XS_PATH_GEMM 1  /* matrix-core GEMM (any M)                       */

/* ===================== standalone API (kernels/matmul_iq4xs) ===================== */

/* Replaces quantize_row_q8_1_gpu, real_stock_dp4a_comparator.hip:266-273.
 * x[K] fp32 -> y[K/32] Q8_1 blocks.  K % 32 == 0. */
int quantize_row_q8_1_gpu(const float* x, void* y, int64_t K, void* stream);

/* Replaces quantize_row_q8_1_batched_gpu, real_stock_dp4a_comparator.hip:308-315.
 * X[k*M + m] -> Y[m*(K/32) + ib].  K % 32 == 0. */
int quantize_row_q8_1_batched_gpu(const float* X, void* Y, int64_t K, int64_t M, void* stream);

/* Replaces gemv_iq4xs_stock_dp4a_gpu, real_stock_dp4a_comparator.hip:480-503:
 * y[N] = W x (x quantised to Q8_1 first).  For K <= 20480 with x 16-byte
 * aligned (K <= 8192 otherwise) the quantisation runs inside the GEMV kernel
 * (one launch, no scratch); otherwise the Q8_1 scratch comes from the
 * library's stream-ordered pool (hipMallocFromPoolAsync/hipFreeAsync on
 * `stream`): no device-wide synchronisation, unlike the reference's
 * hipMalloc/hipFree. */
int gemv_iq4xs_stock_dp4a_gpu(const void* W, const float* x, float* y, int64_t K, int64_t N, void* stream);

/* Replaces the C-linkage gemv_iq4xs_dp4a_coop_gpu, impl_gemv_dp4a_gfx1100.hip:332-341
 * (same contract as gemv_iq4xs_stock_dp4a_gpu). */
int gemv_iq4xs_dp4a_coop_gpu(const void* W, const float* x, float* y, int64_t K, int64_t N, void* stream);

/* Replaces gemv_iq4xs_dp4a_gfx1100_gpu, impl_gemv_dp4a_gfx1100.hip:310-329
 * (same contract as gemv_iq4xs_stock_dp4a_gpu). */
int gemv_iq4xs_dp4a_gfx1100_gpu(const void* W, const float* x, float* y, int64_t K, int64_t N, void* stream);

/* Replaces gemv_iq4xs_dp4a_gfx1100_prequantized_gpu, impl_gemv_dp4a_gfx1100.hip:291-308:
 * y = W * dequant(AQ) for activations already quantised into the reference's
 * 64-byte padded Q8_1 blocks (ds at byte 0, the 32 codes at bytes 16..47;
 * impl_gemv_dp4a_gfx1100.hip:60-66), K/32 of them, 16-byte aligned.  The
 * blocks are copied to a planar workspace from the stream-ordered pool. */
int gemv_iq4xs_dp4a_gfx1100_prequantized_gpu(const void* W, const void* AQ, float* y, int64_t K, int64_t N,
                                             void* stream);

/* Replaces the FP64 comparators gemv_iq4xs_stock_gpu / gemm_iq4xs_stock_gpu,
 * stock_hip_comparator.hip:120-151 (X [K][M], Y [N][M]): per output one double
 * sum of (double)(fp16 d * (ls-32)) * kvalue * (double)x in the loop order of
 * ref_cpu.cpp:12-106, products and sums rounded separately, so the outputs
 * equal the reference's CPU FP64 oracle bit for bit.  One thread per output:
 * a comparator, not a fast path. */
int gemv_iq4xs_stock_gpu(const void* W, const float* x, float* y, int64_t K, int64_t N, void* stream);
int gemm_iq4xs_stock_gpu(const void* W, const float* X, float* Y, int64_t K, int64_t N, int64_t M, void* stream);

/* Replaces gemv_iq4xs_gfx1100_gpu, impl_gemv_gfx1100.hip:99-120: the same FP64
 * products, summed as 8 partials per row (one per sub-block index, over all
 * super-blocks) that are then added in index order, as that kernel does. */
int gemv_iq4xs_gfx1100_gpu(const void* W, const float* x, float* y, int64_t K, int64_t N, void* stream);

/* Replace the fp16-WMMA GEMM family and its tiled fallbacks:
 * gemm_iq4xs_wmma_stream_gpu / _wmma_p4_xor_gpu / _wmma_64x64_gpu and
 * gemm_iq4xs_stream_tiled_gpu (impl_gemm_wmma_stream.hip:321-364),
 * gemm_iq4xs_wmma_gpu / gemm_iq4xs_tiled_gpu (impl_gemm_wmma.hip:199-242).
 * Same signature and layout as gemm_iq4xs_stock_dp4a_gpu (X [K][M], Y [N][M]),
 * same argument checks.  They run this library's matrix-core GEMM on Q8_1
 * activations (exact integer sub-block sums, the reference's Q8_1 semantics):
 * the reference's fp16 numerics (dequantised weights x fp16-cast activations)
 * are not reproduced. */
int gemm_iq4xs_wmma_stream_gpu(const void* W, const float* X, float* Y, int64_t K, int64_t N, int64_t M,
                               void* stream);
int gemm_iq4xs_wmma_p4_xor_gpu(const void* W, const float* X, float* Y, int64_t K, int64_t N, int64_t M,
                               void* stream);
int gemm_iq4xs_wmma_64x64_gpu(const void* W, const float* X, float* Y, int64_t K, int64_t N, int64_t M,
                              void* stream);
int gemm_iq4xs_stream_tiled_gpu(const void* W, const float* X, float* Y, int64_t K, int64_t N, int64_t M,
                                void* stream);
int gemm_iq4xs_wmma_gpu(const void* W, const float* X, float* Y, int64_t K, int64_t N, int64_t M, void* stream);
int gemm_iq4xs_tiled_gpu(const void* W, const float* X, float* Y, int64_t K, int64_t N, int64_t M, void* stream);

/* Replaces gemm_iq4xs_lut_gpu, impl_gemm_lut_iq4xs.hip:138-157.  The codebook
 * table LUT is accepted and not read (IQ4_XS fixes it).  Same gate as the
 * reference: hipErrorInvalidConfiguration unless M, N, K are multiples of 16
 * with M >= 512, N >= 32, K >= 32; otherwise as gemm_iq4xs_stock_dp4a_gpu. */
int gemm_iq4xs_lut_gpu(const void* W, const void* LUT, const float* X, float* Y, int64_t K, int64_t N, int64_t M,
                       void* stream);

/* Replaces gemm_iq4xs_stock_dp4a_gpu, real_stock_dp4a_comparator.hip:505-548:
 * Y[n*M + m] = sum_k W[n,k] X[k*M + m].  M <= 8 runs the streaming GEMV,
 * larger M the matrix-core GEMM. */
int gemm_iq4xs_stock_dp4a_gpu(const void* W, const float* X, float* Y, int64_t K, int64_t N, int64_t M,
                              void* stream);

/* Replaces dequant_iq4xs_gpu, kernels/demo_iq4xs_dequant/impl.hip:51-69:
 * n_blocks super-blocks -> 256*n_blocks fp32 weights, bit-identical to the
 * reference's CPU dequantiser (ref_cpu.cpp:6-27).  warp_size is accepted for
 * signature compatibility (32 or 64, anything else is hipErrorInvalidValue);
 * the kernel always runs wave64.  n_blocks == 0 launches nothing and succeeds. */
int dequant_iq4xs_gpu(const void* src, float* dst, int64_t n_blocks, int warp_size, void* stream);

/* ============================ ggml mul_mat boundary ============================ */

/* Replaces custom_gemv_iq4xs_can_handle, patch:274-277.  True for
 * type == GGML_TYPE_IQ4_XS, M == 1 (custom_gemv_iq4xs_dispatch computes one
 * column), K > 0, K % 256 == 0, N > 0 (the reference's K/N whitelist is
 * dropped).  Batches of 2..8 columns are served by custom_gemm_iq4xs_dispatch,
 * which routes them to the small-batch GEMV. */
bool custom_gemv_iq4xs_can_handle(int64_t K, int64_t N, int64_t M, int type);

/* Replaces custom_gemv_iq4xs_dispatch, patch:278-280 (called from the mmvq.cu
 * hook, patch:327-334): y[N] = W x for ggml's src0/src1/dst of one column.
 * Stream-ordered; no host synchronisation (the reference synchronises the
 * stream and refuses graph capture, patch:269-272). */
int custom_gemv_iq4xs_dispatch(const void* W, const float* x, float* y, int64_t K, int64_t N, void* stream);

/* Replaces custom_gemm_iq4xs_can_handle, patch:148-151: type == IQ4_XS,
 * M >= 1, K > 0, K % 256 == 0, N > 0. */
bool custom_gemm_iq4xs_can_handle(int64_t K, int64_t N, int64_t M, int type);

/* Replaces custom_gemm_iq4xs_dispatch, patch:152-154 (mmq.cu hook,
 * patch:299-306): ggml layout X[m*K + k] -> Y[m*N + n]. */
int custom_gemm_iq4xs_dispatch(const void* W, const float* X, float* Y, int64_t K, int64_t N, int64_t M,
                               void* stream);

/* ====================== explicit-workspace API (capture-safe) ======================
 * No counterpart in the reference (which allocates per call, e.g.
 * real_stock_dp4a_comparator.hip:491,501).  For callers that own their memory:
 * the calls below allocate nothing and never synchronise.  The workspace holds
 * Q8_1 activations in planar form: int8 codes [M][K] at offset 0, then the
 * uint32 ds words [M][K/32], then the same codes as fp16 pairs [M][K/32][16]
 * (uint32 word p of a 32-element block = elements p and p + 16), each part at
 * a 256-byte aligned offset: 3 * K * M + K * M / 8 bytes and padding.  Every
 * call that writes a workspace fills all three parts. */

/* Bytes of workspace for M activation columns of length K; 0 for shapes the
 * entry points refuse (K not a positive multiple of 32, M < 1, K or M >= 2^31). */
size_t iq4xs_workspace_bytes(int64_t K, int64_t M);

/* X (layout IQ4XS_LAYOUT_KM or _MK) -> planar Q8_1 in ws. */
int iq4xs_quantize_q8_1(const float* X, int64_t K, int64_t M, int layout, void* ws, size_t ws_bytes,
                        void* stream);

/* Fused producers: the op that writes a mul_mat activation, quantised to
 * planar Q8_1 in ws on the way out (row-major inputs, row m at [m*K]).  They
 * stand for ggml's RMS_NORM + MUL and SWIGLU ahead of the projections
 * (profiled by the reference at benchmarks/profiling/BOTTLENECK-TABLE.md:
 * 24,26,30) and have no kernel counterpart in the reference.  K % 32 == 0.
 *
 * rms norm: h = X + R (R may be NULL), written to H when H is non-NULL
 * (H may be exactly X or R: the in-place residual add); then
 *   mean = (float)(sum (double)(h*h) / K), scale = 1.0f / sqrtf(mean + eps),
 *   y = (h * scale) * gamma[k]       (gamma NULL: y = h * scale)
 * with the sum in a fixed order, so results are reproducible bit for bit.
 * The Qwen-27B-class models use eps = 1e-6
 * (benchmarks/environment/startup-log.txt:128).  X, R, H 16-byte aligned. */
int iq4xs_rms_norm_q8_1(const float* X, const float* R, float* H, const float* gamma, float eps, int64_t K,
                        int64_t M, void* ws, size_t ws_bytes, void* stream);

/* swiglu: y = silu(G) * U, silu(g) = g / (1 + exp(-g)) (exp computed by the
 * library's own Cody-Waite reduction, <= 1 ulp). */
int iq4xs_swiglu_q8_1(const float* G, const float* U, int64_t K, int64_t M, void* ws, size_t ws_bytes,
                      void* stream);

/* RMS norm fused into a grouped bs=1 GEMV: the same result as
 * iq4xs_rms_norm_q8_1(X, R, H, gamma, eps, K, 1, ws) followed by
 * iq4xs_mul_mat_q8_1_group(count, W, Y, N, ws, K, 1, ...) -- Y and H bit for
 * bit -- in one launch and with no workspace: every workgroup of the GEMV
 * runs the norm's passes on the row and quantises it into its own LDS, and
 * workgroup 0 writes H.  For the norm ahead of q/k/v or gate/up at decode.
 * No counterpart in the reference, which runs RMS_NORM, MUL and each
 * projection as separate ggml ops.
 *   - H (may be NULL) must not overlap X or R, and no Y[i] may overlap X, R or H
 *     (in-place forms are rejected with hipErrorInvalidValue);
 *   - X, R, H, gamma 16-byte aligned; K % 256 == 0, eps >= 0;
 *   - hipErrorNotSupported for K < 2048 or K > 8192, or when the row does not
 *     fit the kernel's LDS: use the two calls. */
int iq4xs_rms_norm_mul_mat_group(int count, const void* const* W, float* const* Y, const int64_t* N, const float* X,
                                 const float* R, float* H, const float* gamma, float eps, int64_t K, void* stream);

/* RMS norm, the gate/up pair of a SwiGLU MLP and the SwiGLU itself in one bs=1
 * launch: the same h, gate and up as iq4xs_rms_norm_mul_mat_group(2,
 * {W_gate, W_up}, {Y_gate, Y_up}, {N, N}, X, R, H, gamma, eps, K) -- bit for
 * bit -- and S[n] = silu(gate[n]) * up[n] in fp32 with iq4xs_swiglu_q8_1's
 * arithmetic, so iq4xs_mul_mat(W_down, S, ...) gives the bits of the SwiGLU
 * producer followed by the down GEMV, one launch earlier.  Each workgroup
 * owns the same rows of gate and up.  No counterpart in the reference, which
 * runs RMS_NORM, MUL, the two projections and SWIGLU as separate ggml ops.
 *   - Y_gate, Y_up may be NULL (not written); S must not be NULL;
 *   - H (may be NULL) must not overlap X or R; Y_gate, Y_up and S must not
 *     overlap X, R, H or each other;
 *   - X, R, H, gamma 16-byte aligned; K % 256 == 0, eps >= 0;
 *   - hipErrorNotSupported as iq4xs_rms_norm_mul_mat_group, or when N has no
 *     divisor that makes every workgroup's rows whole steps: use the group
 *     call and iq4xs_swiglu_q8_1. */
int iq4xs_rms_norm_mul_mat_swiglu(const void* W_gate, const void* W_up, int64_t N, const float* X, const float* R,
                                  float* H, const float* gamma, float eps, int64_t K, float* Y_gate, float* Y_up,
                                  float* S, void* stream);

/* Y = W * dequant(ws) from an already quantised workspace; `layout` selects
 * the Y layout; `path` is one of IQ4XS_PATH_*. */
int iq4xs_mul_mat_q8_1(const void* W, const void* ws, float* Y, int64_t K, int64_t N, int64_t M, int layout,
                       int path, void* stream);

/* Several weight matrices (1 <= count <= 4, each N[i] x K) against the same
 * quantised activations in ws: Y[i] = W[i] * dequant(ws), Y[i] laid out as
 * `layout` selects.  For M <= 8 one launch of the streaming GEMV covers
 * every matrix (q/k/v, gate/up of a decode step) and pays the per-launch
 * fixed cost once; the matrices that take the matrix-core GEMV (M >= 4 and
 * N >= 2048, or M == 8 and N >= 1024) share one launch of it per wave count
 * (the count follows N),
 * the others one launch of the streaming GEMV.  For M > 8 one GEMM launch, whose
 * small matrices fill the CUs that the big ones' last round of tiles leaves
 * idle (a short last round lying in the last matrix is a second launch of
 * the small-tile kernel).  Each output is bit-identical to
 * iq4xs_mul_mat_q8_1 (path AUTO) on its own matrix.  W, Y, N are host arrays
 * of count entries.  No
 * counterpart in the reference, which runs every projection as its own
 * mul_mat. */
int iq4xs_mul_mat_q8_1_group(int count, const void* const* W, float* const* Y, const int64_t* N, const void* ws,
                             int64_t K, int64_t M, int layout, void* stream);

/* Quantise + multiply in one call.  For M == 1 and K <= 20480 with X 16-byte
 * aligned (K <= 8192 otherwise) the quantisation runs inside the GEMV kernel
 * and ws is not written (it is still validated). */
int iq4xs_mul_mat(const void* W, const float* X, float* Y, int64_t K, int64_t N, int64_t M, int layout, void* ws,
                  size_t ws_bytes, void* stream);

/* Largest Q8_1 workspace (iq4xs_workspace_bytes(K, M)) iq4xs_mul_mat_noalloc
 * serves: 128 MiB, e.g. M <= 2460 at K = 17408, M <= 8380 at K = 5120. */
#define IQ4XS_NOALLOC_SCRATCH_BYTES (128u << 20)

/* iq4xs_mul_mat without a workspace argument and without any allocation: the
 * Q8_1 workspace is a static device array of IQ4XS_NOALLOC_SCRATCH_BYTES held
 * by the library (one per GPU, for the life of the process).  The array is part
 * of the library's code object, so every process that runs any kernel of this
 * library on a GPU holds those 128 MiB of that GPU's memory, whether or not it
 * ever calls iq4xs_mul_mat_noalloc.  No counterpart
 * in the reference; for callers that cannot allocate -- code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  Same results
 * as iq4xs_mul_mat bit for bit.  IQ4XS_ERROR_INVALID_VALUE when
 * iq4xs_workspace_bytes(K, M) exceeds IQ4XS_NOALLOC_SCRATCH_BYTES.  Every call
 * on one GPU shares that GPU's scratch: calls that overlap on one GPU (other
 * streams, other host threads) race; serialise them. */
int iq4xs_mul_mat_noalloc(const void* W, const float* X, float* Y, int64_t K, int64_t N, int64_t M, int layout,
                          void* stream);

/* Small-batch (1 <= M <= 8) multiply that quantises X to Q8_1 inside the GEMV
 * kernel (one launch, no workspace).  Same Q8_1 codes and sums as
 * iq4xs_quantize_q8_1 + iq4xs_mul_mat_q8_1.  Returns IQ4XS_ERROR_NOT_SUPPORTED
 * when M*K does not fit the kernel's on-chip activation buffer; the caller then
 * uses the two-step path.  S (may be NULL) receives the per-sub-block int32
 * sums exactly as iq4xs_subblock_sums lays them out. */
int iq4xs_mul_mat_fused(const void* W, const float* X, float* Y, int64_t K, int64_t N, int64_t M, int layout,
                        int32_t* S, void* stream);

/* ================================ debug exports ================================
 * No counterpart in the reference; they exist so the Q8_1 blocks and the
 * per-32-element int32 sums can be checked bit for bit. */

/* Planar workspace -> M*(K/32) 36-byte Q8_1 blocks (block (m, ib) at m*(K/32)+ib). */
int iq4xs_q8_1_to_blocks(const void* ws, void* blocks, int64_t K, int64_t M, void* stream);

/* S[(m*N + n)*(K/32) + kb] = sumi * (ls - 32) of sub-block kb, row n, column m,
 * computed by the production kernel selected by `path` (IQ4XS_PATH_GEMV or
 * _GEMM: the same device code as iq4xs_mul_mat_q8_1, with one extra store).
 * The kernel also writes its outputs to Y (M*N floats, layout IQ4XS_LAYOUT_MK). */
int iq4xs_subblock_sums(const void* W, const void* ws, int32_t* S, float* Y, int64_t K, int64_t N, int64_t M,
                        int path, void* stream);

/* One v_mfma_i32_32x32x32_i8 through the operand and result layouts that the
 * small-batch matrix-core GEMV relies on: C[i*32 + j] = sum_k A[i*32 + k] * B[j*32 + k]. */
int iq4xs_probe_mfma_i8(const int8_t* A, const int8_t* B, int32_t* C, void* stream);

/* ============================ synthetic inputs ============================ */

/* n_blocks IQ4_XS blocks made on the device from `seed` (block i is the
 * recipe's block first_block + i). */
int iq4xs_fill_synthetic_weights(void* W, int64_t n_blocks, uint64_t seed, int64_t first_block, void* stream);

/* n fp32 activations ~ N(0,1); outliers != 0 scales 1 % of them x20. */
int iq4xs_fill_synthetic_activations(float* x, int64_t n, uint64_t seed, int outliers, void* stream);

/* Library version string. */
const char* iq4xs_version(void);

#ifdef __cplusplus
}
#endif
#endif
