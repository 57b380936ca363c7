/*
 * iq4xs_oracle.h -- CPU restatement of the reference IQ4_XS x Q8_1 mul_mat path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py may load it.
 * The product (libiq4xs_mi355x.so) never links or calls it.
 *
 * Every function names the reference file:line it restates.  All reference
 * paths are relative to the reference repository root.
 *
 * Pinning (what checks each function against something independent):
 *   orc_fp16_to_fp32          exhaustive over 65536 patterns vs numpy float16
 *   orc_fp32_to_fp16_trunc    structured sweep vs numpy RNE + round-toward-zero
 *                             correction and closed-form special cases
 *   block layout / generator  5 reference KAT sha256 values
 *                             (kernels/fixtures/manifest.json:3-81)
 *   orc_dequant               closed-form hand values of the KAT blocks, and
 *                             the compiled reference dequant_mat_iq4xs_cpu
 *   orc_quantize_q8_1         hand-derived known answers (zero block, single
 *                             nonzero, exact .5 ties, -0.0, order-sensitive
 *                             sums) and brute force on tiny inputs
 *   orc_subblock_sums         exact int64 brute force over dequantised codes
 *   orc_gemv_fp64/gemm_fp64   bit-exact vs the compiled reference ref_cpu.cpp
 *                             golden outputs (tests/golden) and numpy float64
 *   orc_gemv_fp64_by_subblock numpy float64 (1e-12), and the golden FP64
 *                             outputs to float rounding
 *   orc_exp_cw / orc_silu     error bound vs float64 exp / silu (<= 2 / 4 ulp)
 *                             over a dense sweep, exact special values
 *   orc_rms_norm_q8_1         scale vs float64 RMS within 2^-22 (eps-sensitive
 *                             small-magnitude rows included), closed forms
 *                             (constant rows, one nonzero), blocks through
 *                             orc_quantize_q8_1 of the returned values
 *   orc_swiglu_q8_1           values vs float64 silu(g)*u, blocks through
 *                             orc_quantize_q8_1 of the returned values
 *   orc_gemv_q8_1_host        bit-identical to orc_quantize_q8_1 +
 *                             orc_gemv_semantics (tests/test_oracle.py)
 *   orc_gemv_semantics        fp32 summation ORDER of the gfx1100 kernel is
 *   orc_gemm_semantics        parity unpinned (no gfx1100 here); the integer
 *                             terms are pinned by orc_subblock_sums and the
 *                             value by the FP64 oracle on dequantised Q8_1.
 */
#ifndef IQ4XS_ORACLE_H
#define IQ4XS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK_K 256
#define ORC_QK8_1 32

/* kernels/common/block_iq4_xs.h:10-19 -- 136-byte super-block. */
typedef struct __attribute__((packed)) {
    uint16_t d;
    uint16_t scales_h;
    uint8_t scales_l[4];
    uint8_t qs[128];
} orc_block_iq4_xs;

/* real_stock_dp4a_comparator.hip:22-26 -- ds = {fp16 d (lo), fp16 sum (hi)}. */
typedef struct {
    uint32_t ds;
    int8_t qs[ORC_QK8_1];
} orc_block_q8_1;

/* Activation layouts of the batched quantiser. */
#define ORC_LAYOUT_KM 0 /* X[k*M + m]: standalone API (real_stock_dp4a_comparator.hip:278-306) */
#define ORC_LAYOUT_MK 1 /* X[m*K + k]: ggml src1 layout (patch:117,129)               */

extern const int8_t orc_kvalues_iq4nl[16];

float orc_fp16_to_fp32(uint16_t h);
uint16_t orc_fp32_to_fp16_trunc(float f);
void orc_fp16_to_fp32_array(const uint16_t* h, float* out, size_t n);
void orc_fp32_to_fp16_trunc_array(const float* f, uint16_t* out, size_t n);

int orc_subblock_scale(const orc_block_iq4_xs* b, int ib);

void orc_quantize_q8_1(const float* x, orc_block_q8_1* y, int64_t K);
void orc_quantize_q8_1_batched(const float* X, orc_block_q8_1* Y, int64_t K, int64_t M, int layout);
void orc_dequant_q8_1(const orc_block_q8_1* y, float* xhat, int64_t n_blocks);

int32_t orc_subblock_sumi(const orc_block_iq4_xs* bq4, const orc_block_q8_1* bq8_chunk, int ib);
void orc_subblock_sums(const orc_block_iq4_xs* W, const orc_block_q8_1* AQ, int32_t* S,
                       int64_t K, int64_t N, int64_t M);

void orc_gemv_semantics(const orc_block_iq4_xs* W, const orc_block_q8_1* AQ, float* y,
                        int64_t K, int64_t N);
void orc_gemm_semantics(const orc_block_iq4_xs* W, const orc_block_q8_1* AQ, float* Y,
                        int64_t K, int64_t N, int64_t M);

void orc_gemv_fp64(const orc_block_iq4_xs* W, const float* x, float* y, int64_t K, int64_t N);
void orc_gemm_fp64(const orc_block_iq4_xs* W, const float* X, float* Y, int64_t K, int64_t N,
                   int64_t M, int nthreads);
void orc_dequant(const orc_block_iq4_xs* W, float* out, int64_t K, int64_t N);
void orc_gemv_fp64_by_subblock(const orc_block_iq4_xs* W, const float* x, float* y, int64_t K, int64_t N);
/* Host int8 timing path: quantise x, then the GEMV; bit-identical to
 * orc_gemv_semantics on the quantised x.  AVX2, nthreads OpenMP threads. */
void orc_gemv_q8_1_host(const orc_block_iq4_xs* W, const float* x, float* y, int64_t K, int64_t N, int nthreads);

/*
 * Fused producers -> Q8_1 (no counterpart in the reference's kernels; they
 * stand for the ggml ops that write a mul_mat activation).  The fp32 value
 * each produces is defined exactly (reduction order included) so that the
 * Q8_1 blocks it yields are bit-exact; the blocks themselves follow
 * orc_quantize_q8_1.
 */
float orc_exp_cw(float x);
float orc_silu(float x);
void orc_swiglu_q8_1(const float* G, const float* U, int64_t K, int64_t M, float* Y, orc_block_q8_1* out);
void orc_rms_norm_q8_1(const float* X, const float* R, float* H, const float* gamma, float eps, int64_t K,
                       int64_t M, float* Y, orc_block_q8_1* out);

void orc_gen_weights(orc_block_iq4_xs* W, int64_t n_blocks, uint64_t seed, int64_t first_block);
void orc_gen_activations(float* x, int64_t n, uint64_t seed, int outliers);

#ifdef __cplusplus
}
#endif
#endif
