/*
 * iq4xs_oracle.c -- CPU restatement of the reference IQ4_XS x Q8_1 path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker).  See iq4xs_oracle.h for what pins
 * each function.  Built with -ffp-contract=off so that every float expression
 * rounds exactly as written, like the reference's scalar code.
 */
#include "iq4xs_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* kernels/common/block_iq4_xs.h:22-24 */
const int8_t orc_kvalues_iq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                       1,    13,   25,  38,  53,  69,  89,  113};

/* kernels/common/block_iq4_xs.h:34-68 -- exact IEEE binary16 -> binary32. */
float orc_fp16_to_fp32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            /* subnormal: value = m * 2^-24; renormalise */
            int shift = 0;
            while ((m & 0x400u) == 0) {
                m <<= 1;
                ++shift;
            }
            m &= 0x3FFu;
            bits = sign | ((uint32_t)(127 - 15 + 1 - shift) << 23) | (m << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 127 - 15) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

/*
 * kernels/common/block_iq4_xs.h:71-86 and real_stock_dp4a_comparator.hip:43-62
 * (pack_half2's f32_to_f16_bits): mantissa truncated (round toward zero),
 * |x| < 2^-24 flushes to signed zero, biased exponent >= 31 (|x| >= 65536,
 * Inf, NaN) saturates to signed Inf.
 */
uint16_t orc_fp32_to_fp16_trunc(float f) {
    uint32_t x;
    memcpy(&x, &f, sizeof x);
    uint32_t sign = (x >> 16) & 0x8000u;
    int32_t e = (int32_t)((x >> 23) & 0xFFu) - 127 + 15;
    uint32_t m = (x >> 13) & 0x3FFu;
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        return (uint16_t)(sign | ((m | 0x400u) >> (1 - e)));
    }
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | ((uint32_t)e << 10) | m);
}

void orc_fp16_to_fp32_array(const uint16_t* h, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_fp16_to_fp32(h[i]);
}

void orc_fp32_to_fp16_trunc_array(const float* f, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_fp32_to_fp16_trunc(f[i]);
}

/* kernels/matmul_iq4xs/ref_cpu.cpp:28-31: 6-bit scale of sub-block ib, 0..63. */
int orc_subblock_scale(const orc_block_iq4_xs* b, int ib) {
    int lo = (b->scales_l[ib / 2] >> (4 * (ib & 1))) & 0x0F;
    int hi = (b->scales_h >> (2 * ib)) & 0x03;
    return lo | (hi << 4);
}

static uint32_t pack_half2_trunc(float lo, float hi) {
    return (uint32_t)orc_fp32_to_fp16_trunc(lo) | ((uint32_t)orc_fp32_to_fp16_trunc(hi) << 16);
}

/*
 * real_stock_dp4a_comparator.hip:230-264 -- DEVICE semantics of one Q8_1
 * block (not the host helper at :204-227, which multiplies by 1/d and sums
 * sequentially).  32 lanes hold x[0..31]; five xor-butterfly steps with
 * offsets 16,8,4,2,1 reduce amax and sum; every lane then holds the same
 * values.  d = amax/127 (true division), q = roundf(x/d), ds = trunc-half2.
 */
static void quantize_block(const float* xs, ptrdiff_t stride, orc_block_q8_1* out) {
    float amax[32], sum[32], x[32];
    for (int t = 0; t < 32; ++t) {
        x[t] = xs[t * stride];
        amax[t] = fabsf(x[t]);
        sum[t] = x[t];
    }
    for (int off = 16; off > 0; off >>= 1) {
        float na[32], ns[32];
        for (int t = 0; t < 32; ++t) {
            na[t] = fmaxf(amax[t], amax[t ^ off]);
            ns[t] = sum[t] + sum[t ^ off];
        }
        memcpy(amax, na, sizeof na);
        memcpy(sum, ns, sizeof ns);
    }
    const float a = amax[0];
    const float d = a / 127.0f;
    for (int t = 0; t < 32; ++t) {
        out->qs[t] = (a != 0.0f) ? (int8_t)roundf(x[t] / d) : (int8_t)0;
    }
    out->ds = pack_half2_trunc(d, sum[0]);
}

/* real_stock_dp4a_comparator.hip:230-273 (one row x[K] -> K/32 blocks). */
void orc_quantize_q8_1(const float* x, orc_block_q8_1* y, int64_t K) {
    const int64_t nb = K / ORC_QK8_1;
    for (int64_t ib = 0; ib < nb; ++ib) quantize_block(x + ib * ORC_QK8_1, 1, y + ib);
}

/*
 * real_stock_dp4a_comparator.hip:278-306 -- batched: column m of X quantised
 * into Y[m*nb + ib].  layout ORC_LAYOUT_KM reads X[k*M+m] (standalone API),
 * ORC_LAYOUT_MK reads X[m*K+k] (ggml src1).
 */
void orc_quantize_q8_1_batched(const float* X, orc_block_q8_1* Y, int64_t K, int64_t M, int layout) {
    const int64_t nb = K / ORC_QK8_1;
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t ib = 0; ib < nb; ++ib) {
            const int64_t k0 = ib * ORC_QK8_1;
            if (layout == ORC_LAYOUT_KM)
                quantize_block(X + k0 * M + m, (ptrdiff_t)M, Y + m * nb + ib);
            else
                quantize_block(X + m * K + k0, 1, Y + m * nb + ib);
        }
    }
}

/*
 * ---------------------------------------------------------------------------
 * Fused producers.  The reference's kernels stop at the quantiser; the op
 * that writes the activation lives in ggml (RMS_NORM + MUL before the
 * attention/FFN projections, SWIGLU before ffn_down; their cost is profiled
 * in benchmarks/profiling/BOTTLENECK-TABLE.md:24,26,30, and the model's
 * rms epsilon is 1e-6, benchmarks/environment/startup-log.txt:128).  The
 * fp32 values below are this library's definition of those ops; they must
 * be reproduced bit for bit by the device kernels, so every rounding step
 * and the reduction order are spelled out.
 * ---------------------------------------------------------------------------
 */

/*
 * exp(x): Cody & Waite range reduction (x = n ln2 + r, ln2 split into a
 * 16-significant-bit head, so n*head is exact for |n| <= 255, and a tail),
 * then the degree-7 Taylor polynomial of e^r on |r| <= ln2/2 by Horner with
 * fused multiply-adds (truncation error < 2^-27 relative), then r -> 2^n.
 * Inputs below -87 are raised to -87 (no subnormal results: the only user
 * adds the value to 1); above 88.72283935546875 the result is +inf.
 */
float orc_exp_cw(float x) {
    if (x != x) return x + x;
    if (x > 0x1.62e430p+6f) return INFINITY;
    if (x < -87.0f) x = -87.0f;
    const float n = rintf(x * 0x1.715476p+0f);
    float r = fmaf(-n, 0x1.62e400p-1f, x);
    r = fmaf(-n, 0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;
    p = fmaf(p, r, 0x1.6c16c2p-10f);
    p = fmaf(p, r, 0x1.111112p-7f);
    p = fmaf(p, r, 0x1.555556p-5f);
    p = fmaf(p, r, 0x1.555556p-3f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)n);
}

/* silu(x) = x / (1 + exp(-x)), the form ggml's SILU/SWIGLU use. */
float orc_silu(float x) { return x / (1.0f + orc_exp_cw(-x)); }

/* y = silu(g) * u, row-major [M][K]; y -> Q8_1 blocks [M][K/32]. */
void orc_swiglu_q8_1(const float* G, const float* U, int64_t K, int64_t M, float* Y, orc_block_q8_1* out) {
    const int64_t n = K * M;
    for (int64_t i = 0; i < n; ++i) {
        const float s = orc_silu(G[i]);
        Y[i] = s * U[i];
    }
    orc_quantize_q8_1(Y, out, n);
}

/*
 * RMS norm of one row h[K] (h = x + r when a residual r is given), then an
 * elementwise gain, then Q8_1:
 *   ss    = sum of (double)(h*h)            in the order below
 *   mean  = (float)(ss / K)                 (division in double)
 *   scale = 1.0f / sqrtf(mean + eps)
 *   y     = (h * scale) * gamma             (two fp32 roundings; no gamma: h*scale)
 * This is ggml's CPU rms_norm (double sum of float squares, float scale)
 * followed by its MUL.  Summation order: element k goes to accumulator
 * a = (k / 4) % 1024 (a work-group of 1024 threads reading 4-float vectors,
 * 4096 elements per sweep), each accumulator adds its elements in increasing
 * k; the 1024 accumulators reduce as sixteen 64-lane butterflies (v[l] +=
 * v[l ^ o] for o = 32, 16, 8, 4, 2, 1, lane 0 kept) and then a pairwise tree
 * over the 16 wave sums: ((w0 + w1) + (w2 + w3)) + ((w4 + w5) + (w6 + w7))
 * and so on.
 */
static double rms_sum_squares(const float* h, int64_t K) {
    enum { THREADS = 1024, WAVES = THREADS / 64 };
    double acc[THREADS];
    for (int a = 0; a < THREADS; ++a) acc[a] = 0.0;
    for (int64_t k = 0; k < K; ++k) {
        const float sq = h[k] * h[k];
        acc[(k >> 2) & (THREADS - 1)] += (double)sq;
    }
    double w[WAVES];
    for (int wv = 0; wv < WAVES; ++wv) {
        double v[64];
        for (int l = 0; l < 64; ++l) v[l] = acc[64 * wv + l];
        for (int o = 32; o > 0; o >>= 1) {
            double nv[64];
            for (int l = 0; l < 64; ++l) nv[l] = v[l] + v[l ^ o];
            memcpy(v, nv, sizeof nv);
        }
        w[wv] = v[0];
    }
    for (int n = WAVES / 2; n > 0; n >>= 1)
        for (int i = 0; i < n; ++i) w[i] = w[2 * i] + w[2 * i + 1];
    return w[0];
}

void orc_rms_norm_q8_1(const float* X, const float* R, float* H, const float* gamma, float eps, int64_t K,
                       int64_t M, float* Y, orc_block_q8_1* out) {
    for (int64_t m = 0; m < M; ++m) {
        const float* x = X + m * K;
        float* y = Y + m * K;
        /* h first lands in y (or H), so H may alias X or R */
        float* h = H ? H + m * K : y;
        for (int64_t k = 0; k < K; ++k) h[k] = R ? x[k] + R[m * K + k] : x[k];
        const double ss = rms_sum_squares(h, K);
        const float mean = (float)(ss / (double)K);
        const float scale = 1.0f / sqrtf(mean + eps);
        for (int64_t k = 0; k < K; ++k) {
            const float t = h[k] * scale;
            y[k] = gamma ? t * gamma[k] : t;
        }
        orc_quantize_q8_1(y, out + m * (K / ORC_QK8_1), K);
    }
}

/* x_hat = fp16(d) * q : the values a Q8_1 path actually multiplies. */
void orc_dequant_q8_1(const orc_block_q8_1* y, float* xhat, int64_t n_blocks) {
    for (int64_t b = 0; b < n_blocks; ++b) {
        const float d = orc_fp16_to_fp32((uint16_t)(y[b].ds & 0xFFFFu));
        for (int t = 0; t < 32; ++t) xhat[b * 32 + t] = d * (float)y[b].qs[t];
    }
}

static inline int32_t dot4_i8(uint32_t a, uint32_t b, int32_t c) {
    for (int i = 0; i < 4; ++i) c += (int32_t)(int8_t)(a >> (8 * i)) * (int32_t)(int8_t)(b >> (8 * i));
    return c;
}

static inline uint32_t load_u32(const void* p) {
    uint32_t v;
    memcpy(&v, p, 4);
    return v;
}

/*
 * real_stock_dp4a_comparator.hip:145-166 with :105-131 and :68-88 -- integer
 * part of vec_dot_iq4_xs_q8_1 for sub-block ib (iqs = 4*ib): qs word iqs+j
 * gives 4 low-nibble codes (weights 4j..4j+3, paired with q8 word j) and 4
 * high-nibble codes (weights 16+4j.., paired with q8 word j+4); the sum is
 * then multiplied by (ls - 32).  bq8_chunk points at the 8 Q8_1 blocks of the
 * super-block.
 */
int32_t orc_subblock_sumi(const orc_block_iq4_xs* bq4, const orc_block_q8_1* bq8_chunk, int ib) {
    const orc_block_q8_1* a = bq8_chunk + ib;
    int32_t sumi = 0;
    for (int j = 0; j < 4; ++j) {
        const uint32_t q4 = load_u32(bq4->qs + 16 * ib + 4 * j);
        uint32_t vx = 0, vy = 0;
        for (int i = 0; i < 4; ++i) {
            vx |= (uint32_t)(uint8_t)orc_kvalues_iq4nl[(q4 >> (8 * i)) & 0xF] << (8 * i);
            vy |= (uint32_t)(uint8_t)orc_kvalues_iq4nl[(q4 >> (8 * i + 4)) & 0xF] << (8 * i);
        }
        sumi = dot4_i8(vx, load_u32(a->qs + 4 * j), sumi);
        sumi = dot4_i8(vy, load_u32(a->qs + 4 * j + 16), sumi);
    }
    return sumi * (orc_subblock_scale(bq4, ib) - 32);
}

/* S[(m*N + n)*(K/32) + kb]: scaled int32 sum of every 32-element sub-block. */
void orc_subblock_sums(const orc_block_iq4_xs* W, const orc_block_q8_1* AQ, int32_t* S,
                       int64_t K, int64_t N, int64_t M) {
    const int64_t bpr = K / ORC_QK_K, nb = K / ORC_QK8_1;
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n)
            for (int64_t b = 0; b < bpr; ++b)
                for (int ib = 0; ib < 8; ++ib)
                    S[(m * N + n) * nb + b * 8 + ib] =
                        orc_subblock_sumi(W + n * bpr + b, AQ + m * nb + b * 8, ib);
}

/* real_stock_dp4a_comparator.hip:160-165: fp32 term of one sub-block. */
static inline float subblock_term(const orc_block_iq4_xs* bq4, const orc_block_q8_1* chunk, int ib) {
    const int32_t sumi = orc_subblock_sumi(bq4, chunk, ib);
    const float d = orc_fp16_to_fp32(bq4->d) * orc_fp16_to_fp32((uint16_t)(chunk[ib].ds & 0xFFFFu));
    return d * (float)sumi;
}

/*
 * real_stock_dp4a_comparator.hip:325-360 -- fp32 output of the reference
 * GEMV kernel, in its order: lane t (0..31) sums super-blocks t/8, t/8+4, ...
 * at sub-block t%8, then a 16,8,4,2,1 xor butterfly; lane 0 stores.
 */
void orc_gemv_semantics(const orc_block_iq4_xs* W, const orc_block_q8_1* AQ, float* y,
                        int64_t K, int64_t N) {
    const int64_t bpr = K / ORC_QK_K;
    for (int64_t r = 0; r < N; ++r) {
        float tmp[32];
        for (int t = 0; t < 32; ++t) {
            float acc = 0.0f;
            for (int64_t kbx = t / 8; kbx < bpr; kbx += 4)
                acc += subblock_term(W + r * bpr + kbx, AQ + kbx * 8, t % 8);
            tmp[t] = acc;
        }
        for (int off = 16; off > 0; off >>= 1) {
            float nt[32];
            for (int t = 0; t < 32; ++t) nt[t] = tmp[t] + tmp[t ^ off];
            memcpy(tmp, nt, sizeof nt);
        }
        y[r] = tmp[0];
    }
}

/*
 * real_stock_dp4a_comparator.hip:374-443 (tiled GEMM, same per-element order
 * as the simple kernel :446-472): acc over super-blocks, then sub-blocks.
 * AQ is [M][K/32] blocks; Y[n*M + m].
 */
void orc_gemm_semantics(const orc_block_iq4_xs* W, const orc_block_q8_1* AQ, float* Y,
                        int64_t K, int64_t N, int64_t M) {
    const int64_t bpr = K / ORC_QK_K, nb = K / ORC_QK8_1;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t m = 0; m < M; ++m) {
            float acc = 0.0f;
            for (int64_t kbx = 0; kbx < bpr; ++kbx)
                for (int ib = 0; ib < 8; ++ib)
                    acc += subblock_term(W + n * bpr + kbx, AQ + m * nb + kbx * 8, ib);
            Y[n * M + m] = acc;
        }
}

/*
 * kernels/matmul_iq4xs/ref_cpu.cpp:12-52 -- FP64 oracle GEMV:
 * dl = double(d) * double(float(ls) - 32), w = dl * kvalue, acc += w * x.
 */
static double row_dot_fp64(const orc_block_iq4_xs* row, const float* x, ptrdiff_t xstride, int64_t bpr) {
    double acc = 0.0;
    for (int64_t b = 0; b < bpr; ++b) {
        const float d = orc_fp16_to_fp32(row[b].d);
        for (int ib = 0; ib < 8; ++ib) {
            const double dl = (double)d * (double)((float)orc_subblock_scale(row + b, ib) - 32.0f);
            const uint8_t* qs = row[b].qs + ib * 16;
            const int64_t k0 = b * ORC_QK_K + ib * 32;
            for (int j = 0; j < 16; ++j) {
                const double wlo = dl * (double)orc_kvalues_iq4nl[qs[j] & 0x0F];
                const double whi = dl * (double)orc_kvalues_iq4nl[(qs[j] >> 4) & 0x0F];
                acc += wlo * (double)x[(k0 + j) * xstride];
                acc += whi * (double)x[(k0 + j + 16) * xstride];
            }
        }
    }
    return acc;
}

void orc_gemv_fp64(const orc_block_iq4_xs* W, const float* x, float* y, int64_t K, int64_t N) {
    const int64_t bpr = K / ORC_QK_K;
    for (int64_t r = 0; r < N; ++r) y[r] = (float)row_dot_fp64(W + r * bpr, x, 1, bpr);
}

/*
 * kernels/matmul_iq4xs/ref_cpu.cpp:54-106 -- FP64 oracle GEMM, X[k*M+m],
 * Y[n*M+m]; same per-element order as the GEMV.  Rows are split over
 * nthreads OpenMP threads; each element's arithmetic is unchanged, so the
 * result is identical for every thread count.
 */
void orc_gemm_fp64(const orc_block_iq4_xs* W, const float* X, float* Y, int64_t K, int64_t N,
                   int64_t M, int nthreads) {
    const int64_t bpr = K / ORC_QK_K;
    (void)nthreads;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads > 0 ? nthreads : 1)
#endif
    for (int64_t n = 0; n < N; ++n)
        for (int64_t m = 0; m < M; ++m)
            Y[n * M + m] = (float)row_dot_fp64(W + n * bpr, X + m, (ptrdiff_t)M, bpr);
}

/*
 * impl_gemv_gfx1100.hip:6-93 -- the FP64 GEMV of the
 * reference's gfx1100 kernel: the products of ref_cpu.cpp, summed as 8
 * partials per row (partial ib runs over all super-blocks b, j = 0..15, low
 * then high nibble), the partials then added in ib order.
 */
void orc_gemv_fp64_by_subblock(const orc_block_iq4_xs* W, const float* x, float* y, int64_t K, int64_t N) {
    const int64_t bpr = K / ORC_QK_K;
    for (int64_t r = 0; r < N; ++r) {
        double part[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int ib = 0; ib < 8; ++ib) {
            for (int64_t b = 0; b < bpr; ++b) {
                const orc_block_iq4_xs* blk = W + r * bpr + b;
                const float d = orc_fp16_to_fp32(blk->d);
                const double dl = (double)d * (double)((float)orc_subblock_scale(blk, ib) - 32.0f);
                const float* xs = x + b * ORC_QK_K + ib * 32;
                for (int j = 0; j < 16; ++j) {
                    const uint8_t q = blk->qs[ib * 16 + j];
                    const double wl = dl * (double)orc_kvalues_iq4nl[q & 15];
                    const double wh = dl * (double)orc_kvalues_iq4nl[q >> 4];
                    part[ib] += wl * (double)xs[j];
                    part[ib] += wh * (double)xs[j + 16];
                }
            }
        }
        double acc = 0.0;
        for (int ib = 0; ib < 8; ++ib) acc += part[ib];
        y[r] = (float)acc;
    }
}

/*
 * Host int8 path (real_stock_dp4a_comparator.hip:230-264 quantiser, :145-166
 * sub-block dot, :325-360 GEMV order), for timing the CPU against the GPU on
 * the same integer semantics: x is quantised to Q8_1, each sub-block's codes
 * are decoded with a byte shuffle and dotted against the Q8_1 codes in 16-bit
 * lanes (exact: |kv * q| <= 16129), eight sub-block sums are reduced
 * together, and the fp32 terms (fp16(d_w) * fp16(d_x)) * float(sumi * (ls-32))
 * are added in orc_gemv_semantics' lane order -- so y is bit-identical to it.
 * Rows are split over nthreads OpenMP threads.
 */
__attribute__((target("avx2"))) static inline __m256i dot_subblock_avx2(const uint8_t* qs16, const int8_t* a32,
                                                                         __m128i table) {
    const __m128i q = _mm_loadu_si128((const __m128i*)qs16);
    const __m128i m4 = _mm_set1_epi8(0x0F);
    const __m128i wl = _mm_shuffle_epi8(table, _mm_and_si128(q, m4));
    const __m128i wh = _mm_shuffle_epi8(table, _mm_and_si128(_mm_srli_epi16(q, 4), m4));
    const __m128i al = _mm_loadu_si128((const __m128i*)a32);
    const __m128i ah = _mm_loadu_si128((const __m128i*)(a32 + 16));
    const __m256i pl = _mm256_madd_epi16(_mm256_cvtepi8_epi16(wl), _mm256_cvtepi8_epi16(al));
    const __m256i ph = _mm256_madd_epi16(_mm256_cvtepi8_epi16(wh), _mm256_cvtepi8_epi16(ah));
    return _mm256_add_epi32(pl, ph);
}

__attribute__((target("avx2"))) void orc_gemv_q8_1_host(const orc_block_iq4_xs* W, const float* x, float* y,
                                                        int64_t K, int64_t N, int nthreads) {
    const int64_t bpr = K / ORC_QK_K, nb = K / ORC_QK8_1;
    orc_block_q8_1* AQ = (orc_block_q8_1*)malloc((size_t)nb * sizeof(orc_block_q8_1));
    float* dx = (float*)malloc((size_t)nb * sizeof(float));
    int8_t* codes = (int8_t*)malloc((size_t)K);
    orc_quantize_q8_1(x, AQ, K);
    for (int64_t i = 0; i < nb; ++i) {
        dx[i] = orc_fp16_to_fp32((uint16_t)(AQ[i].ds & 0xFFFFu));
        memcpy(codes + i * ORC_QK8_1, AQ[i].qs, ORC_QK8_1);
    }
    const __m128i table = _mm_loadu_si128((const __m128i*)orc_kvalues_iq4nl);
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1)
    {
        float* T = (float*)malloc((size_t)nb * sizeof(float));
#pragma omp for schedule(static)
        for (int64_t r = 0; r < N; ++r) {
            for (int64_t b = 0; b < bpr; ++b) {
                const orc_block_iq4_xs* blk = W + r * bpr + b;
                const int8_t* a = codes + b * ORC_QK_K;
                __m256i v[8];
                for (int ib = 0; ib < 8; ++ib) v[ib] = dot_subblock_avx2(blk->qs + 16 * ib, a + 32 * ib, table);
                const __m256i h0 = _mm256_hadd_epi32(_mm256_hadd_epi32(v[0], v[1]), _mm256_hadd_epi32(v[2], v[3]));
                const __m256i h1 = _mm256_hadd_epi32(_mm256_hadd_epi32(v[4], v[5]), _mm256_hadd_epi32(v[6], v[7]));
                const __m256i s8 = _mm256_add_epi32(_mm256_permute2x128_si256(h0, h1, 0x20),
                                                    _mm256_permute2x128_si256(h0, h1, 0x31));
                int32_t ls[8];
                for (int ib = 0; ib < 8; ++ib) ls[ib] = orc_subblock_scale(blk, ib) - 32;
                const __m256i sumi = _mm256_mullo_epi32(s8, _mm256_loadu_si256((const __m256i*)ls));
                const __m256 d = _mm256_mul_ps(_mm256_set1_ps(orc_fp16_to_fp32(blk->d)), _mm256_loadu_ps(dx + 8 * b));
                _mm256_storeu_ps(T + 8 * b, _mm256_mul_ps(d, _mm256_cvtepi32_ps(sumi)));
            }
            float tmp[32];
            for (int t = 0; t < 32; ++t) {
                float acc = 0.0f;
                for (int64_t kbx = t / 8; kbx < bpr; kbx += 4) acc += T[kbx * 8 + t % 8];
                tmp[t] = acc;
            }
            for (int off = 16; off > 0; off >>= 1) {
                float nt[32];
                for (int t = 0; t < 32; ++t) nt[t] = tmp[t] + tmp[t ^ off];
                memcpy(tmp, nt, sizeof nt);
            }
            y[r] = tmp[0];
        }
        free(T);
    }
    free(AQ);
    free(dx);
    free(codes);
}

/* kernels/matmul_iq4xs/ref_cpu.cpp:108-139 -- fp32 dequantisation. */
void orc_dequant(const orc_block_iq4_xs* W, float* out, int64_t K, int64_t N) {
    const int64_t bpr = K / ORC_QK_K;
    for (int64_t r = 0; r < N; ++r)
        for (int64_t b = 0; b < bpr; ++b) {
            const orc_block_iq4_xs* blk = W + r * bpr + b;
            const float d = orc_fp16_to_fp32(blk->d);
            for (int ib = 0; ib < 8; ++ib) {
                const float dl = d * ((float)orc_subblock_scale(blk, ib) - 32.0f);
                float* o = out + r * K + b * ORC_QK_K + ib * 32;
                for (int j = 0; j < 16; ++j) {
                    o[j] = dl * (float)orc_kvalues_iq4nl[blk->qs[ib * 16 + j] & 0x0F];
                    o[j + 16] = dl * (float)orc_kvalues_iq4nl[(blk->qs[ib * 16 + j] >> 4) & 0x0F];
                }
            }
        }
}

/* ------------------------------------------------------------------------ */
/* Seeded synthetic inputs.  Counter-based, so any block/element can be made
 * independently (the product library's device generator makes the same
 * weights bit for bit).  splitmix64 finaliser: Steele, Lea, Flood, "Fast
 * splittable pseudorandom number generators", OOPSLA 2014.                   */

static inline uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline uint64_t draw(uint64_t seed, uint64_t stream, uint64_t ctr) {
    return mix64(mix64(seed ^ (stream * 0xD1B54A32D192ED03ull)) ^ ctr);
}

/*
 * Weights per the synthetic recipe: fp16 d ~ U(0.005, 0.02) (stored with the
 * reference's truncating encoder, kernels/common/matmul_test_util.h:58),
 * eight 6-bit sub-block scales uniform in 0..63, codebook indices uniform
 * over the 16 entries.  Block g (global index first_block + i) uses draws
 * 18g .. 18g+17 of stream 1.
 */
void orc_gen_weights(orc_block_iq4_xs* W, int64_t n_blocks, uint64_t seed, int64_t first_block) {
    for (int64_t i = 0; i < n_blocks; ++i) {
        const uint64_t g = (uint64_t)(first_block + i);
        orc_block_iq4_xs* b = W + i;
        const uint64_t r0 = draw(seed, 1, g * 18 + 0);
        const float t = (float)(uint32_t)(r0 >> 40) * 8.94069671630859375e-10f; /* 0.015 / 2^24 */
        b->d = orc_fp32_to_fp16_trunc(t + 0.005f);
        const uint64_t r1 = draw(seed, 1, g * 18 + 1);
        uint16_t sh = 0;
        for (int ib = 0; ib < 8; ++ib) {
            const unsigned ls = (unsigned)(r1 >> (6 * ib)) & 63u;
            if ((ib & 1) == 0)
                b->scales_l[ib / 2] = (uint8_t)(ls & 0xF);
            else
                b->scales_l[ib / 2] |= (uint8_t)((ls & 0xF) << 4);
            sh |= (uint16_t)((ls >> 4) << (2 * ib));
        }
        b->scales_h = sh;
        for (int w = 0; w < 16; ++w) {
            const uint64_t r = draw(seed, 1, g * 18 + 2 + (uint64_t)w);
            memcpy(b->qs + 8 * w, &r, 8);
        }
    }
}

/*
 * Activations: x_i ~ N(0,1) by Box-Muller on draws i of streams 2 and 3;
 * with outliers != 0, element i is scaled x20 when draw i of stream 4 is
 * 0 mod 100 (1 % of positions, seeded).
 */
void orc_gen_activations(float* x, int64_t n, uint64_t seed, int outliers) {
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < n; ++i) {
        const double u1 = (double)((draw(seed, 2, (uint64_t)i) >> 11) + 1) * 0x1.0p-53;
        const double u2 = (double)(draw(seed, 3, (uint64_t)i) >> 11) * 0x1.0p-53;
        float v = (float)(sqrt(-2.0 * log(u1)) * cos(two_pi * u2));
        if (outliers && draw(seed, 4, (uint64_t)i) % 100 == 0) v *= 20.0f;
        x[i] = v;
    }
}
