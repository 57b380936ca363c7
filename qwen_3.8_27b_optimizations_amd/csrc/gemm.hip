// gemm.hip -- IQ4_XS x Q8_1 prefill GEMM on gfx950 matrix cores.
//
// Semantics: the reference GEMM (real_stock_dp4a_comparator.hip:374-443):
//   Y[n,m] = sum_kb fp16(W.d) * fp16(ds[m,kb].d) * (float)(sumi[n,m,kb] * (ls-32))
// where sumi is the exact int32 dot of a 32-weight sub-block with the
// matching Q8_1 block.
//
// Default kernel: gemm_f16_kernel (128x128 tile, 8 waves, two LDS stages),
// which runs the integer products on v_mfma_f32_32x32x16_f16 -- codebook
// values and Q8_1 codes are exact in fp16 and a sub-block's 32-term sum is an
// integer below 2^24, so the MFMA returns sumi exactly, as a float -- and
// leaves one FMA per output and sub-block for the epilogue.  Its design notes
// are with the kernel below.
//
// The int8 kernels below it, gemm_iq4xs_db_kernel (128x128 tile, 16 waves,
// double-buffered LDS) and gemm_iq4xs_mfma_kernel (64x64 tile, 4 waves,
// three per CU), run the products on v_mfma_i32_32x32x32_i8 and need a
// convert as well as the FMA per output and sub-block; they serve K beyond
// the fp16 kernel's 32-bit offsets and stay selectable for comparison
// (IQ4XS_GEMM_KIND = 0 / 1 / -1).  Notes on them:
//
// Both are VALU-issue bound.  Every output needs its own scale per sub-block,
// d_w[n] * d_x[m], so the epilogue costs VALU work per output and sub-block
// against 1/16 of a 32x32x32 int8 MFMA per lane.  The scale tile is formed by
// a bf16 MFMA from exact hi/lo splits of the two scales (scale_outer2), which
// leaves 2 VALU ops per output and sub-block (convert, fused add) instead of
// 3 and removes the per-lane row-scale LDS reads: in the 128x128 kernel 8-20 %
// faster than the multiply version.  The 64x64 kernel measured 3-5 % slower
// with it than with the multiplies, but uses it too: both kernels then give
// bit-identical outputs, so the tile choice (which depends on the shape, and
// for grouped launches on the group) never changes a result.
//
// Measured on the 128x128 kernel with the multiply epilogue: removing the
// int8 MFMA changed little and every VALU op removed showed up in full; an
// f32 MFMA (32x32x2) for the same outer product cost as much as the 16
// multiplies; keeping (ls - 32) as int8 with d_w applied once per super-block
// (exact int32 sumi*(ls-32)) was 4-8 % slower.
//
// Non-finite scales (an fp16 d of Inf/NaN) give NaN in the int8 kernels where
// the reference's product would give +-Inf: the hi/lo split of an infinite
// scale is Inf + NaN.  The fp16 kernel keeps the reference's +-Inf: no
// infinite half of one scale meets a zero half of the other.
//
// MI355X mapping (64x64 int8 kernel).  A workgroup (4 waves) owns a 64-row x
// 64-token output tile and walks K one 256-weight super-block at a time:
//   1. the 64 weight rows' super-blocks are decoded (v_perm codebook lookup,
//      decode_codes_x)
//      straight into int8 LDS tiles, the per-sub-block weight scales
//      d*(ls-32) into a table of exact bf16 hi/lo pairs (bf16_pair);
//   2. the 64 tokens' Q8_1 codes are copied to LDS, their d into a pair table;
//   3. each wave issues one v_mfma_i32_32x32x32_i8 per 32-wide sub-block --
//      K=32 is exactly one sub-block, so the MFMA result IS the reference's
//      int32 sumi -- and folds it into fp32 accumulators with the scale tile
//      of scale_outer2.
// LDS rows are 256 bytes; the 16-byte chunk index is XORed with (row & 15)
// so the 32 lanes that read one k-chunk of 32 different rows hit 16
// distinct chunk positions (no bank conflicts from the 256-byte row stride).
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <functional>
#include <map>
#include <mutex>
#include <queue>
#include <tuple>
#include <vector>

#include "iq4xs_device.h"
#include "iq4xs_internal.h"

namespace iq4xs {

constexpr int GEMM_BN = 64;  // weight rows per workgroup
constexpr int GEMM_BM = 64;  // tokens per workgroup

__device__ inline int lds_swz(int row, int chunk) { return row * 256 + ((chunk ^ (row & 15)) << 4); }

// MFMA 32x32x32 i8 operand / result layout used throughout:
//   A: lane l supplies row (l & 31), k = 16*(l >> 5) .. +15
//   B: lane l supplies column (l & 31), k = 16*(l >> 5) .. +15
//   C: element e of lane l is row 8*(e>>2) + 4*(l>>5) + (e&3), column (l & 31)
__device__ inline int mfma_c_row(int e, int lane) { return 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3); }

// Up to GEMV_GROUP_MAX matrices with the same K and the same quantised
// activations, run by one launch: the N-tiles of matrix i are blockIdx.x in
// [tile_end[i-1], tile_end[i]).  Single-matrix launches use entry 0 only.
struct GemmGroup {
    const uint8_t* W[GEMV_GROUP_MAX];
    float* Y[GEMV_GROUP_MAX];
    int64_t N[GEMV_GROUP_MAX];
    int64_t ldy_m[GEMV_GROUP_MAX];
    int tile_end[GEMV_GROUP_MAX];
};

// This workgroup's matrix and its first N-tile, by scalar selects on the
// by-value descriptor (no dynamic index into the argument block).
template <bool kGroup>
__device__ inline void gemm_select(const GemmGroup& grp, const uint8_t*& W, float*& Y, int64_t& N, int64_t& ldy_m,
                                   int& tile0) {
    W = grp.W[0];
    Y = grp.Y[0];
    N = grp.N[0];
    ldy_m = grp.ldy_m[0];
    tile0 = 0;
    if (kGroup) {
        int g = 0;
#pragma unroll
        for (int i = 0; i + 1 < GEMV_GROUP_MAX; ++i) g += (int)blockIdx.x >= grp.tile_end[i] ? 1 : 0;
#pragma unroll
        for (int i = 1; i < GEMV_GROUP_MAX; ++i) {
            if (g == i) {
                W = grp.W[i];
                Y = grp.Y[i];
                N = grp.N[i];
                ldy_m = grp.ldy_m[i];
                tile0 = grp.tile_end[i - 1];
            }
        }
    }
}

typedef short v4s __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

// x = hi + lo exactly, as two bf16 halves (hi | lo << 16), for any finite x
// with at most 16 significant bits: d_w * (ls - 32) (11 + 5 bits) and the
// fp16 d_x both qualify.  hi keeps the top 8 bits, lo the rest.
__device__ inline uint32_t bf16_pair(float x) {
    const uint32_t hb = __builtin_bit_cast(uint32_t, x) & 0xFFFF0000u;
    const float lo = x - __builtin_bit_cast(float, hb);
    return (hb >> 16) | (__builtin_bit_cast(uint32_t, lo) & 0xFFFF0000u);
}

// Scale products d_w[row] * d_x[col] of every element of the 32x32 tiles of
// two sub-blocks s, s+1, in the int8 MFMA's C layout, from two
// v_mfma_f32_32x32x8_bf16.  pa holds the bf16 pairs of this lane's row scale
// for s (low dword) and s+1 (high dword); pb0 / pb1 those of its column's.
// Lane half h supplies k = 4h..4h+3: A = (w_hi, w_lo) of s, then of s+1; B =
// x_hi (h = 0) or x_lo (h = 1) of s twice, then two zeros (for s; the other
// way round for s+1), the copy picked by the per-lane selector bsel.  The four
// nonzero products hi*hi, lo*hi, hi*lo, lo*lo are exact in fp32, so each tile
// holds d_w * d_x to within fp32 rounding of their sum.  This replaces 16
// multiplies and 16 row-scale LDS reads per lane and sub-block at one v_perm.
__device__ inline void scale_outer2(v2u pa, uint32_t pb0, uint32_t pb1, uint32_t bsel, v16f& sc0, v16f& sc1) {
    const v2u b0 = {__builtin_amdgcn_perm(pb0, pb0, bsel), 0u};
    const v2u b1 = {0u, __builtin_amdgcn_perm(pb1, pb1, bsel)};
    sc0 = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(__builtin_bit_cast(v4s, pa), __builtin_bit_cast(v4s, b0), v16f{}, 0,
                                                   0, 0);
    sc1 = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(__builtin_bit_cast(v4s, pa), __builtin_bit_cast(v4s, b1), v16f{}, 0,
                                                   0, 0);
}

template <bool kDebug, bool kGroup>
__global__ __launch_bounds__(256) void gemm_iq4xs_mfma_kernel(const GemmGroup grp, const int8_t* __restrict__ aqs,
                                                              const uint32_t* __restrict__ ads, int64_t K, int64_t M,
                                                              int64_t ldy_n, int32_t* __restrict__ dbg) {
    __shared__ __attribute__((aligned(16))) int8_t sW[GEMM_BN * 256];
    __shared__ __attribute__((aligned(16))) int8_t sX[GEMM_BM * 256];
    __shared__ __attribute__((aligned(16))) uint32_t sA[4][GEMM_BN][2];  // bf16 pairs of d_w * (ls - 32), sub-block pairs
    __shared__ __attribute__((aligned(16))) uint32_t sB[8][GEMM_BM];     // bf16 pairs of d_x
    __shared__ int sL[kDebug ? 8 : 1][GEMM_BN];  // ls - 32, only for the debug export

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wn = wave & 1, wm = wave >> 1;
    const uint8_t* W;
    float* Y;
    int64_t N, ldy_m;
    int tile0;
    gemm_select<kGroup>(grp, W, Y, N, ldy_m, tile0);
    const int64_t n0 = (int64_t)((int)blockIdx.x - tile0) * GEMM_BN;
    const int64_t m0 = (int64_t)blockIdx.y * GEMM_BM;
    const int64_t bpr = K / QK_K, nb = K / QK8_1, row_bytes = bpr * BLOCK_BYTES;

    float acc[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.0f;

    // This thread's share of a super-block's global loads, held in registers:
    // the next super-block is in flight during the current MFMA phase (a lone
    // workgroup on a CU, as for k/v-sized grids, would otherwise wait one DRAM
    // round trip per super-block).  Rows / tokens past the end are clamped.
    struct Pref64 {
        uint2 h[2];
        v4i w[2];
        v4i x[4];
        uint32_t ds[2];
    };
    auto load = [&](Pref64& g, int64_t kb) {
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const int p = tid + 256 * it;
            const int r = p >> 3, s = p & 7;
            const int64_t n = (n0 + r < N) ? n0 + r : N - 1;
            const uint8_t* blk = W + n * row_bytes + kb * BLOCK_BYTES;
            g.h[it] = *reinterpret_cast<const uint2*>(blk);
            g.w[it] = *reinterpret_cast<const v4i_a8*>(blk + 8 + 16 * s);
        }
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int p = tid + 256 * it;
            const int r = p >> 4, c = p & 15;
            const int64_t m = (m0 + r < M) ? m0 + r : M - 1;
            g.x[it] = *reinterpret_cast<const v4i*>(aqs + m * K + kb * QK_K + 16 * c);
        }
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const int p = tid + 256 * it;
            const int r = p >> 3, s = p & 7;
            const int64_t m = (m0 + r < M) ? m0 + r : M - 1;
            g.ds[it] = ads[m * nb + kb * 8 + s];
        }
    };
    Pref64 g;
    load(g, 0);

    for (int64_t kb = 0; kb < bpr; ++kb) {
        __syncthreads();
        // 1. weights: 64 rows x 8 sub-blocks, two (row, sub-block) pairs per thread
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const int p = tid + 256 * it;
            const int r = p >> 3, s = p & 7;
            const uint2 h = g.h[it];
            const v4i w = g.w[it];
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) decode_codes_x((uint32_t)w[j], lo[j], hi[j]);
            *reinterpret_cast<v4i*>(sW + lds_swz(r, 2 * s)) = v4i{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3]};
            *reinterpret_cast<v4i*>(sW + lds_swz(r, 2 * s + 1)) = v4i{(int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
            sA[s >> 1][r][s & 1] = bf16_pair(half_bits_to_float(h.x & 0xFFFFu) * (float)(subblock_ls(h.x, h.y, s) - 32));
            if (kDebug) sL[s][r] = subblock_ls(h.x, h.y, s) - 32;
        }
        // 2. activations: 64 tokens x 16 chunks of 16 codes, four per thread
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int p = tid + 256 * it;
            const int r = p >> 4, c = p & 15;
            *reinterpret_cast<v4i*>(sX + lds_swz(r, c)) = g.x[it];
        }
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const int p = tid + 256 * it;
            const int r = p >> 3, s = p & 7;
            sB[s][r] = bf16_pair(half_bits_to_float(g.ds[it] & 0xFFFFu));
        }
        __syncthreads();
        if (kb + 1 < bpr) load(g, kb + 1);  // in flight during the MFMA phase

        // 3. one int8 MFMA per sub-block; the scale tiles of two sub-blocks
        //    from two bf16 MFMAs (scale_outer2), exactly as in the 128x128
        //    kernel, so that both kernels give bit-identical outputs and the
        //    tile choice never changes a result
        const int ra = 32 * wn + (lane & 31);
        const int rb = 32 * wm + (lane & 31);
        const uint32_t bsel = (lane >> 5) ? 0x03020302u : 0x01000100u;
#pragma unroll 1
        for (int s = 0; s < 8; s += 2) {
            v16f sc[2];
            scale_outer2(*reinterpret_cast<const v2u*>(&sA[s >> 1][ra][0]), sB[s][rb], sB[s + 1][rb], bsel, sc[0], sc[1]);
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int ch = 2 * (s + u) + (lane >> 5);
                const v4i a = *reinterpret_cast<const v4i*>(sW + lds_swz(ra, ch));
                const v4i b = *reinterpret_cast<const v4i*>(sX + lds_swz(rb, ch));
                const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, v16i{}, 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int i = 32 * wn + mfma_c_row(e, lane);
                    acc[e] += sc[u][e] * (float)c[e];
                    if (kDebug) {
                        const int64_t n = n0 + i, m = m0 + rb;
                        if (n < N && m < M) dbg[(m * N + n) * nb + kb * 8 + s + u] = c[e] * sL[s + u][i];
                    }
                }
            }
        }
    }

    const int64_t m = m0 + 32 * wm + (lane & 31);
    if (m < M) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int64_t n = n0 + 32 * wn + mfma_c_row(e, lane);
            if (n < N) Y[m * ldy_m + n * ldy_n] = acc[e];
        }
    }
}

// ---------------------------------------------------------------- 128 x 128 double-buffered kernel
// 16 waves own a 128-row x 128-token tile; wave w computes the 32x32 block at
// rows 32*(w&3), tokens 32*(w>>2) (one MFMA per 32-wide sub-block).  LDS holds
// two stages; while the waves run the MFMAs and the scale epilogue of
// super-block kb from one stage, the global loads of super-block kb+1 are in
// flight, and they are decoded into the other stage afterwards: one barrier
// per super-block.  Rows are padded to 272 bytes instead of swizzled: the 16
// lanes of a ds_read_b128 phase still hit 16 distinct 16-byte bank groups
// (272*r mod 256 = 16*r), and the address of sub-block s is a constant
// offset from sub-block 0 (no per-sub-block address arithmetic).
constexpr int G2_BN = 128, G2_BM = 128, G2_THREADS = 1024;
constexpr int G2_ROW = 272;                                  // padded LDS row (256 codes + 16)
// Stage layout: the two scale tables first, then the code tiles, so that every
// read of the MFMA phase is a 16-bit immediate offset from the stage base.
constexpr int G2_W_BYTES = G2_BN * G2_ROW, G2_X_BYTES = G2_BM * G2_ROW;
constexpr int G2_SA_OFF = 0;                                 // uint32 [4][128][2]: bf16 pairs of d_w * (ls - 32)
constexpr int G2_SB_OFF = G2_SA_OFF + 8 * G2_BN * 4;        // uint32 [8][128]: bf16 pairs of d_x
constexpr int G2_W_OFF = G2_SB_OFF + 8 * G2_BM * 4;         // int8 [128][272] weight codes
constexpr int G2_X_OFF = G2_W_OFF + G2_W_BYTES;             // int8 [128][272] token codes
constexpr int G2_SL_OFF = G2_X_OFF + G2_X_BYTES;            // int8  [8][128] (debug only)
constexpr int G2_STAGE = G2_SL_OFF;                          // bytes per stage without the debug table
static_assert(G2_X_OFF + 7 * 32 + 16 < 65536, "MFMA-phase LDS immediate offsets fit 16 bits");
constexpr int G2_STAGE_DBG = G2_SL_OFF + 8 * G2_BN;

struct GemmPref {
    v4i wq;
    v2u wh;
    v4i x[2];
    uint32_t ds;
};

template <bool kDebug, bool kGroup>
__global__ __launch_bounds__(G2_THREADS) void gemm_iq4xs_db_kernel(const GemmGroup grp, const int8_t* __restrict__ aqs,
                                                                   const uint32_t* __restrict__ ads, int64_t K,
                                                                   int64_t M, int64_t ldy_n,
                                                                   int32_t* __restrict__ dbg) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr int kStage = kDebug ? G2_STAGE_DBG : G2_STAGE;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wn = wave & 3, wm = wave >> 2;
    const uint8_t* W;
    float* Y;
    int64_t N, ldy_m;
    int tile0;
    gemm_select<kGroup>(grp, W, Y, N, ldy_m, tile0);
    const int64_t n0 = (int64_t)((int)blockIdx.x - tile0) * G2_BN;
    const int64_t m0 = (int64_t)blockIdx.y * G2_BM;
    const int64_t bpr = K / QK_K, nb = K / QK8_1, row_bytes = bpr * BLOCK_BYTES;

    // this thread's share of a super-block's loads (rows / tokens past the end
    // are clamped to the last one; their results are never stored).  Each is a
    // 32-bit lane offset from a workgroup-uniform base (the launcher bounds the
    // tile's span below 2^32 bytes), which keeps the pointers out of VGPRs.
    const int wr = tid >> 3, wsb = tid & 7;  // weight row, sub-block
    const uint8_t* wbase = W + n0 * row_bytes;
    const uint32_t woff = (uint32_t)(((n0 + wr < N) ? wr : N - 1 - n0) * row_bytes);
    int xr[2], xc[2];
    uint32_t xoff[2];
    const int8_t* xbase = aqs + m0 * K;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int p = tid + G2_THREADS * it;
        xr[it] = p >> 4;
        xc[it] = p & 15;
        xoff[it] = (uint32_t)(((m0 + xr[it] < M) ? xr[it] : M - 1 - m0) * K + 16 * xc[it]);
    }
    const int dr = tid >> 3, ds_s = tid & 7;  // token, sub-block of the d word
    const uint32_t* dbase = ads + m0 * nb;
    const uint32_t doff = (uint32_t)(((m0 + dr < M) ? dr : M - 1 - m0) * nb + ds_s);

    auto load = [&](GemmPref& g, int64_t kb) {
        const uint8_t* wk = wbase + kb * BLOCK_BYTES;
        g.wh = *reinterpret_cast<const v2u*>(wk + woff);
        g.wq = *reinterpret_cast<const v4i_a8*>(wk + woff + 8 + 16 * wsb);
        const int8_t* xk = xbase + kb * QK_K;
#pragma unroll
        for (int it = 0; it < 2; ++it) g.x[it] = *reinterpret_cast<const v4i*>(xk + xoff[it]);
        g.ds = (dbase + kb * 8)[doff];
    };
    auto store = [&](const GemmPref& g, int stage) {
        uint8_t* base = lds + stage * kStage;
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) decode_codes_x((uint32_t)g.wq[j], lo[j], hi[j]);
        int8_t* wdst = reinterpret_cast<int8_t*>(base + G2_W_OFF) + wr * G2_ROW + 32 * wsb;
        *reinterpret_cast<v4i*>(wdst) = v4i{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3]};
        *reinterpret_cast<v4i*>(wdst + 16) = v4i{(int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        const int ls = subblock_ls(g.wh.x, g.wh.y, wsb) - 32;
        reinterpret_cast<uint32_t*>(base + G2_SA_OFF)[((wsb >> 1) * G2_BN + wr) * 2 + (wsb & 1)] =
            bf16_pair(half_bits_to_float(g.wh.x & 0xFFFFu) * (float)ls);
        if (kDebug) reinterpret_cast<int8_t*>(base + G2_SL_OFF)[wsb * G2_BN + wr] = (int8_t)ls;
#pragma unroll
        for (int it = 0; it < 2; ++it)
            *reinterpret_cast<v4i*>(base + G2_X_OFF + xr[it] * G2_ROW + 16 * xc[it]) = g.x[it];
        reinterpret_cast<uint32_t*>(base + G2_SB_OFF)[ds_s * G2_BM + dr] = bf16_pair(half_bits_to_float(g.ds & 0xFFFFu));
    };

    float acc[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
    const int ra = 32 * wn + (lane & 31);
    const int rb = 32 * wm + (lane & 31);
    const int half = lane >> 5;  // k = 16*half .. +15 of each 32-wide sub-block
    const uint32_t bsel = half ? 0x03020302u : 0x01000100u;  // d_x lo (high half) or hi (low half), twice

    GemmPref g;
    load(g, 0);
    store(g, 0);
    __syncthreads();
    for (int64_t kb = 0; kb < bpr; ++kb) {
        const int cur = (int)(kb & 1);
        const bool more = kb + 1 < bpr;
        if (more) load(g, kb + 1);  // in flight during the MFMA phase
        const uint8_t* base = lds + cur * kStage;
        const int8_t* pa = reinterpret_cast<const int8_t*>(base + G2_W_OFF) + ra * G2_ROW + 16 * half;
        const int8_t* pb = reinterpret_cast<const int8_t*>(base + G2_X_OFF) + rb * G2_ROW + 16 * half;
        // row-scale pairs of sub-blocks 2t, 2t+1 are adjacent dwords: the table
        // is [4][128][2] (sub-block pair, row, member)
        const v2u* pA = reinterpret_cast<const v2u*>(base + G2_SA_OFF) + ra;
        const uint32_t* pB = reinterpret_cast<const uint32_t*>(base + G2_SB_OFF) + rb;
#pragma unroll 2
        for (int s = 0; s < 8; s += 2) {
            v16f sc[2];
            scale_outer2(pA[(s >> 1) * G2_BN], pB[s * G2_BM], pB[(s + 1) * G2_BM], bsel, sc[0], sc[1]);
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const v4i a = *reinterpret_cast<const v4i*>(pa + 32 * (s + u));
                const v4i b = *reinterpret_cast<const v4i*>(pb + 32 * (s + u));
                const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, v16i{}, 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    acc[e] += sc[u][e] * (float)c[e];
                    if (kDebug) {
                        const int i = 32 * wn + mfma_c_row(e, lane);
                        const int8_t* sL = reinterpret_cast<const int8_t*>(base + G2_SL_OFF);
                        const int64_t m = m0 + rb;
                        if (m < M && n0 + i < N)
                            dbg[(m * N + n0 + i) * nb + kb * 8 + s + u] = c[e] * (int)sL[(s + u) * G2_BN + i];
                    }
                }
            }
        }
        if (more) store(g, cur ^ 1);
        __syncthreads();
    }

    const int64_t m = m0 + rb;
    if (m < M) {
        float* yrow = Y + m * ldy_m;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int64_t n = n0 + 32 * wn + mfma_c_row(e, lane);
            if (n < N) yrow[n * ldy_n] = acc[e];
        }
    }
}

// ---------------------------------------------------------------- fp16 matrix-core kernel
// The IQ4_XS codebook values (-127..113) and the Q8_1 codes (-127..127) are
// exact in fp16, and every partial sum of a 32-term dot of them is an integer
// below 2^24, so two v_mfma_f32_32x32x16_f16 return the reference's int32 sumi
// of a sub-block exactly, already as a float.  The epilogue is then one FMA
// per output and sub-block, acc += sc * S, where the int8 MFMA path needs a
// convert as well.  The scale tile sc = d_x * (d_w * (ls - 32)) comes from a
// v_mfma_f32_32x32x16_bf16 on exact bf16 hi/lo halves of both factors.
//
// Workgroup: 8 waves, a 128-row x 128-token tile.  Wave w owns weight rows
// 32 * (w & 3) .. + 31 against all 128 tokens (four 32x32 blocks) and the
// sub-blocks 4 * (w >> 2) .. + 3 of every super-block; the two waves of a row
// group share a SIMD and add their partial sums at the end (a fixed order,
// whatever the grid).  The MFMA's A operand is the tokens, B the weights, so a
// lane's 16 accumulators are one weight row (its own) against 16 tokens.
//   * Weights: each lane loads its row's header and the 8 qs bytes its MFMA
//     half needs from each of its 4 sub-blocks straight into registers, two
//     super-blocks ahead of use; a qs byte becomes its fp16 code pair through
//     a 256-word table in LDS (one SDWA shift for the address, one ds_read).
//     The lane halves take the high and low bf16 half of the row's scale.
//   * Tokens: the workspace's fp16 code pairs (word p = elements p, p + 16 of a
//     block), copied by direct-to-LDS loads (global_load_lds_dwordx4, no
//     VGPRs), two stages of a super-block each.  A token row is 512 bytes; its
//     16-byte chunk c sits at c ^ (row & 15), so the 32 lanes of a fragment
//     read hit distinct bank groups.  Word p of a block pairs elements p and
//     p + 16, which is exactly the k order of the weight fragment: lane half h
//     of MFMA u takes qs bytes 8h + 4u .. + 3, low and high nibble of each.
//   * Token scales: bf16 hi/lo pairs of d_x, [token][sub-block], per stage,
//     in two copies: lane half 1's has 0 for a non-finite d_x (see decode).
// Each wave runs its 16 (sub-block, token block) steps of a super-block as a
// software pipeline: step t issues its three MFMAs, each followed by the LDS
// read that refills its A operand for step t + 1 and by a share of the VALU
// work (the FMAs of step t - 1, a third of the next sub-block's decode).
// Measured on gfx950: a wave's VALU ops issue at about half rate while an
// MFMA runs, so this design is bound by VALU issue (FMA, decode) plus half
// the MFMA time; the time per step follows that sum.
// Results are bit-identical for any grid: a row's arithmetic depends on K only.
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// s_waitcnt vmcnt(5) (expcnt and lgkmcnt left at their maxima), gfx9 encoding
constexpr int kVmcnt5 = 5 | (0x7 << 4) | (0xF << 8);

constexpr int H_BN = 128, H_BM = 128, H_THREADS = 512;
constexpr int H_ROW = 512;                           // LDS bytes per token row of a super-block
constexpr int H_T_OFF = H_BM * H_ROW;                // token scale pairs, uint32 [2][128][8]
constexpr int H_T_COPY = H_BM * 8 * 4;               // copy h of them feeds lane half h
constexpr int H_STAGE = H_T_OFF + 2 * H_T_COPY;      // 72 KB
constexpr int H_LUT = 1024;                          // the code pair table
// The same stage layout for a tile of at most TOK tokens: half-height tiles
// (64 rows, 4 waves, at most 64 tokens) use TOK = 64, so that two of them
// fit a CU's LDS.
template <int TOK>
struct HStage {
    static constexpr int t_off = TOK * H_ROW;
    static constexpr int t_copy = TOK * 8 * 4;
    static constexpr int bytes = t_off + 2 * t_copy;
};
// the table and two stages: 145 KB of gfx950's 160 KB of LDS per CU

__device__ inline int h_chunk(int m, int c) { return m * H_ROW + ((c ^ (m & 15)) << 4); }

// bf16 hi | lo << 16 with hi + lo == x exactly for finite x of at most 16
// significant bits; a non-finite x keeps lo = 0, so that the scale product is
// +-Inf (or NaN) exactly as the reference's product would be.
__device__ inline uint32_t bf16_pair_f(float x) {
    const uint32_t hb = __builtin_bit_cast(uint32_t, x) & 0xFFFF0000u;
    const float lo = x - __builtin_bit_cast(float, hb);
    const uint32_t lb = __builtin_isfinite(x) ? (__builtin_bit_cast(uint32_t, lo) & 0xFFFF0000u) : 0u;
    return (hb >> 16) | lb;
}

// Four int8 codebook values of low nibbles (lo) and of high nibbles (hi) ->
// four fp16 pair words {lo byte j, hi byte j}, exactly (v_cvt_f16_i16 on a
// sign-extended byte, written to one half of the word: one op per value).
__device__ inline v4u kv_pairs_f16(uint32_t lo, uint32_t hi) {
    uint32_t r0, r1, r2, r3;
    asm("v_cvt_f16_i16_sdwa %0, sext(%4) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_cvt_f16_i16_sdwa %0, sext(%5) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_0\n\t"
        "v_cvt_f16_i16_sdwa %1, sext(%4) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_1\n\t"
        "v_cvt_f16_i16_sdwa %1, sext(%5) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_1\n\t"
        "v_cvt_f16_i16_sdwa %2, sext(%4) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
        "v_cvt_f16_i16_sdwa %2, sext(%5) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_2\n\t"
        "v_cvt_f16_i16_sdwa %3, sext(%4) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_3\n\t"
        "v_cvt_f16_i16_sdwa %3, sext(%5) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_3"
        : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3)
        : "v"(lo), "v"(hi));
    return v4u{r0, r1, r2, r3};
}

// The fp16 code pair word of a qs byte b, {kv[b & 15], kv[b >> 4]}: the
// MFMA B operand's pair for the two weights that byte encodes (low nibble:
// element p, high nibble: element p + 16 of the sub-block).  A 256-entry
// table of these words sits at LDS address 0 of the fp16 kernel.
__device__ inline uint32_t kv_pair_word(int b) {
    const uint32_t kv[4] = {KV0, KV1, KV2, KV3};
    const int lo = b & 15, hi = b >> 4;
    return codes_to_half2((int8_t)(kv[lo >> 2] >> (8 * (lo & 3))), (int8_t)(kv[hi >> 2] >> (8 * (hi & 3))));
}

// The four qs bytes of q -> their four pair words, from the table at `lut`:
// one v_lshlrev_b32_sdwa (byte k -> its word's byte offset) and one
// ds_read_b32 per byte, against 19 VALU ops for the in-register decode.
__device__ inline v4u lut_pairs(const uint8_t* lut, uint32_t q) {
    uint32_t o0, o1, o2, o3;
    asm("v_lshlrev_b32_sdwa %0, 2, %4 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0\n\t"
        "v_lshlrev_b32_sdwa %1, 2, %4 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1\n\t"
        "v_lshlrev_b32_sdwa %2, 2, %4 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2\n\t"
        "v_lshlrev_b32_sdwa %3, 2, %4 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3"
        : "=&v"(o0), "=&v"(o1), "=&v"(o2), "=&v"(o3)  // early clobber: q is read after o0 is written
        : "v"(q));
    return v4u{*reinterpret_cast<const uint32_t*>(lut + o0), *reinterpret_cast<const uint32_t*>(lut + o1),
               *reinterpret_cast<const uint32_t*>(lut + o2), *reinterpret_cast<const uint32_t*>(lut + o3)};
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// 32-bit LDS address of a __shared__ object.
__device__ inline uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(lds_ptr_t)(const_cast<void*>(p));
}

// One 16-byte chunk per lane, global (sbase + voff) -> LDS at lds + 16 * lane
// (lds wave-uniform, in M0).  Written as asm so that the compiler does not
// treat it as an LDS store: it would otherwise make every later LDS read wait
// for it, the next stage's copy included.  The kernel itself waits (vmcnt)
// before the barrier that publishes the stage; the compiler's own loads stay
// correct, since vmcnt retires in order and its waits can only over-wait.
// Nothing else in the kernel uses M0.
__device__ inline void dma16(const void* sbase, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds)
                 : "memory", "m0");
}

struct HWeights {  // one super-block of this lane's weight row: header, and qs bytes 8h..8h+7 of 4 sub-blocks
    v2u hdr;
    v2u qs[4];
};

// One super-block of the fp16 kernel for one wave: the MFMAs and epilogue of
// its 4 sub-blocks x 4 token blocks from stage `st` (tokens) and `w` (its
// weight row), as a software pipeline over the 16 (sub-block, token block)
// steps: step t issues its three MFMAs, then the FMAs of step t - 1 (whose
// results have landed meanwhile) while the LDS fragments of step t + 1 are in
// flight; the next sub-block's weights are decoded during the current one.
// `w` is reloaded with the next super-block (load_next) once its last
// sub-block is decoded, so one set of weight registers serves both.
template <bool kDebug, int T, int TOK, typename LoadNext>
__device__ __forceinline__ void f16_superblock(const uint8_t* st, const uint8_t* lut, HWeights& w, v16f (&acc)[4],
                                               int kh, int h, int col, int lane, int64_t kb, int64_t m0, int64_t M,
                                               int64_t n, int64_t N, int64_t nb, int32_t* __restrict__ dbg,
                                               LoadNext&& load_next) {
    // this wave's half of the 6-bit scales at sub-block positions 0-3
    const uint32_t h0 = (w.hdr.x & 0xFFFFu) | ((w.hdr.x >> (8 * kh)) & 0xFF0000u), h1 = w.hdr.y >> (16 * kh);
    const float dw = half_bits_to_float(h0 & 0xFFFFu);
    // lane half h = 1 takes the low bf16 half of each weight scale; for an
    // infinite or NaN d_w that half is 0 and lane half 0 puts the high half
    // in k slot 2i only, against d_x's high half (slot 2i + 1 meets d_x's low
    // half, which may be 0): the scale tile is then +-Inf where the
    // reference's d_w * d_x is, and NaN where it is
    const uint32_t hmask = h ? 0xFFFF0000u : 0u;
    const bool finite = __builtin_isfinite(dw), zap = h && !finite;
    const uint32_t bsel = (h || finite) ? 0x07060706u : 0x0C0C0706u;
    // B operands of sub-block i, built in three parts spread over the steps
    // of the previous sub-block: the fp16 codes (b0: k 0-15, b1: k 16-31 of
    // the MFMA pair) and the scale column bsc: this row's d_w * (ls - 32)
    // split into exact bf16 halves, the high half in lane half 0 and the low
    // half in lane half 1, at k slots 2i, 2i + 1 of that half
    auto decode = [&](int i, int part, v4u& b0, v4u& b1, v4u& bsc) {
        if (part == 2) {
            // d_w * (ls - 32), exact: at most 16 significant bits (as the
            // product, not fma(d_w, ls, -32 d_w), which is Inf - Inf for an
            // infinite d_w)
            const float x = dw * (float)((int)subblock_ls(h0, h1, i) - 32);
            const uint32_t xb = __builtin_bit_cast(uint32_t, x);
            uint32_t v = __builtin_bit_cast(uint32_t, x - __builtin_bit_cast(float, xb & hmask));
            v = zap ? 0u : v;
            bsc = v4u{0u, 0u, 0u, 0u};
            bsc[i] = __builtin_amdgcn_perm(v, v, bsel);
        } else {
            (part ? b1 : b0) = lut_pairs(lut, part ? w.qs[i].y : w.qs[i].x);
        }
    };
    // operand r of step t (token block j = t % T, sub-block 4 kh + t / T):
    // r = 0, 1: the A operands of the two code MFMAs; r = 2: the scale MFMA's
    // A operand, the bf16 pairs of d_x of this wave's 4 sub-blocks for token
    // 32 j + col -- the same for all four sub-blocks, so it is read once per
    // super-block and token block (T registers of 4; measured 1-3 % faster
    // than re-reading it every step)
    auto frag = [&](int t, int r, v4u& a) {
        const int m = 32 * (t % T) + col, s = 4 * kh + t / T;
        if (r < 2)
            a = *reinterpret_cast<const v4u*>(st + h_chunk(m, 4 * s + 2 * h + r));
        else
            a = *reinterpret_cast<const v4u*>(st + HStage<TOK>::t_off + h * HStage<TOK>::t_copy + m * 32 + 16 * kh);
    };
    // half q of the epilogue of step t: acc += sp * dp for accumulators 8q .. 8q + 7
    auto epilogue = [&](int t, const v16f& dp, const v16f& sp, int q) {
        const int jp = t % T;
#pragma unroll
        for (int e = 8 * q; e < 8 * q + 8; ++e) {
            acc[jp][e] = __builtin_fmaf(sp[e], dp[e], acc[jp][e]);
            if (kDebug) {
                const int s = 4 * kh + t / T;
                const int64_t mg = m0 + 32 * jp + mfma_c_row(e, lane);
                if (mg < M && n < N)
                    dbg[(mg * N + n) * nb + kb * 8 + s] = (int)dp[e] * (subblock_ls(h0, h1, t / T) - 32);
            }
        }
        // pin the epilogue here: without it the optimiser sinks every FMA to
        // the end of the super-block and spills the MFMA results
        asm volatile("" : "+v"(acc[jp]));
    };

    v4u b0, b1, bsc, nb0, nb1, nbsc, a0, a1, ts[T];
#pragma unroll
    for (int part = 0; part < 3; ++part) decode(0, part, b0, b1, bsc);
    frag(0, 0, a0);
    frag(0, 1, a1);
#pragma unroll
    for (int j = 0; j < T; ++j) frag(j, 2, ts[j]);
    v16f dp, sp;
    constexpr int STEPS = 4 * T;
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
        const int i = t / T, j = t % T;
        // each MFMA is followed by the LDS read that refills its A operand for
        // step t + 1 and by a share of the VALU work (the FMAs of step t - 1,
        // then a part of the next sub-block's decode), so that the wave issues
        // VALU ops while its MFMAs run instead of stalling on a busy matrix
        // pipe; the scheduling barriers keep that order
        v16f d = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a0), __builtin_bit_cast(v8h, b0),
                                                        v16f{}, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if (t + 1 < STEPS) frag(t + 1, 0, a0);
        if (t > 0) epilogue(t - 1, dp, sp, 0);
        __builtin_amdgcn_sched_barrier(0);
        d = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a1), __builtin_bit_cast(v8h, b1), d, 0, 0,
                                                   0);
        __builtin_amdgcn_sched_barrier(0);
        if (t + 1 < STEPS) frag(t + 1, 1, a1);
        if (t > 0) epilogue(t - 1, dp, sp, 1);
        __builtin_amdgcn_sched_barrier(0);
        const v16f sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, ts[j]),
                                                                __builtin_bit_cast(v8bf, bsc), v16f{}, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        // the next sub-block's three decode parts: part p in step min(p, T - 1)
        if (i < 3) {
#pragma unroll
            for (int part = 0; part < 3; ++part)
                if (j == (part < T ? part : T - 1)) decode(i + 1, part, nb0, nb1, nbsc);
            if (j == T - 1) {
                b0 = nb0;
                b1 = nb1;
                bsc = nbsc;
            }
        }
        if (i == 2 && j == T - 1) load_next(w);  // decode(3) above was the last use of w
        dp = d;
        sp = sc;
        __builtin_amdgcn_sched_barrier(0);
    }
    epilogue(STEPS - 1, dp, sp, 0);
    epilogue(STEPS - 1, dp, sp, 1);
}

// One 128-row x 32T-token tile (T token blocks per wave; the per-output
// arithmetic does not depend on T, so neither do the results).
// W, Y, N, ldy_m: the tile's matrix, whose first row tile is tile0.
// RG row groups of 32 rows (4: the 128-row tile of 8 waves; 2: the 64-row
// half-height tile of 4 waves, at most 64 tokens); wave w computes row group
// w % RG on the sub-block half w / RG, so a row's arithmetic is the same in
// both.
template <bool kDebug, int T, int RG>
__device__ __forceinline__ void f16_tile(const uint8_t* __restrict__ W, float* __restrict__ Y, int64_t N,
                                         int64_t ldy_m, int tile0, const uint32_t* __restrict__ ahq,
                                         const uint32_t* __restrict__ ads, int64_t K, int64_t M, int64_t ldy_n, int bx,
                                         int by, uint8_t* smem, int32_t* __restrict__ dbg) {
    static_assert(RG == 4 || (RG == 2 && T <= 2), "half-height tiles hold at most 64 tokens");
    constexpr int TOK = 32 * RG, STAGE = HStage<TOK>::bytes;
    constexpr int CPW = 8 * T / RG;  // 1 KB token copies per wave and stage (16 T per stage)
    uint8_t(*const stages)[STAGE] = reinterpret_cast<uint8_t(*)[STAGE]>(smem + H_LUT);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, in an SGPR
    const int rg = wave % RG, kh = wave / RG, h = lane >> 5, col = lane & 31;
    const int64_t n0 = (int64_t)(bx - tile0) * (32 * RG);
    const int64_t m0 = (int64_t)by * (32 * T);
    const int64_t bpr = K / QK_K, nb = K / QK8_1, row_bytes = bpr * BLOCK_BYTES;

    // ---- this lane's weight row (rows past N repeat the last; never stored)
    const int64_t n = n0 + 32 * rg + col;
    const uint8_t* wtile = W + n0 * row_bytes;
    const uint32_t woff = (uint32_t)(((n < N) ? n - n0 : N - 1 - n0) * row_bytes);
    auto load_w = [&](HWeights& g, int64_t kb) {
        const uint8_t* p = wtile + kb * BLOCK_BYTES + woff;
        g.hdr = *reinterpret_cast<const v2u*>(p);
#pragma unroll
        for (int i = 0; i < 4; ++i) g.qs[i] = *reinterpret_cast<const v2u*>(p + 8 + 16 * (4 * kh + i) + 8 * h);
    };

    // ---- token staging (32 T token rows of 512 bytes): instruction i of this
    // wave fills LDS chunks (wave * CPW + i) * 64 + lane of a stage, i.e. row
    // 2 CPW wave + 2i + h, chunk col ^ (row & 15) of it (the swizzle)
    const uint8_t* xtile = reinterpret_cast<const uint8_t*>(ahq) + m0 * (2 * K);
    const int xrow = 2 * CPW * wave + h, xlast = (int)min<int64_t>(M - 1 - m0, 32 * T - 1);  // rows past M repeat the last
    const uint32_t xstride = (uint32_t)(2 * K);
    const uint32_t lds_wave = __builtin_amdgcn_readfirstlane(lds_addr(&stages[0][0]) + wave * CPW * 1024);
    // for CPW = 2, 4, 8 the bits of xrow & 15 and of 2i are disjoint, so the
    // swizzled chunk is (col ^ (xrow & 15)) ^ 2i: one XOR per copy
    const uint32_t xcol = 16u * (uint32_t)(col ^ (xrow & 15));
    auto issue_x = [&](int64_t kb, int stage) {
        const uint8_t* src = xtile + kb * 512;
#pragma unroll
        for (int i = 0; i < CPW; ++i) {
            const int m = xrow + 2 * i;
            const uint32_t c16 = (CPW & (CPW - 1)) ? 16u * (uint32_t)(col ^ (m & 15)) : (xcol ^ (32u * i));
            dma16(src, (uint32_t)min(m, xlast) * xstride + c16, lds_wave + stage * STAGE + i * 1024);
        }
    };
    // token scales: thread tid -> token tid >> 2, sub-blocks 2 (tid & 3), + 1
    const int tm = tid >> 2, ts = 2 * (tid & 3);
    const uint32_t* dtile = ads + m0 * nb;
    const uint32_t doff = (uint32_t)(((m0 + tm < M) ? tm : M - 1 - m0) * nb + ts);
    auto load_d = [&](int64_t kb) { return *reinterpret_cast<const v2u*>(dtile + kb * 8 + doff); };
    // copy 1 (lane half 1, which meets the weight scale's low half) has 0
    // for a non-finite d_x, so that no Inf meets a zero low half (0 * Inf)
    auto store_d = [&](v2u d, uint8_t* stage) {
        uint32_t* t = reinterpret_cast<uint32_t*>(stage + HStage<TOK>::t_off) + tm * 8 + ts;
        const float x0 = half_bits_to_float(d.x & 0xFFFFu), x1 = half_bits_to_float(d.y & 0xFFFFu);
        const v2u p = v2u{bf16_pair_f(x0), bf16_pair_f(x1)};
        *reinterpret_cast<v2u*>(t) = p;
        *reinterpret_cast<v2u*>(t + HStage<TOK>::t_copy / 4) =
            v2u{__builtin_isfinite(x0) ? p.x : 0u, __builtin_isfinite(x1) ? p.y : 0u};
    };

    v16f acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = v16f{};

    // weights run two super-blocks ahead: w holds super-block kb, wn kb + 1,
    // and kb + 2 is loaded into w's registers once kb's decode is done
    if (tid < 256) reinterpret_cast<uint32_t*>(smem)[tid] = kv_pair_word(tid);  // published by the barrier below

    HWeights w, wn;
    load_w(w, 0);
    if (bpr > 1) load_w(wn, 1);
    issue_x(0, 0);
    {
        const v2u d0 = load_d(0);
        __builtin_amdgcn_s_waitcnt(0);
        store_d(d0, stages[0]);
    }
    __syncthreads();

    // one super-block from stage kb & 1 while super-block kb + 1 streams into
    // the other; wc holds kb's weights, wo kb + 1's
    // The loads are issued unconditionally (past the end they repeat the last
    // super-block into registers and a stage that nothing reads any more), so
    // that every iteration issues the same sequence: 2T copies + 1 token-scale
    // load at the start, 5 weight loads after sub-block 2; the wait before the
    // barrier then leaves exactly the 5 weight loads in flight.
    auto superblock = [&](int64_t kb, HWeights& wc) {
        const int cur = (int)(kb & 1);
        const int64_t kb1 = min(kb + 1, bpr - 1), kb2 = min(kb + 2, bpr - 1);
        issue_x(kb1, cur ^ 1);
        v2u dnext = load_d(kb1);
        f16_superblock<kDebug, T, TOK>(stages[cur], smem, wc, acc, kh, h, col, lane, kb, m0, M, n, N, nb, dbg,
                               [&](HWeights& g) { load_w(g, kb2); });
        // this thread's direct-to-LDS copies and token scales have landed; the
        // 5 weight loads of super-block kb + 2, issued after them, may still
        // be in flight (vmcnt counts completions in issue order)
        __builtin_amdgcn_s_waitcnt(kVmcnt5);
        // keep the conversion of the token scales here: hoisted next to their
        // load it would need a vmcnt(0) there, i.e. wait for the whole next
        // stage before computing this one
        asm volatile("" : "+v"(dnext));
        if (kb + 1 < bpr) store_d(dnext, stages[cur ^ 1]);
        __syncthreads();
    };
    // two super-blocks per iteration, so that the weight registers swap
    // roles without copies (a copy of a register still being loaded would
    // have to wait for the load)
    // (an odd last super-block is peeled off, so that the loop is always
    // entered from the second half: the compiler's own waits then know which
    // weight loads are still in flight)
    int64_t kb = 0;
    for (; kb + 1 < bpr; kb += 2) {
        superblock(kb, w);
        superblock(kb + 1, wn);
    }
    if (kb < bpr) superblock(kb, w);

    // the two sub-block halves of each row group add their partial sums:
    // kh = 0 finalises token blocks j < (T + 1) / 2, kh = 1 the others, each
    // taking the other half's partial sums through LDS (constant indices
    // only: a runtime index into acc would put it in scratch memory)
    constexpr int HALF = (T + 1) / 2;
    float* red = reinterpret_cast<float*>(&stages[0][0]);  // both stages are free now
    auto slot = [&](int from_kh, int j) { return red + ((rg * 2 + from_kh) * 4 + j) * 1024 + lane; };
    auto store = [&](const v16f& a, int j) {
        if (n >= N) return;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int64_t mg = m0 + 32 * j + mfma_c_row(e, lane);
            if (mg < M) Y[mg * ldy_m + n * ldy_n] = a[e];
        }
    };
#pragma unroll
    for (int j = 0; j < T; ++j) {
        if ((j < HALF) == (kh == 1)) {  // the other half finalises block j
#pragma unroll
            for (int e = 0; e < 16; ++e) slot(kh, j)[e * 64] = acc[j][e];
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < T; ++j) {
        if ((j < HALF) == (kh == 0)) {
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[j][e] += slot(kh ^ 1, j)[e * 64];
            store(acc[j], j);
        }
    }
}

// Workgroups of a launch fall into up to F16_SEGS segments, each a range of
// row tiles (128 rows) x all tokens in tiles of 32T tokens; segment 0's
// workgroups take their tiles in XCD-aware order.  A host-side plan picks
// the segments so that the workgroups fill the CUs' rounds evenly.
constexpr int F16_SEGS = 3;
struct F16Seg {
    int wg_end;  // one past this segment's last workgroup
    int rt0;     // first row tile
    int rts;     // row tiles
    int T;       // token blocks (of 32) per tile: 1..4
};
struct F16Plan {
    F16Seg seg[F16_SEGS];
};

// RG = 4: 128-row tiles of 8 waves (one workgroup per CU); RG = 2: 64-row
// tiles of 4 waves and at most 64 tokens (two per CU), for launches with too
// few big tiles to fill the CUs.  A row's arithmetic is the same in both.
template <bool kDebug, bool kGroup, int RG = 4>
__global__ __launch_bounds__(128 * RG) void gemm_f16_kernel(const GemmGroup grp, const uint32_t* __restrict__ ahq,
                                                            const uint32_t* __restrict__ ads, int64_t K, int64_t M,
                                                            int64_t ldy_n, const F16Plan plan,
                                                            int32_t* __restrict__ dbg) {
    // LDS: the 1 KB code pair table at address 0, then the two stages
    __shared__ __attribute__((aligned(1024))) uint8_t smem[H_LUT + 2 * HStage<32 * RG>::bytes];
    const int b = (int)blockIdx.x;
    // the segment (scalar selects on the by-value plan)
    int g = 0;
#pragma unroll
    for (int i = 0; i + 1 < F16_SEGS; ++i) g += b >= plan.seg[i].wg_end ? 1 : 0;
    F16Seg sg = plan.seg[0];
    int start = 0;
#pragma unroll
    for (int i = 1; i < F16_SEGS; ++i) {
        if (g == i) {
            sg = plan.seg[i];
            start = plan.seg[i - 1].wg_end;
        }
    }
    int tile = b - start;
    if (g == 0) {
        // XCD-aware tile order: the 8 XCDs take workgroups round-robin, so
        // workgroup b runs on XCD b % 8; each XCD is given a contiguous range
        // of the token-major tile order, so its tiles share few token tiles
        const int tiles = sg.wg_end, x = b & 7, q = tiles >> 3, r = tiles & 7;
        tile = x * q + min(x, r) + (b >> 3);
    }
    const int bx = sg.rt0 + tile % sg.rts, by = tile / sg.rts;
    // the matrix of this tile: gemm_select's choice, by the logical tile index
    const uint8_t* W = grp.W[0];
    float* Y = grp.Y[0];
    int64_t N = grp.N[0], ldy_m = grp.ldy_m[0];
    int tile0 = 0;
    if (kGroup) {
        int gsel = 0;
#pragma unroll
        for (int i = 0; i + 1 < GEMV_GROUP_MAX; ++i) gsel += bx >= grp.tile_end[i] ? 1 : 0;
#pragma unroll
        for (int i = 1; i < GEMV_GROUP_MAX; ++i) {
            if (gsel == i) {
                W = grp.W[i];
                Y = grp.Y[i];
                N = grp.N[i];
                ldy_m = grp.ldy_m[i];
                tile0 = grp.tile_end[i - 1];
            }
        }
    }
    if constexpr (RG == 2) {
        if (sg.T == 1) f16_tile<kDebug, 1, 2>(W, Y, N, ldy_m, tile0, ahq, ads, K, M, ldy_n, bx, by, smem, dbg);
        else f16_tile<kDebug, 2, 2>(W, Y, N, ldy_m, tile0, ahq, ads, K, M, ldy_n, bx, by, smem, dbg);
    } else {
        switch (sg.T) {
            case 1: f16_tile<kDebug, 1, 4>(W, Y, N, ldy_m, tile0, ahq, ads, K, M, ldy_n, bx, by, smem, dbg); break;
            case 2: f16_tile<kDebug, 2, 4>(W, Y, N, ldy_m, tile0, ahq, ads, K, M, ldy_n, bx, by, smem, dbg); break;
            case 3: f16_tile<kDebug, 3, 4>(W, Y, N, ldy_m, tile0, ahq, ads, K, M, ldy_n, bx, by, smem, dbg); break;
            default: f16_tile<kDebug, 4, 4>(W, Y, N, ldy_m, tile0, ahq, ads, K, M, ldy_n, bx, by, smem, dbg); break;
        }
    }
}

static int gemm_kind() {
    static const int kind = []() {
        const char* v = getenv("IQ4XS_GEMM_KIND");  // tuning override: 0 = 64x64, 1 = 128x128, 2 = fp16 matrix cores
        return v ? atoi(v) : 2;
    }();
    return kind;
}

// Time of one workgroup of T token blocks relative to T = 4 with every CU
// busy, for the round planner below (per-tile work is T token blocks against
// the same weight decode, DMA and barrier cost per super-block).  Measured
// on q_proj (K = 5120) at M = 512 with every workgroup of one size: 1, 2, 3
// or 4 token blocks in 35.9, 47.4, 57.7, 77.3 us per round.
static double f16_tile_cost(int T) {
    static const double c[5] = {0.0, 0.46, 0.61, 0.75, 1.0};
    return c[T < 1 ? 1 : (T > 4 ? 4 : T)];
}

// A launch of fewer workgroups than CUs runs each of them faster (less
// contention for L2 and HBM): o_proj at M = 512, 160 workgroups of 4 token
// blocks, takes 0.85x the per-super-block time of 256.  Modelled as
// alpha + (1 - alpha) * busy fraction.
static double f16_occupancy(int64_t wgs, int cus) {
    const double alpha = 0.6, f = wgs >= cus ? 1.0 : (double)wgs / cus;
    return alpha + (1.0 - alpha) * f;
}

static int64_t f16_token_tiles(int64_t M, int T) { return (M + 32 * T - 1) / (32 * T); }

// Makespan of the plan's workgroups, dispatched in order to `cus` CUs that
// each run one at a time (one workgroup fills a CU's LDS).
static double f16_makespan(const F16Plan& p, int cus) {
    std::priority_queue<double, std::vector<double>, std::greater<double>> free_at;
    for (int c = 0; c < cus; ++c) free_at.push(0.0);
    const double occ = f16_occupancy(p.seg[F16_SEGS - 1].wg_end, cus);
    double end = 0.0;
    int start = 0;
    for (int g = 0; g < F16_SEGS; ++g) {
        const double d = f16_tile_cost(p.seg[g].T) * occ;
        for (int w = start; w < p.seg[g].wg_end; ++w) {
            const double t = free_at.top() + d;
            free_at.pop();
            free_at.push(t);
            end = std::max(end, t);
        }
        start = p.seg[g].wg_end;
    }
    return end;
}

static F16Plan f16_plan_of(std::initializer_list<std::pair<int64_t, int>> segs, int64_t M) {
    F16Plan p{};
    int64_t rt = 0, wg = 0;
    int g = 0;
    for (const auto& sgm : segs) {
        p.seg[g] = F16Seg{0, (int)rt, (int)sgm.first, sgm.second};
        wg += sgm.first * f16_token_tiles(M, sgm.second);
        p.seg[g].wg_end = (int)wg;
        rt += sgm.first;
        ++g;
    }
    for (; g < F16_SEGS; ++g) p.seg[g] = F16Seg{(int)wg, (int)rt, 1, 4};  // empty
    return p;
}

// The tiling of `row_tiles` row tiles x M tokens: one segment of one token
// tile size, or a bulk of whole rounds plus a tail of smaller tiles that
// spreads the last round over the CUs -- whichever finishes first by
// f16_makespan.  A shape's plan depends on the shape and the CU count only,
// and no plan changes a result bit.
static F16Plan f16_plan(int64_t row_tiles, int64_t M) {
    static const int forced = []() {
        const char* v = getenv("IQ4XS_GEMM_T");  // tuning override: one segment of this token tile size
        const int t = v ? atoi(v) : 0;
        return (t >= 1 && t <= 4) ? t : 0;
    }();
    if (forced) return f16_plan_of({{row_tiles, forced}}, M);
    const int cus = device_cu_count();
    static std::mutex mu;
    static std::map<std::tuple<int64_t, int64_t, int>, F16Plan> cache;
    const auto key = std::make_tuple(row_tiles, M, cus);
    {
        std::lock_guard<std::mutex> lock(mu);
        const auto it = cache.find(key);
        if (it != cache.end()) return it->second;
    }
    F16Plan best = f16_plan_of({{row_tiles, 4}}, M);
    double best_t = f16_makespan(best, cus);
    auto consider = [&](const F16Plan& p) {
        const double t = f16_makespan(p, cus);
        if (t < best_t - 1e-9) {
            best = p;
            best_t = t;
        }
    };
    for (int T = 3; T >= 1; --T) consider(f16_plan_of({{row_tiles, T}}, M));
    for (int Tb = 4; Tb >= 2; --Tb) {
        const int64_t per_rt = f16_token_tiles(M, Tb);
        const int64_t rounds = row_tiles * per_rt / cus;
        for (int64_t k = rounds; k >= 1 && k + 2 >= rounds; --k) {
            const int64_t rb = k * cus / per_rt;  // whole row tiles within k rounds
            if (rb <= 0 || rb >= row_tiles) continue;
            for (int Tt = Tb - 1; Tt >= 1; --Tt) consider(f16_plan_of({{rb, Tb}, {row_tiles - rb, Tt}}, M));
        }
    }
    if (getenv("IQ4XS_GEMM_PLAN_LOG") != nullptr) {  // tuning aid: the chosen segments, on stderr
        fprintf(stderr, "[iq4xs] gemm plan row_tiles=%lld M=%lld:", (long long)row_tiles, (long long)M);
        for (int g = 0; g < F16_SEGS; ++g)
            fprintf(stderr, " [wg_end=%d rt0=%d rts=%d T=%d]", best.seg[g].wg_end, best.seg[g].rt0, best.seg[g].rts,
                    best.seg[g].T);
        fprintf(stderr, " est=%.3f\n", best_t);
    }
    std::lock_guard<std::mutex> lock(mu);
    cache.emplace(key, best);
    return best;
}

template <bool kDebug, bool kGroup>
static hipError_t launch_f16_kernel(const GemmGroup& grp, int64_t row_tiles, const uint32_t* ahq, const uint32_t* ads,
                                    int64_t K, int64_t M, int64_t ldy_n, int32_t* dbg, hipStream_t stream) {
    if (row_tiles * f16_token_tiles(M, 1) > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
    // Half-height tiles (64 rows, 4 waves, one token block each) when even
    // single-block 128-row tiles would fill at most half the CUs (k/v at
    // M = 512: 128 -> 256 workgroups, 37 -> 33 us).  They run slower per
    // row than big tiles wherever those fill the chip, so only there.
    const int64_t cus = device_cu_count();
    if (!kGroup && !kDebug && row_tiles * f16_token_tiles(M, 1) * 2 <= cus) {
        GemmGroup g2 = grp;
        const int64_t rt2 = (grp.N[0] + 63) / 64;
        g2.tile_end[0] = (int)rt2;
        const F16Plan plan = f16_plan_of({{rt2, 1}}, M);
        const int wgs = plan.seg[F16_SEGS - 1].wg_end;
        if (wgs <= 0) return hipSuccess;
        hipLaunchKernelGGL((gemm_f16_kernel<false, false, 2>), dim3((unsigned)wgs), dim3(256), 0, stream, g2, ahq,
                           ads, K, M, ldy_n, plan, dbg);
        return hipGetLastError();
    }
    const F16Plan plan = kDebug ? f16_plan_of({{row_tiles, 4}}, M) : f16_plan(row_tiles, M);
    const int wgs = plan.seg[F16_SEGS - 1].wg_end;
    if (wgs <= 0) return hipSuccess;
    hipLaunchKernelGGL((gemm_f16_kernel<kDebug, kGroup>), dim3((unsigned)wgs), dim3(H_THREADS), 0, stream, grp, ahq,
                       ads, K, M, ldy_n, plan, dbg);
    return hipGetLastError();
}

// The fp16 kernel addresses a tile's weight rows and tokens with 32-bit offsets.
static bool f16_fits(int64_t K) {
    return (int64_t)H_BN * (K / QK_K) * BLOCK_BYTES < (1ll << 32) && (int64_t)H_BM * 2 * K < (1ll << 32);
}

// The 128x128 kernel runs one workgroup per CU and is faster per tile; the
// 64x64 kernel (three per CU) wins when big tiles would leave many CUs idle:
// fewer tiles than ~9/16 of the CUs (k/v-sized matrices).  Both give
// bit-identical outputs, so this choice is a speed choice only (thresholds
// from measurements on the 27B-class shapes at M = 512 / 2048).
static bool use_big_tiles(int64_t N, int64_t M, int64_t K) {
    // the 128x128 kernel addresses a tile's rows and tokens with 32-bit offsets
    if ((int64_t)G2_BN * (K / QK_K) * BLOCK_BYTES >= (1ll << 32) || (int64_t)G2_BM * K >= (1ll << 32)) return false;
    const int k = gemm_kind();
    if (k == 0 || k == 1) return k == 1;
    const int64_t cus = device_cu_count();
    const int64_t tiles = ((N + G2_BN - 1) / G2_BN) * ((M + G2_BM - 1) / G2_BM);
    return tiles >= cus * 9 / 16;
}

template <bool kDebug, bool kGroup>
static hipError_t launch_gemm_kernel(bool big, const GemmGroup& grp, int64_t gx, const int8_t* aqs, const uint32_t* ads,
                                     int64_t K, int64_t M, int64_t ldy_n, int32_t* dbg, hipStream_t stream) {
    const int64_t gy = (M + (big ? G2_BM : GEMM_BM) - 1) / (big ? G2_BM : GEMM_BM);
    if (gx > 0x7FFFFFFF || gy > 65535) return hipErrorInvalidConfiguration;
    if (big) {
        static const bool attrs = []() {
            // two stages exceed the default dynamic-LDS cap; gfx950 has 160 KB per CU
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_iq4xs_db_kernel<kDebug, kGroup>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      2 * (kDebug ? G2_STAGE_DBG : G2_STAGE));
            return true;
        }();
        (void)attrs;
        hipLaunchKernelGGL((gemm_iq4xs_db_kernel<kDebug, kGroup>), dim3((unsigned)gx, (unsigned)gy), dim3(G2_THREADS),
                           2 * (size_t)(kDebug ? G2_STAGE_DBG : G2_STAGE), stream, grp, aqs, ads, K, M, ldy_n, dbg);
    } else {
        hipLaunchKernelGGL((gemm_iq4xs_mfma_kernel<kDebug, kGroup>), dim3((unsigned)gx, (unsigned)gy), dim3(256), 0,
                           stream, grp, aqs, ads, K, M, ldy_n, dbg);
    }
    return hipGetLastError();
}

hipError_t launch_gemm(const uint8_t* W, const int8_t* aqs, const uint32_t* ads, const uint32_t* ahq, float* Y,
                       int64_t K, int64_t N, int64_t M, int64_t ldy_m, int64_t ldy_n, int32_t* dbg,
                       hipStream_t stream) {
    clear_launch_error();
    if (gemm_kind() == 2 && f16_fits(K)) {
        GemmGroup grp{};
        grp.W[0] = W;
        grp.Y[0] = Y;
        grp.N[0] = N;
        grp.ldy_m[0] = ldy_m;
        const int64_t gx = (N + H_BN - 1) / H_BN;
        if (gx > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
        grp.tile_end[0] = (int)gx;
        return dbg ? launch_f16_kernel<true, false>(grp, gx, ahq, ads, K, M, ldy_n, dbg, stream)
                   : launch_f16_kernel<false, false>(grp, gx, ahq, ads, K, M, ldy_n, dbg, stream);
    }
    const bool big = use_big_tiles(N, M, K);
    GemmGroup grp{};
    grp.W[0] = W;
    grp.Y[0] = Y;
    grp.N[0] = N;
    grp.ldy_m[0] = ldy_m;
    const int64_t gx = (N + (big ? G2_BN : GEMM_BN) - 1) / (big ? G2_BN : GEMM_BN);
    if (gx > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
    grp.tile_end[0] = (int)gx;
    if (big && dbg == nullptr) {
        // Big tiles whose last round on the CUs would hold only a few (at most
        // a quarter): the rows of that round go to the 64x64 kernel in a
        // second launch, whose small tiles spread them over the chip.  Both
        // kernels give bit-identical outputs.  M = 512 gate/up: 544 tiles =
        // 2 full rounds + 32 on 256 CUs.
        const int64_t gy = (M + G2_BM - 1) / G2_BM;
        const int64_t cus = device_cu_count();
        const int64_t full = gx * gy / cus, rem = gx * gy - full * cus;
        if (full >= 1 && rem > 0 && 4 * rem <= cus && (full * cus) % gy == 0) {
            const int64_t gx_big = full * cus / gy;  // whole N-tiles, every token tile
            const int64_t n_big = gx_big * G2_BN;    // < N, since rem > 0
            grp.N[0] = n_big;
            grp.tile_end[0] = (int)gx_big;
            const hipError_t e = launch_gemm_kernel<false, false>(true, grp, gx_big, aqs, ads, K, M, ldy_n, dbg, stream);
            if (e != hipSuccess) return e;
            GemmGroup rest{};
            rest.W[0] = W + n_big * ((K / QK_K) * BLOCK_BYTES);
            rest.Y[0] = Y + n_big * ldy_n;
            rest.N[0] = N - n_big;
            rest.ldy_m[0] = ldy_m;
            const int64_t gx_rest = (N - n_big + GEMM_BN - 1) / GEMM_BN;
            rest.tile_end[0] = (int)gx_rest;
            return launch_gemm_kernel<false, false>(false, rest, gx_rest, aqs, ads, K, M, ldy_n, dbg, stream);
        }
    }
    return dbg ? launch_gemm_kernel<true, false>(big, grp, gx, aqs, ads, K, M, ldy_n, dbg, stream)
               : launch_gemm_kernel<false, false>(big, grp, gx, aqs, ads, K, M, ldy_n, dbg, stream);
}

// One launch for `count` matrices sharing K and the activations (two when a
// short last round is split off, below): the tile size is chosen for the
// summed rows, so the small matrices fill CUs that the big ones' last round
// leaves idle.
hipError_t launch_gemm_group(int count, const uint8_t* const* W, float* const* Y, const int64_t* N, const int8_t* aqs,
                             const uint32_t* ads, const uint32_t* ahq, int64_t K, int64_t M, bool layout_mk,
                             hipStream_t stream) {
    clear_launch_error();
    if (count < 1 || count > GEMV_GROUP_MAX) return hipErrorInvalidValue;
    int64_t n_sum = 0;
    for (int i = 0; i < count; ++i) n_sum += N[i];
    if (gemm_kind() == 2 && f16_fits(K)) {
        GemmGroup grp{};
        int64_t tiles = 0;
        for (int i = 0; i < GEMV_GROUP_MAX; ++i) {
            const int j = i < count ? i : count - 1;  // unused entries repeat the last matrix, past every tile
            if (i < count) tiles += (N[j] + H_BN - 1) / H_BN;
            if (tiles > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
            grp.W[i] = W[j];
            grp.Y[i] = Y[j];
            grp.N[i] = N[j];
            grp.ldy_m[i] = layout_mk ? N[j] : 1;
            grp.tile_end[i] = (int)tiles;
        }
        return launch_f16_kernel<false, true>(grp, tiles, ahq, ads, K, M, layout_mk ? 1 : M, nullptr, stream);
    }
    const bool big = use_big_tiles(n_sum, M, K);
    const int bn = big ? G2_BN : GEMM_BN;
    GemmGroup grp{};
    int64_t tiles = 0;
    for (int i = 0; i < GEMV_GROUP_MAX; ++i) {
        const int j = i < count ? i : count - 1;  // unused entries repeat the last matrix, past every tile
        if (i < count) tiles += (N[j] + bn - 1) / bn;
        if (tiles > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
        grp.W[i] = W[j];
        grp.Y[i] = Y[j];
        grp.N[i] = N[j];
        grp.ldy_m[i] = layout_mk ? N[j] : 1;
        grp.tile_end[i] = (int)tiles;
    }
    if (big) {
        // As for single calls: a short last round of big tiles, when it lies
        // in the last matrix, becomes a 64x64 launch over that matrix's
        // trailing rows (M = 512 gate+up: 1088 tiles = 4 rounds + 64).
        const int64_t gy = (M + G2_BM - 1) / G2_BM;
        const int64_t cus = device_cu_count();
        const int64_t full = tiles * gy / cus, rem = tiles * gy - full * cus;
        const int last = count - 1;
        const int64_t first_last = last > 0 ? grp.tile_end[last - 1] : 0;  // the last matrix's first N-tile
        if (full >= 1 && rem > 0 && 4 * rem <= cus && (full * cus) % gy == 0 && full * cus / gy > first_last) {
            const int64_t t_big = full * cus / gy;                 // N-tiles of the grouped launch
            const int64_t n_keep = (t_big - first_last) * G2_BN;  // rows of the last matrix it keeps (< N)
            for (int i = last; i < GEMV_GROUP_MAX; ++i) {
                grp.N[i] = n_keep;
                grp.tile_end[i] = (int)t_big;
            }
            const hipError_t e =
                launch_gemm_kernel<false, true>(true, grp, t_big, aqs, ads, K, M, layout_mk ? 1 : M, nullptr, stream);
            if (e != hipSuccess) return e;
            GemmGroup rest{};
            rest.W[0] = W[last] + n_keep * ((K / QK_K) * BLOCK_BYTES);
            rest.Y[0] = Y[last] + n_keep * (layout_mk ? 1 : M);
            rest.N[0] = N[last] - n_keep;
            rest.ldy_m[0] = layout_mk ? N[last] : 1;
            const int64_t gx_rest = (N[last] - n_keep + GEMM_BN - 1) / GEMM_BN;
            rest.tile_end[0] = (int)gx_rest;
            return launch_gemm_kernel<false, false>(false, rest, gx_rest, aqs, ads, K, M, layout_mk ? 1 : M, nullptr,
                                                    stream);
        }
    }
    return launch_gemm_kernel<false, true>(big, grp, tiles, aqs, ads, K, M, layout_mk ? 1 : M, nullptr, stream);
}

__global__ __launch_bounds__(64) void probe_mfma_kernel(const int8_t* __restrict__ A, const int8_t* __restrict__ B,
                                                        int32_t* __restrict__ C) {
    const int lane = threadIdx.x;
    const int k0 = 16 * (lane >> 5);
    const v4i a = *reinterpret_cast<const v4i*>(A + (lane & 31) * 32 + k0);
    const v4i b = *reinterpret_cast<const v4i*>(B + (lane & 31) * 32 + k0);
    const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, v16i{}, 0, 0, 0);
#pragma unroll
    for (int e = 0; e < 16; ++e) C[mfma_c_row(e, lane) * 32 + (lane & 31)] = c[e];
}

hipError_t launch_probe_mfma(const int8_t* A, const int8_t* B, int32_t* C, hipStream_t stream) {
    clear_launch_error();
    hipLaunchKernelGGL(probe_mfma_kernel, dim3(1), dim3(64), 0, stream, A, B, C);
    return hipGetLastError();
}

}  // namespace iq4xs
