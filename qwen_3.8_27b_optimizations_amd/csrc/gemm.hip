// gemm.hip -- IQ4_XS x Q8_1 prefill GEMM on gfx950 matrix cores.
//
// Semantics: the reference GEMM (real_stock_dp4a_comparator.hip:374-443):
//   Y[n,m] = sum_kb fp16(W.d) * fp16(ds[m,kb].d) * (float)(sumi[n,m,kb] * (ls-32))
// where sumi is the exact int32 dot of a 32-weight sub-block with the
// matching Q8_1 block.
//
// The kernel: gemm_f16_kernel (128x128 tile, 8 waves, two LDS stages),
// which runs the integer products on v_mfma_f32_32x32x16_f16 -- codebook
// values and Q8_1 codes are exact in fp16 and a sub-block's 32-term sum is an
// integer below 2^24, so the MFMA returns sumi exactly, as a float -- and
// leaves one FMA per output and sub-block for the epilogue.  Its design notes
// are with the kernel below.
//
// Non-finite scales keep the reference's class: the scale tile never puts an
// infinite half of one scale against a zero half of the other, and a token
// block whose activation scale d_x is not finite is recomputed term by term
// with the reference's arithmetic (nonfinite_fixup below).
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

// 32x32 MFMA result layout (v_mfma_f32_32x32x16_f16 here, and the
// v_mfma_i32_32x32x32_i8 of the small-batch GEMV and the layout probe):
//   C: element e of lane l is row 8*(e>>2) + 4*(l>>5) + (e&3), column (l & 31)
// (i8 operands: lane l supplies row / column l & 31, k = 16*(l >> 5) .. +15)
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

typedef float v16f __attribute__((ext_vector_type(16)));

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
constexpr int H_LUT = 1024;                          // the code pair table
// A stage of a tile of at most TOK tokens: the token rows, then the token scale
// pairs uint32 [2][TOK][8] (copy h feeds lane half h).  Full tiles use TOK =
// 128 (72 KB); half-height tiles (64 rows, 4 waves, at most 64 tokens) TOK =
// 64, so that two of them fit a CU's LDS.
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

// The outputs of a tile's tokens whose Q8_1 block scale d_x is not finite
// (|x| >= 65520 * 127 in a 32-block, or a NaN), term by term with the
// reference's arithmetic (real_stock_dp4a_comparator.hip:164-165):
// (fp16 d_w * fp16 d_x) * float(sumi * (ls - 32)).  Every output of such a
// token holds at least one non-finite term, so its value is the fp32 sum of
// its non-finite terms alone (+-Inf, or NaN for a NaN term or both signs of
// Inf): a finite term cannot change that sum, and finite partial sums of this
// format stay far below the fp32 range.  The scale-tile MFMA cannot give this
// class (an infinite d_x meets the zero k slots of the other sub-blocks), so
// the tile recomputes these outputs instead.  `flags` is LDS for `toks` ints.
// Reached only when the tile holds such a token; all threads take part.
__device__ __noinline__ void nonfinite_fixup(const uint8_t* __restrict__ W, float* __restrict__ Y, int64_t N,
                                             int64_t ldy_m, int64_t ldy_n, const int8_t* __restrict__ aqs,
                                             const uint32_t* __restrict__ ads, int64_t K, int64_t M, int64_t n0,
                                             int rows, int64_t m0, int toks, int* flags) {
    const int tid = threadIdx.x, nth = blockDim.x;
    const int64_t nb = K / QK8_1, bpr = K / QK_K;
    for (int t = tid; t < toks; t += nth) {
        int bad = 0;
        if (m0 + t < M)
            for (int64_t b = 0; b < nb; ++b)
                bad |= __builtin_isfinite(half_bits_to_float(ads[(m0 + t) * nb + b] & 0xFFFFu)) ? 0 : 1;
        flags[t] = bad;
    }
    __syncthreads();
    const uint32_t kv[4] = {KV0, KV1, KV2, KV3};
    auto kval = [&](uint32_t c) { return (int)(int8_t)(kv[c >> 2] >> (8 * (c & 3))); };
    for (int i = tid; i < toks * rows; i += nth) {
        const int t = i / rows, r = i % rows;
        const int64_t m = m0 + t, n = n0 + r;
        if (!flags[t] || m >= M || n >= N) continue;
        float y = 0.0f;
        for (int64_t kb = 0; kb < bpr; ++kb) {
            const uint8_t* blk = W + (n * bpr + kb) * BLOCK_BYTES;
            const uint32_t h0 = *reinterpret_cast<const uint32_t*>(blk), h1 = *reinterpret_cast<const uint32_t*>(blk + 4);
            const float dw = half_bits_to_float(h0 & 0xFFFFu);
            for (int s = 0; s < 8; ++s) {
                const float dx = half_bits_to_float(ads[m * nb + kb * 8 + s] & 0xFFFFu);
                if (__builtin_isfinite(dw) && __builtin_isfinite(dx)) continue;
                const int8_t* x = aqs + m * K + kb * QK_K + 32 * s;
                int sumi = 0;
                for (int j = 0; j < 16; ++j) {
                    const uint32_t q = blk[8 + 16 * s + j];
                    sumi += kval(q & 15u) * (int)x[j] + kval(q >> 4) * (int)x[j + 16];
                }
                y += (dw * dx) * (float)(sumi * (subblock_ls(h0, h1, s) - 32));
            }
        }
        Y[m * ldy_m + n * ldy_n] = y;
    }
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
                                         int64_t ldy_m, int tile0, const int8_t* __restrict__ aqs,
                                         const uint32_t* __restrict__ ahq,
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
    // for a non-finite d_x, so that no Inf meets a zero low half (0 * Inf);
    // such a token's outputs are recomputed at the end (nonfinite_fixup), and
    // nf records that this thread saw one among the tile's own tokens
    const bool own_token = tm < 32 * T && m0 + tm < M;
    bool nf = false;
    auto store_d = [&](v2u d, uint8_t* stage) {
        uint32_t* t = reinterpret_cast<uint32_t*>(stage + HStage<TOK>::t_off) + tm * 8 + ts;
        const float x0 = half_bits_to_float(d.x & 0xFFFFu), x1 = half_bits_to_float(d.y & 0xFFFFu);
        nf |= own_token && !(__builtin_isfinite(x0) && __builtin_isfinite(x1));
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
    const int any_nf = __syncthreads_or(nf ? 1 : 0);
#pragma unroll
    for (int j = 0; j < T; ++j) {
        if ((j < HALF) == (kh == 0)) {
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[j][e] += slot(kh ^ 1, j)[e * 64];
            store(acc[j], j);
        }
    }
    if (any_nf) {  // workgroup-uniform, and only for a token with a non-finite d_x
        __syncthreads();  // the reduction slots are read above; the fix-up reuses the LDS
        nonfinite_fixup(W, Y, N, ldy_m, ldy_n, aqs, ads, K, M, n0, 32 * RG, m0, 32 * T,
                        reinterpret_cast<int*>(&stages[0][0]));
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
__global__ __launch_bounds__(128 * RG) void gemm_f16_kernel(const GemmGroup grp, const int8_t* __restrict__ aqs,
                                                            const uint32_t* __restrict__ ahq,
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
    // the matrix of this tile, by scalar selects on the by-value descriptor
    // (no dynamic index into the argument block), from the logical tile index
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
        if (sg.T == 1) f16_tile<kDebug, 1, 2>(W, Y, N, ldy_m, tile0, aqs, ahq, ads, K, M, ldy_n, bx, by, smem, dbg);
        else f16_tile<kDebug, 2, 2>(W, Y, N, ldy_m, tile0, aqs, ahq, ads, K, M, ldy_n, bx, by, smem, dbg);
    } else {
        switch (sg.T) {
            case 1: f16_tile<kDebug, 1, 4>(W, Y, N, ldy_m, tile0, aqs, ahq, ads, K, M, ldy_n, bx, by, smem, dbg); break;
            case 2: f16_tile<kDebug, 2, 4>(W, Y, N, ldy_m, tile0, aqs, ahq, ads, K, M, ldy_n, bx, by, smem, dbg); break;
            case 3: f16_tile<kDebug, 3, 4>(W, Y, N, ldy_m, tile0, aqs, ahq, ads, K, M, ldy_n, bx, by, smem, dbg); break;
            default: f16_tile<kDebug, 4, 4>(W, Y, N, ldy_m, tile0, aqs, ahq, ads, K, M, ldy_n, bx, by, smem, dbg); break;
        }
    }
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
static hipError_t launch_f16_kernel(const GemmGroup& grp, int64_t row_tiles, const int8_t* aqs, const uint32_t* ahq,
                                    const uint32_t* ads,
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
        hipLaunchKernelGGL((gemm_f16_kernel<false, false, 2>), dim3((unsigned)wgs), dim3(256), 0, stream, g2, aqs, ahq,
                           ads, K, M, ldy_n, plan, dbg);
        return hipGetLastError();
    }
    const F16Plan plan = kDebug ? f16_plan_of({{row_tiles, 4}}, M) : f16_plan(row_tiles, M);
    const int wgs = plan.seg[F16_SEGS - 1].wg_end;
    if (wgs <= 0) return hipSuccess;
    hipLaunchKernelGGL((gemm_f16_kernel<kDebug, kGroup>), dim3((unsigned)wgs), dim3(H_THREADS), 0, stream, grp, aqs, ahq,
                       ads, K, M, ldy_n, plan, dbg);
    return hipGetLastError();
}

// The kernel addresses a tile's weight rows and tokens with 32-bit offsets
// (K below 2^24: far past any matrix of this format in use).
static bool f16_fits(int64_t K) {
    return (int64_t)H_BN * (K / QK_K) * BLOCK_BYTES < (1ll << 32) && (int64_t)H_BM * 2 * K < (1ll << 32);
}

hipError_t launch_gemm(const uint8_t* W, const int8_t* aqs, const uint32_t* ads, const uint32_t* ahq, float* Y,
                       int64_t K, int64_t N, int64_t M, int64_t ldy_m, int64_t ldy_n, int32_t* dbg,
                       hipStream_t stream) {
    clear_launch_error();
    if (!f16_fits(K)) return hipErrorInvalidConfiguration;
    GemmGroup grp{};
    grp.W[0] = W;
    grp.Y[0] = Y;
    grp.N[0] = N;
    grp.ldy_m[0] = ldy_m;
    const int64_t gx = (N + H_BN - 1) / H_BN;
    if (gx > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
    grp.tile_end[0] = (int)gx;
    return dbg ? launch_f16_kernel<true, false>(grp, gx, aqs, ahq, ads, K, M, ldy_n, dbg, stream)
               : launch_f16_kernel<false, false>(grp, gx, aqs, ahq, ads, K, M, ldy_n, dbg, stream);
}

// One launch for `count` matrices sharing K and the activations: the round
// planner sees the summed row tiles, so the small matrices fill CUs that the
// big ones' last round leaves idle.
hipError_t launch_gemm_group(int count, const uint8_t* const* W, float* const* Y, const int64_t* N, const int8_t* aqs,
                             const uint32_t* ads, const uint32_t* ahq, int64_t K, int64_t M, bool layout_mk,
                             hipStream_t stream) {
    clear_launch_error();
    if (count < 1 || count > GEMV_GROUP_MAX) return hipErrorInvalidValue;
    if (!f16_fits(K)) return hipErrorInvalidConfiguration;
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
    return launch_f16_kernel<false, true>(grp, tiles, aqs, ahq, ads, K, M, layout_mk ? 1 : M, nullptr, stream);
}

// One v_mfma_i32_32x32x32_i8 on a 32x32 A and B (k-contiguous rows), C row-major:
// pins the operand and result layout that the small-batch matrix-core GEMV uses.
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
