// gemv_mfma.hip -- small-batch IQ4_XS x Q8_1 GEMV (2 <= M <= 8 columns) on
// the gfx950 int8 matrix cores.
//
// Semantics: those of the GEMV / GEMM (real_stock_dp4a_comparator.hip:
// 68-166, 374-443): per 32-weight sub-block the exact int32 dot sumi of the
// IQ4_XS codes with the Q8_1 codes, scaled by fp16(d_w)*(ls-32) and the
// column's fp16 d.
//
// Why a second GEMV.  The dot4 GEMV spends VALU work per weight byte and per
// column, so from 4 columns on it is VALU-bound (bs = 8 ran at 1.35 TB/s).
// Here one v_mfma_i32_32x32x32_i8 takes 32 weight rows x 32 k of one
// sub-block against all columns at once (the A operand is the activations,
// one token per MFMA row; rows past M hold any token and only produce C rows
// that are never stored), so the VALU cost per weight byte no longer grows
// with M: decoding the codes into the B operand, then per useful output a
// convert, a scale product and a fused add.
//
// Mapping.  A workgroup of GM_WAVES (8 or 16) waves owns up to 32 weight rows
// (one MFMA block; rows past its own are masked); its waves take
// the super-blocks kb = wave, wave + GM_WAVES, ... (at any moment they stream
// GM_WAVES consecutive super-blocks of the same rows), each wave keeping one
// super-block of loads in flight while it computes the previous one.  Its
// loads are coalesced (each of the 4 weight loads covers the qs of 8 whole
// rows, the 2 activation loads a token's 256 codes per 8 lanes) and staged in
// LDS rows of the wave's own, from which the MFMA operands are read.  The
// MFMA sums over k, so any order of k that A and B share gives the same
// int32: lane l (half h = l >> 5) supplies weight row l & 31 with both
// nibbles of qs bytes 8h .. 8h+7 of the sub-block (sub-block weights
// 8h .. 8h+7 and 16+8h .. 16+8h+7), decoded in registers, and the A lanes the
// activation codes of the same 16 weights.  The C element e of lane l is
// token 8*(e>>2) + 4h + (e&3) of that row.  The token scales of a
// super-block ride in the activation ring (one ds word per lane) and are
// staged with its codes, so no workgroup-wide prologue or barrier precedes
// the stream (staging every column scale up front measured 3-12 % slower).
// The GM_WAVES partial sums of every output are added in LDS in wave order
// (deterministic).
#include "iq4xs_device.h"
#include "iq4xs_internal.h"

namespace iq4xs {

constexpr int GM_LDS_MAX = 160 * 1024;

constexpr int GM_AROW = 272;  // LDS row of one token's 256 codes, padded (bank spread)
constexpr int GM_WROW = 144;  // LDS row of one weight row's 128 qs bytes, padded
// per-wave staging bytes: weight rows, token rows, then the super-block's
// column scales [8 sub-blocks][8 tokens]
constexpr int GM_WAVE_LDS = 32 * GM_WROW + 8 * GM_AROW + 8 * 8 * 4;
// Register ring of weight super-blocks per wave (one in flight while one is
// computed); the activations, read by every workgroup and so L2-resident,
// have a ring of their own, also one super-block ahead.  Depths 3 and 4
// measured slower (more VGPRs, no better overlap).
constexpr int GM_RING = 2;

struct GmW {      // weights of one super-block (from HBM: the deep ring)
    v2u h;       // d, scales_h, scales_l of this lane's row's super-block
    v4i q[4];    // qs chunk (lane % 8) of rows lane/8 + 8i: 8 whole rows per load instruction
};
struct GmA {      // activations of one super-block (L2-resident: one ahead)
    v4i a[2];    // 32 of the super-block's activation codes: token lane/8, bytes 32*(lane%8) ..
    uint32_t ds; // Q8_1 ds word of token lane/8, sub-block lane%8
};

// The matrices of one launch (same K and activations): workgroups
// [tile_end[i-1], tile_end[i]) run matrix i, rows[i] rows each.  Entries past
// the group's count repeat its last matrix with tile_end = the grid size, so
// no workgroup selects them.
struct GmGroup {
    const uint8_t* W[GEMV_GROUP_MAX];
    float* Y[GEMV_GROUP_MAX];
    int64_t ldy_m[GEMV_GROUP_MAX];
    int N[GEMV_GROUP_MAX];
    int rows[GEMV_GROUP_MAX];
    int tile_end[GEMV_GROUP_MAX];
};

template <int GM_WAVES, bool kDebug>
__global__ __launch_bounds__(64 * GM_WAVES) void gemv_mfma_kernel(const GmGroup grp,
                                                                  const int8_t* __restrict__ aqs,
                                                                  const uint32_t* __restrict__ ads, int K, int M,
                                                                  int64_t ldy_n, int32_t* __restrict__ dbg) {
    constexpr int G = 1;  // M <= 8: tokens 4h + e of element e < 4
    extern __shared__ __attribute__((aligned(16))) float gm_lds[];
    // this workgroup's matrix: scalar selects on the by-value descriptor (a
    // dynamic index into it would go through scratch)
    const uint8_t* __restrict__ W = grp.W[0];
    float* __restrict__ Y = grp.Y[0];
    int64_t ldy_m = grp.ldy_m[0];
    int N = grp.N[0], rows = grp.rows[0], tile0 = 0;
#pragma unroll
    for (int i = 1; i < GEMV_GROUP_MAX; ++i) {
        if ((int)blockIdx.x >= grp.tile_end[i - 1]) {
            W = grp.W[i];
            Y = grp.Y[i];
            ldy_m = grp.ldy_m[i];
            N = grp.N[i];
            rows = grp.rows[i];
            tile0 = grp.tile_end[i - 1];
        }
    }
    const int bpr = K / QK_K, nb = K / QK8_1;
    float* red = gm_lds;                        // [GM_WAVES][4G][64] partial sums
    const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, col = lane & 31;
    uint8_t* swave = reinterpret_cast<uint8_t*>(red + GM_WAVES * 4 * G * 64) + (tid >> 6) * GM_WAVE_LDS;
    uint8_t* sw = swave;                                          // [32][144] qs of the 32 rows
    int8_t* sact = reinterpret_cast<int8_t*>(swave + 32 * GM_WROW);  // [8][272] activations
    const int wave = tid >> 6;
    const int r0 = ((int)blockIdx.x - tile0) * rows;
    const int nrow = min(rows, N - r0);  // this workgroup's rows (1..32; MFMA rows past them are masked)
    // Global loads are 32-bit lane offsets from workgroup-uniform bases (a
    // 32-row block spans 32 * K/256 * 136 bytes), which keeps the load ring
    // in VGPRs.  MFMA rows past nrow are clamped to its last row (a repeat
    // of bytes already loaded, so no extra HBM traffic): computed, never stored.
    const uint32_t row_bytes = (uint32_t)bpr * BLOCK_BYTES;
    const uint8_t* wbase = W + (size_t)r0 * row_bytes;
    const uint32_t off_h = (uint32_t)min(col, nrow - 1) * row_bytes;     // this lane's row (header)
    uint32_t off_q[4];                                                    // rows lane/8 + 8i, qs chunk lane%8
#pragma unroll
    for (int i = 0; i < 4; ++i)
        off_q[i] = (uint32_t)min((lane >> 3) + 8 * i, nrow - 1) * row_bytes + 8 + 16 * (lane & 7);
    uint8_t* wwrite = sw + (lane >> 3) * GM_WROW + 16 * (lane & 7);
    const uint8_t* wread = sw + col * GM_WROW + 8 * h;
    // this lane's share of a super-block's activations, and its MFMA A row in LDS
    const uint32_t off_a = (uint32_t)min(lane >> 3, M - 1) * (uint32_t)K + 32 * (lane & 7);
    int8_t* awrite = sact + (lane >> 3) * GM_AROW + 32 * (lane & 7);
    const int8_t* aread = sact + min(col, M - 1) * GM_AROW + 8 * h;
    // the current super-block's column scales, [sub-block][token] (0 past M),
    // and this lane's ds word in every super-block: token lane/8, sub-block lane%8
    float* sdx = reinterpret_cast<float*>(sact + 8 * GM_AROW);
    const uint32_t off_d = (uint32_t)min(lane >> 3, M - 1) * (uint32_t)nb + (lane & 7);

    const int my_n = wave < bpr ? (bpr - wave + GM_WAVES - 1) / GM_WAVES : 0;
    auto load_w = [&](GmW& p, int kb) {
        const uint8_t* wk = wbase + (size_t)kb * BLOCK_BYTES;   // uniform
        p.h = *reinterpret_cast<const v2u*>(wk + off_h);
#pragma unroll
        for (int i = 0; i < 4; ++i) p.q[i] = *reinterpret_cast<const v4i_a8*>(wk + off_q[i]);
    };
    auto load_a = [&](GmA& p, int kb) {
        const int8_t* ak = aqs + (size_t)kb * QK_K;               // uniform
        p.a[0] = *reinterpret_cast<const v4i*>(ak + off_a);
        p.a[1] = *reinterpret_cast<const v4i*>(ak + off_a + 16);
        p.ds = ads[(size_t)kb * 8 + off_d];
    };

    float acc[4 * G];
#pragma unroll
    for (int e = 0; e < 4 * G; ++e) acc[e] = 0.0f;
    auto compute = [&](const GmW& p, const GmA& pa, int kb) {
        // the wave's own LDS rows: written here, read below by other lanes of
        // the same wave (LDS operations of one wave complete in order; the
        // previous super-block's reads were issued before these writes)
        *reinterpret_cast<v4i*>(awrite) = pa.a[0];
        *reinterpret_cast<v4i*>(awrite + 16) = pa.a[1];
        sdx[(lane & 7) * 8 + (lane >> 3)] = (lane >> 3) < M ? half_bits_to_float(pa.ds & 0xFFFFu) : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<v4i*>(wwrite + 8 * i * GM_WROW) = p.q[i];
        const float dw = half_bits_to_float(p.h.x & 0xFFFFu);
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            uint32_t lo0, hi0, lo1, hi1;
            const v2u q = *reinterpret_cast<const v2u*>(wread + 16 * s);
            decode_codes_x(q.x, lo0, hi0);
            decode_codes_x(q.y, lo1, hi1);
            const v4i b = v4i{(int)lo0, (int)lo1, (int)hi0, (int)hi1};
            const v2u a0 = *reinterpret_cast<const v2u*>(aread + 32 * s);
            const v2u a1 = *reinterpret_cast<const v2u*>(aread + 32 * s + 16);
            const v4i a = v4i{(int)a0.x, (int)a0.y, (int)a1.x, (int)a1.y};
            const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, v16i{}, 0, 0, 0);
            const int ls = subblock_ls(p.h.x, p.h.y, s) - 32;
            const float sa = dw * (float)ls;
            const float* bxp = sdx + s * 8 + 4 * h;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const v4f bx = *reinterpret_cast<const v4f*>(bxp + 8 * g);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int e = 4 * g + j;
                    acc[e] = __builtin_fmaf((float)c[e], sa * bx[j], acc[e]);
                    if (kDebug) {
                        const int t = 8 * g + 4 * h + j;
                        if (t < M && col < nrow) dbg[((size_t)t * N + r0 + col) * nb + kb * 8 + s] = c[e] * ls;
                    }
                }
            }
        }
    };
    // ring of GM_RING super-blocks with constant indices (unrolled by its
    // depth); every load is unconditional (past this wave's last super-block
    // it repeats that one)
    // the loop is unrolled by 2 * GM_RING so that both rings have constant
    // indices (registers, not scratch)
    constexpr int UNR = 2 * GM_RING;
    GmW wb[GM_RING];
    GmA ab[2];
    if (my_n > 0) {
#pragma unroll
        for (int d = 0; d < GM_RING - 1; ++d) load_w(wb[d], wave + GM_WAVES * min(d, my_n - 1));
        load_a(ab[0], wave);
    }
    for (int i0 = 0; i0 < my_n; i0 += UNR) {
#pragma unroll
        for (int d = 0; d < UNR; ++d) {
            const int i = i0 + d;
            if (i0 + d >= my_n && d > 0) break;  // uniform: no loads past the last round's end
            load_w(wb[(d + GM_RING - 1) % GM_RING], wave + GM_WAVES * min(i + GM_RING - 1, my_n - 1));
            load_a(ab[(d + 1) % 2], wave + GM_WAVES * min(i + 1, my_n - 1));
            if (i < my_n) compute(wb[d % GM_RING], ab[d % 2], wave + GM_WAVES * i);
        }
    }
#pragma unroll
    for (int e = 0; e < 4 * G; ++e) red[(wave * 4 * G + e) * 64 + lane] = acc[e];
    __syncthreads();
    if (wave == 0 && col < nrow) {
#pragma unroll
        for (int e = 0; e < 4 * G; ++e) {
            float v = red[e * 64 + lane];
#pragma unroll
            for (int w = 1; w < GM_WAVES; ++w) v += red[(w * 4 * G + e) * 64 + lane];
            const int t = 8 * (e >> 2) + 4 * h + (e & 3);
            if (t < M) Y[t * ldy_m + (int64_t)(r0 + col) * ldy_n] = v;
        }
    }
}

// Workgroups and rows per workgroup of one matrix.  The wave count fixes each
// row's fp32 summation order; the rows per workgroup only balance the grid (a
// row's arithmetic does not depend on them).
struct GmPlan {
    int waves, rows;
};

static GmPlan gm_plan(int64_t N) {
    // Parallelism comes from splitting K over the waves of a row block: with
    // fewer 32-row blocks than two per CU, 16 waves each (measured: q, o and
    // down 5-15 % faster), otherwise 8 (gate/up: 16 would leave fewer
    // workgroups resident per CU).  With 16 waves the rows per workgroup (at
    // most 32, the MFMA's) are chosen so that every CU gets the same number
    // of workgroups: N = 5120 takes 20 rows on 256 CUs instead of 160 blocks
    // of 32 that leave 96 CUs idle (bs = 8: down 21.3 -> 18.4-19.5 us, o
    // unchanged).  Each workgroup decodes all 32 MFMA rows whatever it keeps,
    // so the 8-wave shapes stay at 32 rows (gate with 17-row workgroups, 4
    // per CU instead of 2.125: 18.9 -> 21.5 us).
    //
    // The wave count is chosen from the shape alone, against MI355X's 256
    // CUs, so a device or partition with another CU count gives the same
    // bits; the rows per workgroup use the device's own CU count.
    constexpr int64_t kWaveChoiceCus = 256;
    const int64_t cus = device_cu_count();
    if ((N + 31) / 32 < 2 * kWaveChoiceCus) {
        const int64_t k = (N + 32 * cus - 1) / (32 * cus);
        // at least 8 rows: narrow matrices (k/v, N = 1024, at 8 columns)
        // measured 6.60 us with 8-row workgroups against 6.99 with 4
        const int64_t rows = (N + cus * k - 1) / (cus * k);
        return {16, (int)(rows < 8 ? 8 : rows)};
    }
    return {8, 32};
}

template <int WAVES>
static hipError_t launch_gm(const GmGroup& grp, int64_t wgs, const int8_t* aqs, const uint32_t* ads, int64_t K,
                            int64_t M, int64_t ldy_n, int32_t* dbg, hipStream_t stream) {
    const size_t lds = (size_t)WAVES * 4 * 64 * sizeof(float) + (size_t)WAVES * GM_WAVE_LDS;
    if (lds > GM_LDS_MAX) return hipErrorNotSupported;
    if (lds > 64 * 1024) {  // beyond the default dynamic-LDS limit of a launch
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemv_mfma_kernel<WAVES, false>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, GM_LDS_MAX);
        if (e == hipSuccess)
            e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemv_mfma_kernel<WAVES, true>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, GM_LDS_MAX);
        if (e != hipSuccess) return e;
    }
    const dim3 grid((unsigned)wgs), block(64 * WAVES);
    if (dbg)
        hipLaunchKernelGGL((gemv_mfma_kernel<WAVES, true>), grid, block, lds, stream, grp, aqs, ads, (int)K, (int)M,
                           ldy_n, dbg);
    else
        hipLaunchKernelGGL((gemv_mfma_kernel<WAVES, false>), grid, block, lds, stream, grp, aqs, ads, (int)K, (int)M,
                           ldy_n, dbg);
    return hipGetLastError();
}

hipError_t launch_gemv_mfma_group(int count, const uint8_t* const* W, float* const* Y, const int64_t* N,
                                  const int64_t* ldy_m, const int8_t* aqs, const uint32_t* ads, int64_t K,
                                  int64_t M, int64_t ldy_n, int32_t* dbg, hipStream_t stream) {
    clear_launch_error();
    if (count < 1 || count > GEMV_GROUP_MAX || (dbg && count != 1)) return hipErrorInvalidValue;
    if (M < 1 || M > 8 || K % QK_K || K >= (1 << 24)) return hipErrorNotSupported;
    // the kernel's 32-bit load offsets span one 32-row block and 8 token rows
    if ((int64_t)32 * (K / QK_K) * BLOCK_BYTES >= ((int64_t)1 << 31) || (int64_t)8 * K >= ((int64_t)1 << 31))
        return hipErrorNotSupported;
    GmGroup grp{};
    int64_t wgs = 0;
    int waves = 0;
    for (int i = 0; i < GEMV_GROUP_MAX; ++i) {
        const int j = i < count ? i : count - 1;
        if (N[j] < 1 || N[j] >= (1 << 30)) return hipErrorNotSupported;
        const GmPlan plan = gm_plan(N[j]);
        if (i == 0) waves = plan.waves;
        if (plan.waves != waves) return hipErrorNotSupported;  // one wave count per launch
        if (i < count) wgs += (N[j] + plan.rows - 1) / plan.rows;
        if (wgs > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
        grp.W[i] = W[j];
        grp.Y[i] = Y[j];
        grp.ldy_m[i] = ldy_m[j];
        grp.N[i] = (int)N[j];
        grp.rows[i] = plan.rows;
        grp.tile_end[i] = (int)wgs;
    }
    return waves == 16 ? launch_gm<16>(grp, wgs, aqs, ads, K, M, ldy_n, dbg, stream)
                       : launch_gm<8>(grp, wgs, aqs, ads, K, M, ldy_n, dbg, stream);
}

int gemv_mfma_waves(int64_t N) { return gm_plan(N).waves; }

hipError_t launch_gemv_mfma(const uint8_t* W, const int8_t* aqs, const uint32_t* ads, float* Y, int64_t K,
                            int64_t N, int64_t M, int64_t ldy_m, int64_t ldy_n, int32_t* dbg, hipStream_t stream) {
    return launch_gemv_mfma_group(1, &W, &Y, &N, &ldy_m, aqs, ads, K, M, ldy_n, dbg, stream);
}

}  // namespace iq4xs
