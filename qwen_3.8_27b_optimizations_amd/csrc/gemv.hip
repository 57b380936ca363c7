// gemv.hip -- IQ4_XS x Q8_1 GEMV / small-batch GEMV (1..8 activation columns)
// for gfx950, wave64.
//
// Semantics: vec_dot_iq4_xs_q8_1 (real_stock_dp4a_comparator.hip:145-166)
// summed over every 32-weight sub-block of a row (:325-360):
//   y[n] = sum_kb fp16(W.d) * fp16(ds.d) * (float)(sumi_kb * (ls_kb - 32)).
// The int32 sumi of every sub-block is exact (bit-identical to the
// reference); only the fp32 summation order differs.
//
// MI355X mapping (streaming kernel, gemv_lds_kernel).  On this path the
// VALU work per weight byte decides how well HBM streaming overlaps with
// compute, so the kernel is built to spend as few instructions per 16 bytes
// of weights as possible:
//   * lane l handles sub-block (l & 7) of super-block (l >> 3) of an
//     8-super-block "step": one dwordx4 per lane reads 1088 contiguous bytes
//     of a row per wave, straight from HBM;
//   * a work item is one row, or two adjacent rows when K/256 = 4 mod 8
//     (K = 5120, 17408): the two rows' super-blocks are contiguous, so a
//     2-row item is exactly (2K/256)/8 full steps and no lane idles;
//   * the Q8_1 activations (codes + fp32 d) sit in LDS, copied or quantised
//     once per workgroup; workgroups are persistent (about two per CU) and
//     walk a contiguous range of items;
//   * each wave keeps the next step's loads in flight while it computes the
//     current one; row sums are reduced with DPP, parked in LDS and written
//     once at the end, so no store sits inside the streaming loop;
//   * codebook decode: decode_codes_x (perm "specials", 11 ops / 8 codes).
// gemv_global_kernel is the fallback for shapes whose activations do not fit
// the LDS budget (large K with many columns): same arithmetic, activations
// read through L1/L2.
#include "iq4xs_device.h"
#include "iq4xs_internal.h"
#include "q8_1_block.h"

namespace iq4xs {

typedef uint32_t v2u __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- fallback
template <int C, bool kDebug>
__global__ __launch_bounds__(256) void gemv_global_kernel(const uint8_t* __restrict__ W,
                                                          const int8_t* __restrict__ aqs,
                                                          const uint32_t* __restrict__ ads, float* __restrict__ Y,
                                                          int64_t K, int64_t N, int64_t ldy_m, int64_t ldy_n,
                                                          int32_t* __restrict__ dbg) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= N) return;
    const int ib = lane & 7;
    const int slot = lane >> 3;
    const int64_t bpr = K / QK_K;
    const int64_t nb = K / QK8_1;
    const uint8_t* wrow = W + row * bpr * BLOCK_BYTES;
    float acc[C];
#pragma unroll
    for (int c = 0; c < C; ++c) acc[c] = 0.0f;
    for (int64_t b = slot; b < bpr; b += 8) {
        const uint8_t* hp = wrow + b * BLOCK_BYTES;
        const v2u h = *reinterpret_cast<const v2u*>(hp);
        const v4i w = *reinterpret_cast<const v4i_a8*>(hp + 8 + 16 * ib);
        const int ls = subblock_ls(h.x, h.y, ib) - 32;
        const float dw = half_bits_to_float(h.x & 0xFFFFu);
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) decode_codes_x((uint32_t)w[j], lo[j], hi[j]);
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const v4i* p = reinterpret_cast<const v4i*>(aqs + c * K + b * QK_K + ib * QK8_1);
            const v4i a0 = p[0], a1 = p[1];
            const float dx = half_bits_to_float(ads[c * nb + b * 8 + ib] & 0xFFFFu);
            int s = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                s = dot4(lo[j], (uint32_t)a0[j], s);
                s = dot4(hi[j], (uint32_t)a1[j], s);
            }
            s = __mul24(s, ls);
            acc[c] += (dw * dx) * (float)s;
            if (kDebug) dbg[((int64_t)c * N + row) * nb + b * 8 + ib] = s;
        }
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const float v = wave_sum_dpp(acc[c]);
        if (lane == 0) Y[c * ldy_m + row * ldy_n] = v;
    }
}

// ---------------------------------------------------------------- streaming kernel
// One step of one lane: the 16 qs bytes of its sub-block and the 8-byte header
// of its super-block.
struct StepRegs {
    v4i q;
    v2u h;
};

struct GemvGeom {
    int K, N, bpr, nb, U, n_items;
    size_t row_bytes;
};

template <int IR>
__device__ inline void load_step(StepRegs& s, const uint8_t* __restrict__ W, const GemvGeom& g, int item, int u,
                                 int slot, int ib) {
    int c = 8 * u + slot;                      // super-block index inside the item
    const int row0 = item * IR;
    if (IR == 1) {
        c = c < g.bpr ? c : g.bpr - 1;         // masked lanes re-read a valid block
    } else if (row0 + 1 >= g.N) {
        c = c < g.bpr ? c : c - g.bpr;         // odd N: the missing second row re-reads the first
    }
    const uint8_t* p = W + (size_t)row0 * g.row_bytes + (size_t)c * BLOCK_BYTES;
    s.h = *reinterpret_cast<const v2u*>(p);
    s.q = *reinterpret_cast<const v4i_a8*>(p + 8 + 16 * ib);
}

// acc[r][c] += contribution of one step.  `which` (wave-uniform): 0 = all lanes
// in row 0, 1 = all lanes in row 1, 2 = split at super-block bpr.
template <int C, int IR, bool kDebug>
__device__ inline void compute_step(const StepRegs& s, float (&acc)[IR][C], const int8_t* sq, const float* sdx,
                                    const GemvGeom& g, int item, int u, int slot, int ib, int32_t* __restrict__ dbg) {
    const int c = 8 * u + slot;
    int r = 0, b = c;
    if (IR == 2 && c >= g.bpr) {
        r = 1;
        b = c - g.bpr;
    }
    if (IR == 1 && c >= g.bpr) return;         // masked lane (only when bpr % 8 != 0)
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) decode_codes_x((uint32_t)s.q[j], lo[j], hi[j]);
    const int ls = subblock_ls(s.h.x, s.h.y, ib) - 32;
    const float dw = half_bits_to_float(s.h.x & 0xFFFFu);
#pragma unroll
    for (int cc = 0; cc < C; ++cc) {
        const v4i* p = reinterpret_cast<const v4i*>(sq + (size_t)cc * g.K + b * QK_K + ib * QK8_1);
        const v4i a0 = p[0], a1 = p[1];
        int sum = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            sum = dot4(lo[j], (uint32_t)a0[j], sum);
            sum = dot4(hi[j], (uint32_t)a1[j], sum);
        }
        sum = __mul24(sum, ls);
        const float t = (dw * sdx[cc * g.nb + b * 8 + ib]) * (float)sum;
        if (IR == 2) {
            acc[0][cc] += r ? 0.0f : t;
            acc[1][cc] += r ? t : 0.0f;
        } else {
            acc[0][cc] += t;
        }
        if (kDebug) {
            const int row = item * IR + r;
            if (row < g.N) dbg[((int64_t)cc * g.N + row) * g.nb + b * 8 + ib] = sum;
        }
    }
}

// Activations into LDS: codes [C][K] int8, d as fp32 [C][K/32].
__device__ inline void stage_activations(const int8_t* __restrict__ aqs, const uint32_t* __restrict__ ads, int C,
                                         int K, int8_t* sq, float* sdx, int tid, int nthreads) {
    const int n16 = C * K / 16;
    for (int i = tid; i < n16; i += nthreads)
        reinterpret_cast<v4i*>(sq)[i] = reinterpret_cast<const v4i*>(aqs)[i];
    const int nbs = C * (K / QK8_1);
    for (int i = tid; i < nbs; i += nthreads) sdx[i] = half_bits_to_float(ads[i] & 0xFFFFu);
}

// Fused prologue: quantise the fp32 activations (element (c, k) at
// X[c*sc + k*sk]) straight into LDS, eight lanes per block.  Only d is kept:
// the dot uses the fp16-truncated d exactly as the planar path does.
__device__ inline void quantize_to_lds(const float* __restrict__ X, int64_t sc, int64_t sk, int C, int K, int8_t* sq,
                                       float* sdx, int tid, int nthreads) {
    const int nb = K / QK8_1;
    const int tasks = C * nb * 8;  // nthreads is a multiple of 64: 8-lane groups stay whole
    for (int t = tid; t < tasks; t += nthreads) {
        const int blk = t >> 3, j = t & 7;
        const int cc = blk / nb, ib = blk - cc * nb;
        const float* p = X + cc * sc + (int64_t)(ib * QK8_1 + j) * sk;
        const Q8Block8 b = quantize_block8(p[0], p[8 * sk], p[16 * sk], p[24 * sk]);
        int8_t* o = sq + cc * K + ib * QK8_1 + j;
        o[0] = (int8_t)b.q0;
        o[8] = (int8_t)b.q1;
        o[16] = (int8_t)b.q2;
        o[24] = (int8_t)b.q3;
        if (j == 0) sdx[blk] = half_bits_to_float(b.ds & 0xFFFFu);
    }
}

template <int C, int IR, bool kDebug, bool kFuse>
__global__ __launch_bounds__(512) void gemv_lds_kernel(const uint8_t* __restrict__ W, const int8_t* __restrict__ aqs,
                                                       const uint32_t* __restrict__ ads,
                                                       const float* __restrict__ X, int64_t sc, int64_t sk,
                                                       float* __restrict__ Y, int K, int N, int64_t ldy_m,
                                                       int64_t ldy_n, int items_per_wg, int32_t* __restrict__ dbg) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    GemvGeom g;
    g.K = K;
    g.N = N;
    g.bpr = K / QK_K;
    g.nb = K / QK8_1;
    g.U = (IR == 2) ? (2 * g.bpr) / 8 : (g.bpr + 7) / 8;
    g.n_items = (N + IR - 1) / IR;
    g.row_bytes = (size_t)g.bpr * BLOCK_BYTES;
    int8_t* sq = reinterpret_cast<int8_t*>(lds);
    float* sdx = reinterpret_cast<float*>(lds + (size_t)C * K);
    float* sy = sdx + C * g.nb;                // [items_per_wg * IR][C]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int nwaves = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ib = lane & 7, slot = lane >> 3;
    const int item_begin = blockIdx.x * items_per_wg;
    const int item_end = min(g.n_items, item_begin + items_per_wg);

    // this wave's items: item_begin + wave, + nwaves, ...; steps: U per item
    int item = item_begin + wave;
    const int my_items = item < item_end ? (item_end - item + nwaves - 1) / nwaves : 0;
    const int total = my_items * g.U;

    StepRegs A, B;
    if (total > 0) load_step<IR>(A, W, g, item, 0, slot, ib);  // first loads fly during the prologue
    if (kFuse)
        quantize_to_lds(X, sc, sk, C, K, sq, sdx, tid, blockDim.x);
    else
        stage_activations(aqs, ads, C, K, sq, sdx, tid, blockDim.x);
    __syncthreads();

    float acc[IR][C];
#pragma unroll
    for (int r = 0; r < IR; ++r)
#pragma unroll
        for (int cc = 0; cc < C; ++cc) acc[r][cc] = 0.0f;

    int u = 0;
    auto finish_item = [&]() {
#pragma unroll
        for (int r = 0; r < IR; ++r) {
#pragma unroll
            for (int cc = 0; cc < C; ++cc) {
                const float v = wave_sum_dpp(acc[r][cc]);
                acc[r][cc] = 0.0f;
                if (lane == 0) sy[((item - item_begin) * IR + r) * C + cc] = v;
            }
        }
    };
    // next (item, u) of the stream, clamped to the last valid step
    auto advance = [&](int it, int uu, int& nit, int& nu) {
        nu = uu + 1;
        nit = it;
        if (nu == g.U) {
            nu = 0;
            nit = it + nwaves;
        }
        if (nit >= item_end) {
            nit = it;
            nu = uu;
        }
    };
    for (int step = 0; step < total; step += 2) {
        int nit, nu;
        advance(item, u, nit, nu);
        load_step<IR>(B, W, g, nit, nu, slot, ib);
        compute_step<C, IR, kDebug>(A, acc, sq, sdx, g, item, u, slot, ib, dbg);
        if (u == g.U - 1) finish_item();
        item = nit;
        u = nu;
        if (step + 1 >= total) break;
        advance(item, u, nit, nu);
        load_step<IR>(A, W, g, nit, nu, slot, ib);
        compute_step<C, IR, kDebug>(B, acc, sq, sdx, g, item, u, slot, ib, dbg);
        if (u == g.U - 1) finish_item();
        item = nit;
        u = nu;
    }
    __syncthreads();
    const int rows_here = min(N - item_begin * IR, items_per_wg * IR);
    for (int i = tid; i < rows_here * C; i += blockDim.x) {
        const int rr = i / C, cc = i - rr * C;
        Y[cc * ldy_m + (int64_t)(item_begin * IR + rr) * ldy_n] = sy[i];
    }
}

// ---------------------------------------------------------------- launchers
constexpr int GEMV_WAVES_PER_WG = 8;
constexpr size_t GEMV_LDS_BUDGET = 64 * 1024;

static int device_cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

template <int C, int IR>
static hipError_t launch_lds(const uint8_t* W, const int8_t* aqs, const uint32_t* ads, const float* X, int64_t sc,
                             int64_t sk, float* Y, int64_t K, int64_t N, int64_t ldy_m, int64_t ldy_n, int32_t* dbg,
                             hipStream_t stream) {
    const int64_t n_items = (N + IR - 1) / IR;
    const int64_t max_wgs = 2 * (int64_t)device_cu_count();
    int64_t wgs = (n_items + GEMV_WAVES_PER_WG - 1) / GEMV_WAVES_PER_WG;
    if (wgs > max_wgs) wgs = max_wgs;
    const int64_t items_per_wg = (n_items + wgs - 1) / wgs;
    wgs = (n_items + items_per_wg - 1) / items_per_wg;
    const size_t lds = (size_t)C * K + (size_t)C * (K / QK8_1) * 4 + (size_t)items_per_wg * IR * C * 4;
    if (lds > GEMV_LDS_BUDGET) return hipErrorNotSupported;
    const dim3 grid((unsigned)wgs), block(64 * GEMV_WAVES_PER_WG);
#define IQ4XS_LAUNCH_LDS(DBG, FUSE)                                                                              \
    hipLaunchKernelGGL((gemv_lds_kernel<C, IR, DBG, FUSE>), grid, block, lds, stream, W, aqs, ads, X, sc, sk, Y,  \
                       (int)K, (int)N, ldy_m, ldy_n, (int)items_per_wg, dbg)
    if (X != nullptr) {
        if (dbg) IQ4XS_LAUNCH_LDS(true, true); else IQ4XS_LAUNCH_LDS(false, true);
    } else {
        if (dbg) IQ4XS_LAUNCH_LDS(true, false); else IQ4XS_LAUNCH_LDS(false, false);
    }
#undef IQ4XS_LAUNCH_LDS
    return hipGetLastError();
}

// X == nullptr: planar Q8_1 activations (aqs, ads); otherwise fp32 X quantised
// in the prologue (fused; returns hipErrorNotSupported when it does not fit).
template <int C>
static hipError_t launch_cols(const uint8_t* W, const int8_t* aqs, const uint32_t* ads, const float* X, int64_t sc,
                              int64_t sk, float* Y, int64_t K, int64_t N, int64_t ldy_m, int64_t ldy_n, int32_t* dbg,
                              hipStream_t stream) {
    const int64_t bpr = K / QK_K;
    hipError_t err = hipErrorNotSupported;
    if (K <= (1 << 24) && N < (1 << 30)) {
        if (bpr % 8 == 4)
            err = launch_lds<C, 2>(W, aqs, ads, X, sc, sk, Y, K, N, ldy_m, ldy_n, dbg, stream);
        else
            err = launch_lds<C, 1>(W, aqs, ads, X, sc, sk, Y, K, N, ldy_m, ldy_n, dbg, stream);
    }
    if (err != hipErrorNotSupported || X != nullptr) return err;
    const int64_t grid = (N + 3) / 4;
    if (grid > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
    if (dbg)
        hipLaunchKernelGGL((gemv_global_kernel<C, true>), dim3((unsigned)grid), dim3(256), 0, stream, W, aqs, ads, Y,
                           K, N, ldy_m, ldy_n, dbg);
    else
        hipLaunchKernelGGL((gemv_global_kernel<C, false>), dim3((unsigned)grid), dim3(256), 0, stream, W, aqs, ads, Y,
                           K, N, ldy_m, ldy_n, dbg);
    return hipGetLastError();
}

static hipError_t dispatch_cols(const uint8_t* W, const int8_t* aqs, const uint32_t* ads, const float* X, int64_t sc,
                                int64_t sk, float* Y, int64_t K, int64_t N, int64_t M, int64_t ldy_m, int64_t ldy_n,
                                int32_t* dbg, hipStream_t stream) {
    switch (M) {
        case 1: return launch_cols<1>(W, aqs, ads, X, sc, sk, Y, K, N, ldy_m, ldy_n, dbg, stream);
        case 2: return launch_cols<2>(W, aqs, ads, X, sc, sk, Y, K, N, ldy_m, ldy_n, dbg, stream);
        case 3: return launch_cols<3>(W, aqs, ads, X, sc, sk, Y, K, N, ldy_m, ldy_n, dbg, stream);
        case 4: return launch_cols<4>(W, aqs, ads, X, sc, sk, Y, K, N, ldy_m, ldy_n, dbg, stream);
        case 5: return launch_cols<5>(W, aqs, ads, X, sc, sk, Y, K, N, ldy_m, ldy_n, dbg, stream);
        case 6: return launch_cols<6>(W, aqs, ads, X, sc, sk, Y, K, N, ldy_m, ldy_n, dbg, stream);
        case 7: return launch_cols<7>(W, aqs, ads, X, sc, sk, Y, K, N, ldy_m, ldy_n, dbg, stream);
        case 8: return launch_cols<8>(W, aqs, ads, X, sc, sk, Y, K, N, ldy_m, ldy_n, dbg, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv(const uint8_t* W, const int8_t* aqs, const uint32_t* ads, float* Y, int64_t K, int64_t N,
                       int64_t M, int64_t ldy_m, int64_t ldy_n, int32_t* dbg, hipStream_t stream) {
    return dispatch_cols(W, aqs, ads, nullptr, 0, 0, Y, K, N, M, ldy_m, ldy_n, dbg, stream);
}

hipError_t launch_gemv_fused(const uint8_t* W, const float* X, int64_t sc, int64_t sk, float* Y, int64_t K, int64_t N,
                             int64_t M, int64_t ldy_m, int64_t ldy_n, int32_t* dbg, hipStream_t stream) {
    return dispatch_cols(W, nullptr, nullptr, X, sc, sk, Y, K, N, M, ldy_m, ldy_n, dbg, stream);
}

}  // namespace iq4xs
