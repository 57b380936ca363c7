// gemv.hip -- IQ4_XS x Q8_1 GEMV / small-batch GEMV (1..8 activation columns)
// for gfx950, wave64.
//
// Semantics: vec_dot_iq4_xs_q8_1 (real_stock_dp4a_comparator.hip:145-166)
// summed over every 32-weight sub-block of a row (:325-360):
//   y[n] = sum_kb fp16(W.d) * fp16(ds.d) * (float)(sumi_kb * (ls_kb - 32)).
// The int32 sumi of every sub-block is exact (bit-identical to the
// reference); only the fp32 summation order differs.
//
// MI355X mapping.  The unit of work is a "step": 8 consecutive 136-byte
// super-blocks (1088 B).  Lane l of a wave handles sub-block (l & 7) of
// super-block (l >> 3): one 16-byte load of codes plus the 8-byte block header
// per lane.  The codebook decode is decode_codes_x (v_perm "specials", 11 ops
// per 8 codes), the integer dot is v_dot4_i32_i8, and activations (codes + d)
// are read from LDS.
//   gemv_tile_kernel   (default, K >= 2048): short-lived workgroups that own a
//       few whole rows; waves interleave the tile's steps, so the grid sweeps
//       the matrix in address order; a ring of D register buffers keeps D-1
//       steps in flight during compute; super-block partials meet in LDS and
//       rows are summed in a fixed order.  Its prologue can also quantise
//       fp32 activations (kFuse) or run the RMS-norm producer on one column
//       (kRms, grouped launches) straight into its LDS operand.
//   gemv_flat_kernel   (when the tile's LDS would not fit, e.g. 8 columns at
//       K = 5120): each wave streams one contiguous range of steps and reduces
//       a row whenever it ends (DPP), row pieces meet in LDS.
//   gemv_lds_kernel    (K < 2048): one or two rows per work item.
//   gemv_global_kernel (activations too large for LDS): activations read
//       through L1/L2.
// Environment overrides for tuning (IQ4XS_GEMV_*) are read once per process.
#include <atomic>
#include <numeric>
#include <stdlib.h>

#include "act_device.h"
#include "iq4xs_device.h"
#include "iq4xs_internal.h"
#include "q8_1_block.h"
#include "rms_device.h"

namespace iq4xs {


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

// Activations into LDS: codes [C][K] int8, d as fp32 [C][K/32].  When they
// fit two rounds of code loads and one of d loads, all three loads are
// issued before the first wait (clamped indices, unconditional), so the d
// words cost no second L2 round trip after the codes (measured: -0.08 us
// per launch of the bs=1 tile GEMV on prequantised activations, ~1 %).
__device__ inline void stage_activations(const int8_t* __restrict__ aqs, const uint32_t* __restrict__ ads, int C,
                                         int K, int8_t* sq, float* sdx, int tid, int nthreads) {
    const int n16 = C * K / 16;
    const int nbs = C * (K / QK8_1);
    const v4i* src = reinterpret_cast<const v4i*>(aqs);
    v4i* dst = reinterpret_cast<v4i*>(sq);
    if (n16 <= 2 * nthreads && nbs <= nthreads) {
        const v4i c0 = src[min(tid, n16 - 1)];
        const v4i c1 = src[min(tid + nthreads, n16 - 1)];
        const uint32_t d = ads[min(tid, nbs - 1)];
        if (tid < n16) dst[tid] = c0;
        if (tid + nthreads < n16) dst[tid + nthreads] = c1;
        if (tid < nbs) sdx[tid] = half_bits_to_float(d & 0xFFFFu);
        return;
    }
    for (int i = tid; i < n16; i += nthreads) dst[i] = src[i];
    for (int i = tid; i < nbs; i += nthreads) sdx[i] = half_bits_to_float(ads[i] & 0xFFFFu);
}

// Single-column fused prologue in two halves, so that the x loads can be
// issued before the weight prefetch and the quantisation + LDS writes after
// it (vmcnt retires in order: x loaded after the weights would wait for
// them).  Loads are unconditional (index clamped): loads inside divergent
// branches make the compiler's wait counts conservative, so every round is
// issued: two rounds cover K <= 8 * threads (8192 for the 16-wave tile, the
// fused bound), and fewer idle rounds keep the prologue short: four rounds,
// two or more of them repeats at K <= 8192, measured 2 % slower on the bs=1
// decode step.  Needs K/4 <= 2 * threads (longer rows take quantize_to_lds).
constexpr int FUSED_ROUNDS = 2;
constexpr int FUSED_VEC_ROUNDS_LONG = 5;  // the vector prologue up to K = 20480
struct FusedRegs {
    float x[FUSED_ROUNDS][4];
};

__device__ inline void fused_load(FusedRegs& r, const float* __restrict__ X, int64_t sk, int tasks, int tid,
                                  int nthreads) {
#pragma unroll
    for (int u = 0; u < FUSED_ROUNDS; ++u) {
        const int t = min(tid + u * nthreads, tasks - 1);  // clamped: the load is unconditional
        const float* p = X + (int64_t)((t >> 3) * QK8_1 + q8_lane_elem(t & 7)) * sk;
        r.x[u][0] = p[0];
        r.x[u][1] = p[8 * sk];
        r.x[u][2] = p[16 * sk];
        r.x[u][3] = p[24 * sk];
    }
}

__device__ inline void fused_store(const FusedRegs& r, int8_t* sq, float* sdx, int tasks, int tid, int nthreads) {
#pragma unroll
    for (int u = 0; u < FUSED_ROUNDS; ++u) {
        const int t = tid + u * nthreads;
        if (t < tasks) {
            const int ib = t >> 3, j = q8_lane_elem(t & 7);
            const Q8Block8 b = quantize_block8(r.x[u][0], r.x[u][1], r.x[u][2], r.x[u][3]);
            int8_t* o = sq + ib * QK8_1 + j;
            o[0] = (int8_t)b.q0;
            o[8] = (int8_t)b.q1;
            o[16] = (int8_t)b.q2;
            o[24] = (int8_t)b.q3;
            if (j == 0) sdx[ib] = half_bits_to_float(b.ds & 0xFFFFu);
        }
    }
}

// The same prologue for a 16-byte aligned column with unit stride: lane t of
// an 8-lane group holds elements 4t .. 4t+3 of its block (one 16-byte load;
// a wave's load covers 1 KB of x, against 64 lines touched by the strided
// form), amax by three DPP steps over the group (max is exact in any order),
// then the d and codes of quantize_block8 -- the same bits.
template <int ROUNDS>
struct FusedVecRegs {
    v4f x[ROUNDS];
};

template <int ROUNDS>
__device__ inline void fused_load_vec(FusedVecRegs<ROUNDS>& r, const float* __restrict__ X, int tasks, int tid,
                                      int nthreads) {
#pragma unroll
    for (int u = 0; u < ROUNDS; ++u)
        r.x[u] = *reinterpret_cast<const v4f*>(X + 4 * min(tid + u * nthreads, tasks - 1));  // clamped
}

template <int ROUNDS>
__device__ inline void fused_store_vec(const FusedVecRegs<ROUNDS>& r, int8_t* sq, float* sdx, int tasks, int tid,
                                       int nthreads) {
#pragma unroll
    for (int u = 0; u < ROUNDS; ++u) {
        const int t = tid + u * nthreads;
        if (t < tasks) {  // tasks % 64 == 0: whole 8-lane groups and waves
            const v4f x = r.x[u];
            float a = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
            a = fmaxf(a, dpp_f32<0xB1>(a));   // quad_perm [1,0,3,2]
            a = fmaxf(a, dpp_f32<0x4E>(a));   // quad_perm [2,3,0,1]
            a = fmaxf(a, dpp_f32<0x141>(a));  // row_half_mirror: lane L <-> 7 - L of the group
            const float d = div127(a);
            const float xs[4] = {x[0], x[1], x[2], x[3]};
            int q[4];
            round_codes(xs, a, d, q);
            *reinterpret_cast<uint32_t*>(sq + 4 * t) = pack_codes4(q[0], q[1], q[2], q[3]);
            if ((t & 7) == 0) sdx[t >> 3] = half_bits_to_float(float_to_half_bits_rtz(d));
        }
    }
}

// Fused prologue: quantise the fp32 activations (element (c, k) at
// X[c*sc + k*sk]) straight into LDS, eight lanes per block.  Only d is kept:
// the dot uses the fp16-truncated d exactly as the planar path does.  Loads of
// up to four rounds are issued before any of them is used, so the prologue
// costs about one memory latency rather than one per round.
template <int C>
__device__ inline void quantize_to_lds(const float* __restrict__ X, int64_t sc, int64_t sk, int K, int8_t* sq,
                                       float* sdx, int tid, int nthreads) {
    constexpr int U = 4;
    const int nb = K / QK8_1;
    const int tasks = nb * 8;  // per column; a multiple of 64 (K % 256 == 0): 8-lane groups and waves stay whole
#pragma unroll
    for (int cc = 0; cc < C; ++cc) {
        const float* Xc = X + cc * sc;
        for (int t0 = tid; t0 < tasks; t0 += U * nthreads) {
            float x[U][4];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int t = t0 + u * nthreads;
                if (t < tasks) {
                    const float* p = Xc + (int64_t)((t >> 3) * QK8_1 + q8_lane_elem(t & 7)) * sk;
                    x[u][0] = p[0];
                    x[u][1] = p[8 * sk];
                    x[u][2] = p[16 * sk];
                    x[u][3] = p[24 * sk];
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int t = t0 + u * nthreads;
                if (t < tasks) {
                    const int ib = t >> 3, j = q8_lane_elem(t & 7);
                    const Q8Block8 b = quantize_block8(x[u][0], x[u][1], x[u][2], x[u][3]);
                    int8_t* o = sq + cc * K + ib * QK8_1 + j;
                    o[0] = (int8_t)b.q0;
                    o[8] = (int8_t)b.q1;
                    o[16] = (int8_t)b.q2;
                    o[24] = (int8_t)b.q3;
                    if (j == 0) sdx[cc * nb + ib] = half_bits_to_float(b.ds & 0xFFFFu);
                }
            }
        }
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
        quantize_to_lds<C>(X, sc, sk, K, sq, sdx, tid, blockDim.x);
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

// ---------------------------------------------------------------- flat-stream kernel
// The weight matrix is one contiguous array of N*bpr super-blocks.  A
// workgroup owns rows [r0, r0 + rows_per_wg) (r0*bpr a multiple of 8, so its
// range starts on a step boundary); its steps of 8 super-blocks are split into
// equal contiguous ranges, one per wave, whatever the row length.  A wave
// streams its range through a ring of D register buffers (each reloaded right
// after it is consumed, so D-1 steps stay in flight during compute), keeps one
// fp32 accumulator per lane and column, and reduces it whenever its current
// row ends (a row may end inside a step: lanes past the end start the next
// row).  Row pieces of neighbouring waves meet in LDS and are summed there in
// wave order, so the result does not depend on timing.
constexpr int FLAT_WAVES = 8;

template <int C>
__device__ inline void flat_flush(float (&acc)[C], float* part, int wave, int J, int j, int lane) {
#pragma unroll
    for (int cc = 0; cc < C; ++cc) {
        const float v = wave_sum_dpp(acc[cc]);
        if (lane == 0) part[(wave * J + j) * C + cc] = v;
    }
}

template <int C, int D, bool kDebug, bool kFuse>
__global__ __launch_bounds__(64 * FLAT_WAVES) void gemv_flat_kernel(
    const uint8_t* __restrict__ W, const int8_t* __restrict__ aqs, const uint32_t* __restrict__ ads,
    const float* __restrict__ X, int64_t sc, int64_t sk, float* __restrict__ Y, int K, int N, int64_t ldy_m,
    int64_t ldy_n, int rows_per_wg, int J, int32_t* __restrict__ dbg) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int bpr = K / QK_K, nb = K / QK8_1;
    int8_t* sq = reinterpret_cast<int8_t*>(lds);
    float* sdx = reinterpret_cast<float*>(lds + (size_t)C * K);
    float* part = sdx + C * nb;                 // [FLAT_WAVES][J][C]
    int* wrows = reinterpret_cast<int*>(part + FLAT_WAVES * J * C);  // [FLAT_WAVES][2]: first row, count

    const int tid = threadIdx.x;
    const int lane = tid & 63, slot = lane >> 3, ib = lane & 7;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r0 = blockIdx.x * rows_per_wg;
    const int nrows = min(rows_per_wg, N - r0);
    const int n_sb = nrows * bpr;
    const int n_steps = (n_sb + 7) >> 3;
    const int q = n_steps / FLAT_WAVES, rem = n_steps - q * FLAT_WAVES;
    const int s_a = wave * q + min(wave, rem);
    const int s_b = s_a + q + (wave < rem ? 1 : 0);
    const uint8_t* Wg = W + (size_t)r0 * bpr * BLOCK_BYTES;

    // Loads of step s (clamped into the workgroup's range; clamped lanes are
    // never accumulated).
    // Step s (0 <= s < n_steps) starts at the wave-uniform address
    // Wg + s*1088; each lane adds its constant offset.  Only the workgroup's
    // last step can be ragged: there lanes past the end re-read the last
    // super-block and are not accumulated.
    const int last_step = n_steps - 1;
    const int last_slot = (n_sb - 1) - 8 * last_step;
    const uint32_t off_n = (uint32_t)slot * BLOCK_BYTES;
    const uint32_t off_l = (uint32_t)min(slot, last_slot) * BLOCK_BYTES;
    const uint32_t off_q = 16u * (uint32_t)ib;
    auto load = [&](StepRegs& r, int s) {
        const uint8_t* base = Wg + (size_t)s * (8 * BLOCK_BYTES);  // scalar
        const uint32_t o = s == last_step ? off_l : off_n;         // lane offset
        r.h = *reinterpret_cast<const v2u*>(base + o);
        r.q = *reinterpret_cast<const v4i_a8*>(base + (o + off_q) + 8);
    };

    // The first D-1 steps of weights fly while the activations are staged
    // (both latencies overlap; vmcnt retires in order, so the staging waits
    // for these loads as well -- keep D small).
    StepRegs buf[D];
    if (s_a < s_b) {
#pragma unroll
        for (int d = 0; d < D - 1; ++d) load(buf[d], min(s_a + d, s_b - 1));
    }
    if (kFuse)
        quantize_to_lds<C>(X, sc, sk, K, sq, sdx, tid, blockDim.x);
    else
        stage_activations(aqs, ads, C, K, sq, sdx, tid, blockDim.x);
    __syncthreads();

    float acc[C];
#pragma unroll
    for (int cc = 0; cc < C; ++cc) acc[cc] = 0.0f;
    const int R_first = (8 * s_a) / bpr;
    int R = R_first;                 // current row, relative to r0 (wave-uniform)
    int row_end = (R + 1) * bpr;     // first super-block past row R
    const int sh_lo = 4 * ib, sh_hi = 16 + 2 * ib;

    auto compute = [&](const StepRegs& cur, int s) {
        const int sb = 8 * s + slot;
        const bool valid = s != last_step || slot <= last_slot;
        const bool nxt = sb >= row_end;     // lane already in row R+1
        // sub-block index inside the lane's row
        const int a_idx = 8 * (8 * s - (row_end - bpr)) + lane - (nxt ? nb : 0);
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) decode_codes_x((uint32_t)cur.q[j], lo[j], hi[j]);
        const int ls = (int)(((cur.h.y >> sh_lo) & 0xFu) | (((cur.h.x >> sh_hi) & 0x3u) << 4)) - 32;
        const float dw = half_bits_to_float(cur.h.x & 0xFFFFu);
        float t[C];
#pragma unroll
        for (int cc = 0; cc < C; ++cc) {
            const v4i* pa = reinterpret_cast<const v4i*>(sq + cc * K + a_idx * QK8_1);
            const v4i a0 = pa[0], a1 = pa[1];
            int sum = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                sum = dot4(lo[j], (uint32_t)a0[j], sum);
                sum = dot4(hi[j], (uint32_t)a1[j], sum);
            }
            sum = __mul24(sum, ls);
            t[cc] = valid ? (dw * sdx[cc * nb + a_idx]) * (float)sum : 0.0f;
            if (kDebug && valid) dbg[((int64_t)cc * N + r0 + R + (nxt ? 1 : 0)) * nb + a_idx] = sum;
        }
        if (8 * s + 8 < row_end) {
#pragma unroll
            for (int cc = 0; cc < C; ++cc) acc[cc] += t[cc];
        } else {                            // row R ends in this step
#pragma unroll
            for (int cc = 0; cc < C; ++cc) acc[cc] += nxt ? 0.0f : t[cc];
            flat_flush<C>(acc, part, wave, J, R - R_first, lane);
#pragma unroll
            for (int cc = 0; cc < C; ++cc) acc[cc] = nxt ? t[cc] : 0.0f;
            ++R;
            row_end += bpr;
        }
    };
    // Sub-step d first refills the buffer consumed by sub-step d-1 (step
    // s+d+D-1), then computes step s+d: D-1 steps are in flight during every
    // compute.  Loads are unconditional (clamped), so the wait counts stay
    // exact across the back edge; only the compute of steps past the end is
    // skipped.  One copy of the body per ring slot keeps the code small: with
    // a handful of steps per wave, instruction fetch is on the critical path.
    for (int s = s_a; s < s_b; s += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            load(buf[(d + D - 1) % D], min(s + d + D - 1, s_b - 1));
            if (s + d < s_b) compute(buf[d], s + d);
        }
    }
    int count = R - R_first;
    if (s_a < s_b && R * bpr < min(8 * s_b, n_sb)) {  // unfinished row piece
        flat_flush<C>(acc, part, wave, J, R - R_first, lane);
        ++count;
    }
    if (lane == 0) {
        wrows[2 * wave] = R_first;
        wrows[2 * wave + 1] = s_a < s_b ? count : 0;
    }
    __syncthreads();
    // Branch-free combine: every wave's piece of row rl (clamped index, masked
    // value), summed in wave order.  All LDS reads issue back to back.
    int f[FLAT_WAVES], n[FLAT_WAVES];
#pragma unroll
    for (int w = 0; w < FLAT_WAVES; ++w) {
        f[w] = wrows[2 * w];
        n[w] = wrows[2 * w + 1];
    }
    for (int rl = tid; rl < nrows; rl += blockDim.x) {
#pragma unroll
        for (int cc = 0; cc < C; ++cc) {
            float v = 0.0f;
#pragma unroll
            for (int w = 0; w < FLAT_WAVES; ++w) {
                const int j = rl - f[w];
                const bool in = j >= 0 && j < n[w];
                const float pv = part[(w * J + (in ? j : 0)) * C + cc];
                v += in ? pv : 0.0f;
            }
            Y[cc * ldy_m + (int64_t)(r0 + rl) * ldy_n] = v;
        }
    }
}

// ---------------------------------------------------------------- row-tile kernel
// Many short-lived workgroups, each owning R whole rows (R*bpr a multiple of
// 8, so the tile is a whole number of 8-super-block steps).  The 16 waves of
// a workgroup interleave the tile's steps (wave w takes steps w, w+16, ...), so
// at any moment a workgroup reads adjacent 1088-byte steps and the grid as a
// whole sweeps the matrix -- the order HBM serves best.  A wave streams its
// steps through a ring of D register buffers (each refilled right after it
// is consumed: D-1 steps in flight during every compute; the first D-1 fly
// while the activations are staged or quantised into LDS).  Each lane's
// sub-block term is summed over the 8 lanes of its super-block (DPP) and
// parked in LDS; rows are summed at the end, in super-block order, so rows
// may cross steps and waves freely and the result is deterministic.
// 16 waves and one tile per CU (38 VGPRs: 4 waves per SIMD) measured ahead of
// 8 waves and two tiles per CU: the same waves per CU, but half the
// workgroups stage (or, fused, quantise) the activations (graph-replayed
// decode set: fused step +5.5 %, prequantised +1.5 %, bs = 2 +4.5 %).
constexpr int TILE_WAVES = 16;
static_assert(4 * FUSED_VEC_ROUNDS_LONG * 64 * TILE_WAVES == GEMV_FUSED_VEC_MAX_K, "vector prologue bound");

// Up to GEMV_GROUP_MAX weight matrices with the same K that read the same
// activations, run by one launch: matrix g owns tiles [tile_end[g-1],
// tile_end[g]).  Every output row is computed exactly as by a launch of its
// own matrix (the tile size does not enter a row's arithmetic).
struct GemvGroup {
    const uint8_t* W[GEMV_GROUP_MAX];
    float* Y[GEMV_GROUP_MAX];
    int64_t ldy_m[GEMV_GROUP_MAX];
    int N[GEMV_GROUP_MAX];
    int tile_end[GEMV_GROUP_MAX];
};

// Arguments of the fused RMS-norm prologue (kRms): h = X (+ R), written to H
// by workgroup 0 only; the Q8_1 codes of (h * scale) * gamma go to LDS.  With
// the SwiGLU epilogue, S receives silu(gate) * up of the tile's rows.
struct RmsArgs {
    const float* R;
    float* H;
    const float* gamma;
    float eps;
    float* S;
};

// kRms: 0 = none; bit 0 = the RMS-norm prologue (C == 1), bit 1 = with a
// residual R, bit 2 = with a gain gamma; bit 4 = the fused single-column
// quantisation loads x as 16-byte vectors (x 16-byte aligned, unit stride),
// bit 5 = in up to five rounds; bit 6 = the SwiGLU pair: the tile is the
// same rows_per_wg rows of two matrices, gate (grp.W[0] -> grp.Y[0]) then up
// (grp.W[1] -> grp.Y[1]), streamed as one run of steps, and the epilogue
// also writes S = silu(gate) * up for those rows (the host makes every tile
// whole: rows_per_wg divides N and a tile's gate part fills whole steps).
template <int C, int D, bool kDebug, bool kFuse, bool kGroup, int kRms = 0>
__global__ __launch_bounds__(64 * TILE_WAVES) void gemv_tile_kernel(
    const GemvGroup grp, const int8_t* __restrict__ aqs, const uint32_t* __restrict__ ads,
    const float* __restrict__ X, int64_t sc, int64_t sk, int K, int64_t ldy_n, int rows_per_wg,
    int32_t* __restrict__ dbg, const RmsArgs rms) {
    constexpr bool kRmsOn = (kRms & 1) != 0, kRmsRes = (kRms & 2) != 0, kRmsGain = (kRms & 4) != 0;
    constexpr bool kVecX = (kRms & 16) != 0;
    constexpr int kVecRounds = (kRms & 32) ? FUSED_VEC_ROUNDS_LONG : FUSED_ROUNDS;
    constexpr bool kSwi = (kRms & 64) != 0;
    static_assert(!kSwi || (kRmsOn && !kGroup), "the SwiGLU epilogue serves the rms-fused gate/up pair");
    static_assert(!kVecX || (kFuse && C == 1 && !kRmsOn), "vector x loads serve the single-column fused prologue");
    static_assert(!kRmsOn || (C == 1 && !kFuse && RMS_THREADS == 64 * TILE_WAVES),
                  "the RMS prologue runs the producer's own 1024-thread reduction on one column");
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const uint8_t* __restrict__ W = grp.W[0];
    float* __restrict__ Y = grp.Y[0];
    int64_t ldy_m = grp.ldy_m[0];
    int N = grp.N[0], tile0 = 0;
    if (kGroup) {
        // this tile's matrix, by scalar selects (no dynamic index into the
        // argument block); a single matrix skips this dependent argument
        // read, which sits ahead of the first weight load
        int g = 0;
#pragma unroll
        for (int i = 0; i + 1 < GEMV_GROUP_MAX; ++i) g += (int)blockIdx.x >= grp.tile_end[i] ? 1 : 0;
#pragma unroll
        for (int i = 1; i < GEMV_GROUP_MAX; ++i) {
            if (g == i) {
                W = grp.W[i];
                Y = grp.Y[i];
                ldy_m = grp.ldy_m[i];
                N = grp.N[i];
                tile0 = grp.tile_end[i - 1];
            }
        }
    }
    const int bpr = K / QK_K, nb = K / QK8_1;
    int8_t* sq = reinterpret_cast<int8_t*>(lds);
    float* sdx = reinterpret_cast<float*>(lds + (size_t)C * K);
    float* part = sdx + C * nb;  // [C][rows_per_wg * bpr] super-block partials

    const int tid = threadIdx.x;
    const int lane = tid & 63, slot = lane >> 3, ib = lane & 7;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Single-matrix launches take their tiles in XCD-contiguous ranges:
    // workgroups are dispatched to the 8 XCDs round-robin (b -> XCD b % 8),
    // and XCD x gets tiles [x*q + min(x, r), ...) of the G = 8q + r (a
    // bijection).  Measured on the bs=1 decode set: -1.8 % per launch; grouped
    // launches measured 2 % slower with it and keep the dispatch order.
    int bid = (int)blockIdx.x;
    if (!kGroup) {
        const int G = (int)gridDim.x, q = G >> 3, r = G & 7, x = bid & 7;
        bid = x * q + min(x, r) + (bid >> 3);
    }
    const int r0 = (bid - tile0) * rows_per_wg;
    const int nrows = min(rows_per_wg, N - r0);
    const int n_sb = (kSwi ? 2 : 1) * nrows * bpr;  // SwiGLU pair: the gate rows, then the same up rows
    const int n_steps = (n_sb + 7) >> 3;
    const int my_n = wave < n_steps ? (n_steps - wave + TILE_WAVES - 1) / TILE_WAVES : 0;
    const uint8_t* Wg = W + (size_t)r0 * bpr * BLOCK_BYTES;
    // SwiGLU pair: steps from up_step on read the up matrix (wave-uniform select)
    const int up_step = kSwi ? (nrows * bpr) >> 3 : n_steps;
    const uint8_t* Wu = kSwi ? grp.W[1] + (size_t)r0 * bpr * BLOCK_BYTES : Wg;

    // Only a matrix's last tile can end inside a step: there the lanes past
    // the end re-read the last super-block and are not accumulated.
    const int last_step = n_steps - 1;
    const int last_slot = (n_sb - 1) - 8 * last_step;
    const uint32_t off_n = (uint32_t)slot * BLOCK_BYTES;
    const uint32_t off_l = (uint32_t)min(slot, last_slot) * BLOCK_BYTES;
    const uint32_t off_q = 16u * (uint32_t)ib;
    auto load = [&](StepRegs& r, int s) {
        const bool up = kSwi && s >= up_step;
        const uint8_t* base = (up ? Wu : Wg) + (size_t)(up ? s - up_step : s) * (8 * BLOCK_BYTES);  // scalar
        const uint32_t o = s == last_step ? off_l : off_n;
        r.h = *reinterpret_cast<const v2u*>(base + o);
        r.q = *reinterpret_cast<const v4i_a8*>(base + (o + off_q) + 8);
    };

    // Single-column fused prologue: x loads first, then the weight prefetch,
    // then the quantisation and the LDS writes, which wait only for the x
    // loads (measured: a gain for the fused path only; prequantised codes are
    // staged after the prefetch, below).
    const int nthreads = blockDim.x;
    const int tasks = K / 4;
    const bool split = kFuse && C == 1 && tasks <= (kVecX ? kVecRounds : FUSED_ROUNDS) * nthreads;
    FusedRegs fx;
    FusedVecRegs<kVecRounds> fv;
    if (split) {
        if constexpr (kVecX)
            fused_load_vec(fv, X, tasks, tid, nthreads);
        else
            fused_load(fx, X, sk, tasks, tid, nthreads);
    }
    RmsBatch rb;  // the RMS prologue's pass-1 loads (one batch: K <= RMS_ONE_BATCH_K), also ahead of the prefetch
    if (kRmsOn) rms_load<kRmsRes>(rb, X, rms.R, 4 * tid, K);
    // and the eight gains the quantisation pass will read (block tid/4, eight
    // elements per lane: one round covers K <= RMS_ONE_BATCH_K), so that pass
    // waits for neither the weight prefetch (vmcnt retires in order) nor a
    // round trip of its own
    static_assert(RMS_ONE_BATCH_K / QK8_1 * 4 <= RMS_THREADS, "one quantisation round per K");
    const int qe = 8 * min(tid, 4 * nb - 1);  // this lane's first element (clamped: every load unconditional)
    v4f gain[2];
    if constexpr (kRmsOn && kRmsGain) {
        gain[0] = *reinterpret_cast<const v4f*>(rms.gamma + qe);
        gain[1] = *reinterpret_cast<const v4f*>(rms.gamma + qe + 4);
    }
    // Every weight load is unconditional (steps past this wave's last one
    // repeat it; a wave with no step loads the tile's last), so the wait
    // counts are compile-time exact.  A branch around this prefetch would
    // make the prologue's own waits count as if it had not been issued
    // (vmcnt(0): the activations would wait for the weights).
    StepRegs buf[D];
#pragma unroll
    for (int d = 0; d < D - 1; ++d) load(buf[d], min(wave + TILE_WAVES * min(d, max(my_n - 1, 0)), last_step));
    // (8*s) mod bpr of this wave's current step, and its advance per own
    // step (64 super-blocks) mod bpr; bpr >= 8, so a few subtractions do.
    int u = 8 * wave;
    while (u >= bpr) u -= bpr;
    int sb_stride = TILE_WAVES * 8;
    while (sb_stride >= bpr) sb_stride -= bpr;
    if constexpr (kRmsOn) {
        // the producer's passes (rms_device.h), with h staged in LDS after the
        // partials and the codes written straight to the GEMV's LDS operand
        __shared__ double rms_part[RMS_WAVES];
        const size_t h_off =
            ((size_t)K + (size_t)nb * 4 + (size_t)(kSwi ? 2 : 1) * rows_per_wg * bpr * 4 + 15) & ~(size_t)15;
        float* shh = reinterpret_cast<float*>(lds + h_off);
        const double acc = rms_accumulate<kRmsRes, true>(rb, blockIdx.x == 0 ? rms.H : nullptr, shh, 4 * tid, K, 0.0);
        const float scale = rms_scale(rms_reduce(acc, rms_part, tid), K, rms.eps);
        if (tid < 4 * nb) {  // uniform per quad: block tid/4, elements qe .. qe+7
            const v4f h0 = *reinterpret_cast<const v4f*>(shh + qe), h1 = *reinterpret_cast<const v4f*>(shh + qe + 4);
            float y[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                y[i] = rms_y<kRmsGain>(h0[i], scale, kRmsGain ? gain[0][i] : 0.0f);
                y[4 + i] = rms_y<kRmsGain>(h1[i], scale, kRmsGain ? gain[1][i] : 0.0f);
            }
            const Q8Quad q = quantize_quad8(y);
            *reinterpret_cast<v2u*>(sq + qe) = v2u{q.q_lo, q.q_hi};
            if ((tid & 3) == 0) sdx[tid >> 2] = half_bits_to_float(q.d_bits);
        }
    } else if (split) {
        if constexpr (kVecX)
            fused_store_vec(fv, sq, sdx, tasks, tid, nthreads);
        else
            fused_store(fx, sq, sdx, tasks, tid, nthreads);
    } else if (kFuse) {
        quantize_to_lds<C>(X, sc, sk, K, sq, sdx, tid, nthreads);
    } else {
        stage_activations(aqs, ads, C, K, sq, sdx, tid, nthreads);
    }
    __syncthreads();

    const int sh_lo = 4 * ib, sh_hi = 16 + 2 * ib;
    auto compute = [&](const StepRegs& cur, int s) {
        const int sb = 8 * s + slot;
        const bool valid = s != last_step || slot <= last_slot;
        int pos = u + slot;                     // position of the super-block inside its row
        pos = pos >= bpr ? pos - bpr : pos;     // bpr >= 8 (host)
        const int a_idx = 8 * pos + ib;
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) decode_codes_x((uint32_t)cur.q[j], lo[j], hi[j]);
        const int ls = (int)(((cur.h.y >> sh_lo) & 0xFu) | (((cur.h.x >> sh_hi) & 0x3u) << 4)) - 32;
        const float dw = half_bits_to_float(cur.h.x & 0xFFFFu);
#pragma unroll
        for (int cc = 0; cc < C; ++cc) {
            const v4i* pa = reinterpret_cast<const v4i*>(sq + cc * K + a_idx * QK8_1);
            const v4i a0 = pa[0], a1 = pa[1];
            int sum = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                sum = dot4(lo[j], (uint32_t)a0[j], sum);
                sum = dot4(hi[j], (uint32_t)a1[j], sum);
            }
            sum = __mul24(sum, ls);
            float t = valid ? (dw * sdx[cc * nb + a_idx]) * (float)sum : 0.0f;
            if (kDebug && valid) {
                const int row = sb / bpr;
                dbg[((int64_t)cc * N + r0 + row) * nb + a_idx] = sum;
            }
            // sum over the 8 sub-blocks of the super-block (lanes 8*slot .. 8*slot+7)
            t += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, t), 0xB1, 0xF, 0xF, true));
            t += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, t), 0x4E, 0xF, 0xF, true));
            t += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, t), 0x141, 0xF, 0xF, true));
            if (ib == 0 && valid) part[cc * rows_per_wg * bpr + sb] = t;
        }
    };
    for (int i0 = 0; i0 < my_n; i0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int i = i0 + d;
            load(buf[(d + D - 1) % D], wave + TILE_WAVES * min(i + D - 1, my_n - 1));
            if (i < my_n) compute(buf[d], wave + TILE_WAVES * i);
            u += sb_stride;
            u = u >= bpr ? u - bpr : u;
        }
    }
    __syncthreads();
    // Row sums: 16 lanes (one DPP row) per output row; lane g sums partials
    // g, g+16, ... in order, then a fixed DPP tree adds the 16 lanes.  Every
    // lane of a DPP row takes the same branches.
    const int rgrp = tid >> 4, gl = tid & 15;
    const int n_grp = blockDim.x >> 4;
    // SwiGLU pair: the row sums also go to LDS (over the activation codes,
    // which no wave reads any more), gate rows first
    float* srow = reinterpret_cast<float*>(lds);
#pragma unroll
    for (int cc = 0; cc < C; ++cc) {
        for (int rl = rgrp; rl < (kSwi ? 2 * nrows : nrows); rl += n_grp) {
            const float* pr = part + cc * rows_per_wg * bpr + rl * bpr;
            float v = 0.0f;
            for (int b = gl; b < bpr; b += 16) v += pr[b];
            v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
            v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
            v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true));
            v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, true));
            if (gl == 0) {
                if constexpr (kSwi) {
                    float* const Yp = rl < nrows ? Y : grp.Y[1];
                    if (Yp) Yp[(int64_t)(r0 + (rl < nrows ? rl : rl - nrows)) * ldy_n] = v;
                    srow[rl] = v;
                } else {
                    Y[cc * ldy_m + (int64_t)(r0 + rl) * ldy_n] = v;
                }
            }
        }
    }
    if constexpr (kSwi) {
        __syncthreads();
        for (int j = tid; j < nrows; j += blockDim.x) rms.S[r0 + j] = swiglu(srow[j], srow[nrows + j]);
    }
}

// ---------------------------------------------------------------- launchers
constexpr int GEMV_WAVES_PER_WG = 8;
constexpr size_t GEMV_LDS_BUDGET = 64 * 1024;

int device_cu_count() {
    static std::atomic<int> cached[64];  // static storage: starts at zero
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
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

static int tuning_knob(const char* name, int def, int lo, int hi) {
    const char* v = getenv(name);
    if (v == nullptr) return def;
    const int x = atoi(v);
    return (x < lo || x > hi) ? def : x;
}

template <int C, int D>
static hipError_t launch_flat(const uint8_t* W, const int8_t* aqs, const uint32_t* aqs_ds, const float* X,
                              int64_t sc, int64_t sk, float* Y, int64_t K, int64_t N, int64_t ldy_m, int64_t ldy_n,
                              int32_t* dbg, hipStream_t stream) {
    const int64_t bpr = K / QK_K, nb = K / QK8_1;
    const int64_t g = 8 / std::gcd<int64_t, int64_t>(bpr, 8);   // rows per 8-super-block boundary
    static const int wgs_per_cu = tuning_knob("IQ4XS_GEMV_WGS_PER_CU", 2, 1, 8);
    const int64_t target = (int64_t)wgs_per_cu * device_cu_count();
    const int64_t units = (N + g - 1) / g;
    const int64_t rows_per_wg = ((units + target - 1) / target) * g;
    const int64_t wgs = (N + rows_per_wg - 1) / rows_per_wg;
    if (rows_per_wg * bpr * BLOCK_BYTES >= ((int64_t)1 << 31)) return hipErrorNotSupported;
    const int64_t steps = (rows_per_wg * bpr + 7) / 8;
    const int64_t q_max = (steps + FLAT_WAVES - 1) / FLAT_WAVES;
    const int64_t J = (8 * q_max - 1) / bpr + 2;
    const size_t lds = (size_t)C * K + (size_t)C * nb * 4 + (size_t)FLAT_WAVES * J * C * 4 + FLAT_WAVES * 8;
    if (lds > GEMV_LDS_BUDGET) return hipErrorNotSupported;
    const dim3 grid((unsigned)wgs), block(64 * FLAT_WAVES);
#define IQ4XS_LAUNCH_FLAT(DBG, FUSE)                                                                              \
    hipLaunchKernelGGL((gemv_flat_kernel<C, D, DBG, FUSE>), grid, block, lds, stream, W, aqs, aqs_ds, X, sc, sk, Y, \
                       (int)K, (int)N, ldy_m, ldy_n, (int)rows_per_wg, (int)J, dbg)
    if (X != nullptr) {
        if (dbg) IQ4XS_LAUNCH_FLAT(true, true); else IQ4XS_LAUNCH_FLAT(false, true);
    } else {
        if (dbg) IQ4XS_LAUNCH_FLAT(true, false); else IQ4XS_LAUNCH_FLAT(false, false);
    }
#undef IQ4XS_LAUNCH_FLAT
    return hipGetLastError();
}

// Rows per tile: a multiple of g (so a tile is a whole number of steps),
// sized for about `tiles_per_cu` tiles per CU.
static int64_t tile_rows(int64_t bpr, int64_t N) {
    const int64_t g = 8 / std::gcd<int64_t, int64_t>(bpr, 8);
    static const int tiles_per_cu = tuning_knob("IQ4XS_GEMV_TILES_PER_CU", 1, 1, 64);
    const int64_t tiles = (int64_t)tiles_per_cu * device_cu_count();
    const int64_t units = (N + g - 1) / g;
    return ((units + tiles - 1) / tiles) * g;
}

// Rows per tile of a grouped launch: tile_rows of the summed rows, raised (by
// whole steps) until the per-matrix tiles, each rounded up, fit the same
// number of tiles -- otherwise three matrices round up to a tile past one per CU.
static int64_t group_tile_rows(int64_t bpr, const int64_t* Ns, int count) {
    const int64_t g = 8 / std::gcd<int64_t, int64_t>(bpr, 8);
    int64_t rows = 0;
    for (int i = 0; i < count; ++i) rows += Ns[i];
    int64_t R = tile_rows(bpr, rows);
    const int64_t cap = std::max<int64_t>((rows + R - 1) / R, count);  // reached once R >= every N
    for (;;) {
        int64_t t = 0;
        for (int i = 0; i < count; ++i) t += (Ns[i] + R - 1) / R;
        if (t <= cap) return R;
        R += g;
    }
}

// One launch over the matrices of `mats` (count >= 1, all with K columns);
// hipErrorNotSupported when a tile's LDS does not fit.
struct TileMat {
    const uint8_t* W;
    float* Y;
    int64_t N, ldy_m;
};

template <int C, int D>
static hipError_t launch_tile_d(const TileMat* mats, int count, const int8_t* aqs, const uint32_t* ads,
                                const float* X, int64_t sc, int64_t sk, int64_t K, int64_t ldy_n, int32_t* dbg,
                                int64_t R, hipStream_t stream) {
    const int64_t bpr = K / QK_K, nb = K / QK8_1;
    GemvGroup grp{};
    int64_t wgs = 0;
    for (int i = 0; i < GEMV_GROUP_MAX; ++i) {
        const TileMat& m = mats[i < count ? i : count - 1];
        if (i < count) wgs += (m.N + R - 1) / R;
        grp.W[i] = m.W;
        grp.Y[i] = m.Y;
        grp.ldy_m[i] = m.ldy_m;
        grp.N[i] = (int)m.N;
        grp.tile_end[i] = (int)(wgs < 0x7FFFFFFF ? wgs : 0x7FFFFFFF);
    }
    const size_t lds = (size_t)C * K + (size_t)C * nb * 4 + (size_t)C * R * bpr * 4;
    if (lds > GEMV_LDS_BUDGET || wgs > 0x7FFFFFFF) return hipErrorNotSupported;
    const dim3 grid((unsigned)wgs), block(64 * TILE_WAVES);
#define IQ4XS_LAUNCH_TILE(DBG, FUSE)                                                                              \
    hipLaunchKernelGGL((gemv_tile_kernel<C, D, DBG, FUSE, false>), grid, block, lds, stream, grp, aqs, ads, X, sc, \
                       sk, (int)K, ldy_n, (int)R, dbg, RmsArgs{})
    if (count > 1) {
        if (X != nullptr || dbg != nullptr) return hipErrorNotSupported;  // grouped: planar activations only
        hipLaunchKernelGGL((gemv_tile_kernel<C, D, false, false, true>), grid, block, lds, stream, grp, aqs, ads, X,
                           sc, sk, (int)K, ldy_n, (int)R, dbg, RmsArgs{});
    } else if (X != nullptr) {
        // unit stride and 16-byte alignment: the prologue's vector loads
        const bool vec = C == 1 && sk == 1 && reinterpret_cast<uintptr_t>(X) % 16 == 0;
        if (dbg) IQ4XS_LAUNCH_TILE(true, true);
        else if (vec && (K / 4) <= FUSED_ROUNDS * 64 * TILE_WAVES)
            hipLaunchKernelGGL((gemv_tile_kernel<C, D, false, true, false, (C == 1 ? 16 : 0)>), grid, block, lds, stream,
                               grp, aqs, ads, X, sc, sk, (int)K, ldy_n, (int)R, dbg, RmsArgs{});
        else if (vec && (K / 4) <= FUSED_VEC_ROUNDS_LONG * 64 * TILE_WAVES)
            hipLaunchKernelGGL((gemv_tile_kernel<C, D, false, true, false, (C == 1 ? 48 : 0)>), grid, block, lds, stream,
                               grp, aqs, ads, X, sc, sk, (int)K, ldy_n, (int)R, dbg, RmsArgs{});
        else IQ4XS_LAUNCH_TILE(false, true);
    } else {
        if (dbg) IQ4XS_LAUNCH_TILE(true, false); else IQ4XS_LAUNCH_TILE(false, false);
    }
#undef IQ4XS_LAUNCH_TILE
    return hipGetLastError();
}

template <int C>
static hipError_t launch_tile_group(const TileMat* mats, int count, const int8_t* aqs, const uint32_t* ads,
                                    const float* X, int64_t sc, int64_t sk, int64_t K, int64_t ldy_n, int32_t* dbg,
                                    hipStream_t stream) {
    const int64_t bpr = K / QK_K;
    int64_t rows = 0, Ns[GEMV_GROUP_MAX];
    for (int i = 0; i < count; ++i) {
        rows += mats[i].N;
        Ns[i] = mats[i].N;
    }
    const int64_t R = group_tile_rows(bpr, Ns, count);
    if (R * bpr * BLOCK_BYTES >= ((int64_t)1 << 31) || rows >= ((int64_t)1 << 30)) return hipErrorNotSupported;
    static const int depth = tuning_knob("IQ4XS_GEMV_TILE_D", 2, 2, 4);
    if (depth == 3) return launch_tile_d<C, 3>(mats, count, aqs, ads, X, sc, sk, K, ldy_n, dbg, R, stream);
    if (depth == 4) return launch_tile_d<C, 4>(mats, count, aqs, ads, X, sc, sk, K, ldy_n, dbg, R, stream);
    return launch_tile_d<C, 2>(mats, count, aqs, ads, X, sc, sk, K, ldy_n, dbg, R, stream);
}

template <int C>
static hipError_t launch_tile(const uint8_t* W, const int8_t* aqs, const uint32_t* ads, const float* X, int64_t sc,
                              int64_t sk, float* Y, int64_t K, int64_t N, int64_t ldy_m, int64_t ldy_n, int32_t* dbg,
                              hipStream_t stream) {
    const TileMat m{W, Y, N, ldy_m};
    return launch_tile_group<C>(&m, 1, aqs, ads, X, sc, sk, K, ldy_n, dbg, stream);
}

template <int C>
static hipError_t launch_flat_depth(const uint8_t* W, const int8_t* aqs, const uint32_t* ads, const float* X,
                                    int64_t sc, int64_t sk, float* Y, int64_t K, int64_t N, int64_t ldy_m,
                                    int64_t ldy_n, int32_t* dbg, hipStream_t stream) {
    static const int depth = tuning_knob("IQ4XS_GEMV_DEPTH", 3, 2, 4);
    switch (depth) {
        case 2: return launch_flat<C, 2>(W, aqs, ads, X, sc, sk, Y, K, N, ldy_m, ldy_n, dbg, stream);
        case 4: return launch_flat<C, 4>(W, aqs, ads, X, sc, sk, Y, K, N, ldy_m, ldy_n, dbg, stream);
        default: return launch_flat<C, 3>(W, aqs, ads, X, sc, sk, Y, K, N, ldy_m, ldy_n, dbg, stream);
    }
}

// Planar columns that go to the matrix-core GEMV: its cost per weight byte
// does not grow with the columns, the dot4 kernels' does.  Measured on the
// graph-replayed decode set (K 5120-17408): from 4 columns on it wins on a
// layer (bs = 4: 2.10 against 2.01 TB/s); below that, and for narrow matrices
// (k/v, N = 1024: too few 32-row blocks to fill the chip) below 8 columns,
// the dot4 kernels are faster.  Grouped launches use the same rule per
// matrix, so their outputs match single calls bit for bit.
static bool use_gemv_mfma(int64_t N, int64_t M) {
    static const int min_cols = tuning_knob("IQ4XS_GEMV_MFMA_MIN_COLS", 4, 1, 9);
    // narrow matrices from 8 columns on: k/v (N = 1024) measured 6.60 us
    // there against 7.05 for dot4 (dot4 wins at 4 and 6 columns)
    return M >= min_cols && (N >= 2048 || (M >= 8 && N >= 1024));
}

// X == nullptr: planar Q8_1 activations (aqs, ads); otherwise fp32 X quantised
// in the prologue (fused; returns hipErrorNotSupported when it does not fit).
template <int C>
static hipError_t launch_cols(const uint8_t* W, const int8_t* aqs, const uint32_t* ads, const float* X, int64_t sc,
                              int64_t sk, float* Y, int64_t K, int64_t N, int64_t ldy_m, int64_t ldy_n, int32_t* dbg,
                              hipStream_t stream) {
    const int64_t bpr = K / QK_K;
    hipError_t err = hipErrorNotSupported;
    if (X == nullptr && use_gemv_mfma(N, C)) {
        err = launch_gemv_mfma(W, aqs, ads, Y, K, N, C, ldy_m, ldy_n, dbg, stream);
        if (err != hipErrorNotSupported) return err;
    }
    static const int kind = tuning_knob("IQ4XS_GEMV_KIND", 2, 0, 2);  // 0 items, 1 flat, 2 tile
    const bool fits = K <= (1 << 24) && N < (1 << 30);
    if (fits && bpr >= 8 && kind == 2)
        err = launch_tile<C>(W, aqs, ads, X, sc, sk, Y, K, N, ldy_m, ldy_n, dbg, stream);
    if (err == hipErrorNotSupported && fits && bpr >= 8 && kind >= 1)
        err = launch_flat_depth<C>(W, aqs, ads, X, sc, sk, Y, K, N, ldy_m, ldy_n, dbg, stream);
    if (err == hipErrorNotSupported && fits) {
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

hipError_t launch_gemv_group(int count, const uint8_t* const* W, float* const* Y, const int64_t* N,
                             const int8_t* aqs, const uint32_t* ads, int64_t K, int64_t M, bool layout_mk,
                             hipStream_t stream) {
    clear_launch_error();
    TileMat mats[GEMV_GROUP_MAX];
    for (int i = 0; i < count; ++i) mats[i] = {W[i], Y[i], N[i], layout_mk ? N[i] : 1};
    const int64_t ldy_n = layout_mk ? 1 : M;
    static const int kind = tuning_knob("IQ4XS_GEMV_KIND", 2, 0, 2);
    // matrix-core matrices first, one launch per wave count (the same
    // routing and kernel as single calls)
    TileMat rest[GEMV_GROUP_MAX];
    int n_rest = 0;
    bool done[GEMV_GROUP_MAX] = {};
    for (int i = 0; i < count; ++i) {
        if (done[i]) continue;
        if (!use_gemv_mfma(N[i], M)) {
            rest[n_rest++] = mats[i];
            continue;
        }
        const uint8_t* gW[GEMV_GROUP_MAX];
        float* gY[GEMV_GROUP_MAX];
        int64_t gN[GEMV_GROUP_MAX], gL[GEMV_GROUP_MAX];
        int n = 0;
        const int waves = gemv_mfma_waves(N[i]);
        for (int j = i; j < count; ++j) {
            if (done[j] || !use_gemv_mfma(N[j], M) || gemv_mfma_waves(N[j]) != waves) continue;
            gW[n] = W[j];
            gY[n] = Y[j];
            gN[n] = N[j];
            gL[n] = mats[j].ldy_m;
            ++n;
            done[j] = true;
        }
        hipError_t err = launch_gemv_mfma_group(n, gW, gY, gN, gL, aqs, ads, K, M, ldy_n, nullptr, stream);
        if (err == hipErrorNotSupported) {  // shapes past its offsets take the single-call route
            err = hipSuccess;
            for (int j = 0; j < n && err == hipSuccess; ++j)
                err = dispatch_cols(gW[j], aqs, ads, nullptr, 0, 0, gY[j], K, gN[j], M, gL[j], ldy_n, nullptr, stream);
        }
        if (err != hipSuccess) return err;
    }
    if (n_rest == 0) return hipSuccess;
    hipError_t err = hipErrorNotSupported;
    if (K / QK_K >= 8 && K <= (1 << 24) && kind == 2) {
        switch (M) {
            case 1: err = launch_tile_group<1>(rest, n_rest, aqs, ads, nullptr, 0, 0, K, ldy_n, nullptr, stream); break;
            case 2: err = launch_tile_group<2>(rest, n_rest, aqs, ads, nullptr, 0, 0, K, ldy_n, nullptr, stream); break;
            case 3: err = launch_tile_group<3>(rest, n_rest, aqs, ads, nullptr, 0, 0, K, ldy_n, nullptr, stream); break;
            case 4: err = launch_tile_group<4>(rest, n_rest, aqs, ads, nullptr, 0, 0, K, ldy_n, nullptr, stream); break;
            case 5: err = launch_tile_group<5>(rest, n_rest, aqs, ads, nullptr, 0, 0, K, ldy_n, nullptr, stream); break;
            case 6: err = launch_tile_group<6>(rest, n_rest, aqs, ads, nullptr, 0, 0, K, ldy_n, nullptr, stream); break;
            case 7: err = launch_tile_group<7>(rest, n_rest, aqs, ads, nullptr, 0, 0, K, ldy_n, nullptr, stream); break;
            case 8: err = launch_tile_group<8>(rest, n_rest, aqs, ads, nullptr, 0, 0, K, ldy_n, nullptr, stream); break;
            default: return hipErrorInvalidValue;
        }
        if (err != hipErrorNotSupported) return err;
    }
    // shapes the tile kernel does not take: one launch per matrix
    for (int i = 0; i < n_rest; ++i) {
        err = dispatch_cols(rest[i].W, aqs, ads, nullptr, 0, 0, rest[i].Y, K, rest[i].N, M, rest[i].ldy_m, ldy_n,
                            nullptr, stream);
        if (err != hipSuccess) return err;
    }
    return hipSuccess;
}

template <int MODE>
static void launch_rms_tile(dim3 grid, dim3 block, size_t lds, hipStream_t stream, const GemvGroup& grp,
                            const float* X, int64_t K, int64_t R, const RmsArgs& a) {
    // grouped tiles (one matrix per tile), except the SwiGLU pair (bit 6): both matrices per tile
    hipLaunchKernelGGL((gemv_tile_kernel<1, 2, false, false, (MODE & 64) == 0, MODE>), grid, block, lds, stream, grp, nullptr,
                       nullptr, X, 0, 1, (int)K, 1, (int)R, nullptr, a);
}

// RMS norm of one column fused into the prologue of a grouped bs=1 GEMV: every
// workgroup runs the producer's passes on the whole row (h staged in LDS, the
// Q8_1 codes straight into the GEMV's operand), workgroup 0 writes H.  The
// codes, and so every output, are those of iq4xs_rms_norm_q8_1 followed by the
// grouped GEMV.  hipErrorNotSupported past one pass-1 batch (K > 8192), below
// the tile kernel's K >= 2048, or when the LDS does not fit.
hipError_t launch_gemv_rms_group(int count, const uint8_t* const* W, float* const* Y, const int64_t* N,
                                 const float* X, const float* R, float* H, const float* gamma, float eps, int64_t K,
                                 hipStream_t stream) {
    clear_launch_error();
    const int64_t bpr = K / QK_K, nb = K / QK8_1;
    if (count < 1 || count > GEMV_GROUP_MAX || bpr < 8 || K > RMS_ONE_BATCH_K) return hipErrorNotSupported;
    int64_t rows = 0;
    for (int i = 0; i < count; ++i) rows += N[i];
    const int64_t Rr = group_tile_rows(bpr, N, count);
    if (Rr * bpr * BLOCK_BYTES >= ((int64_t)1 << 31) || rows >= ((int64_t)1 << 30)) return hipErrorNotSupported;
    GemvGroup grp{};
    int64_t wgs = 0;
    for (int i = 0; i < GEMV_GROUP_MAX; ++i) {
        const int k = i < count ? i : count - 1;
        if (i < count) wgs += (N[k] + Rr - 1) / Rr;
        grp.W[i] = W[k];
        grp.Y[i] = Y[k];
        grp.ldy_m[i] = N[k];
        grp.N[i] = (int)N[k];
        grp.tile_end[i] = (int)(wgs < 0x7FFFFFFF ? wgs : 0x7FFFFFFF);
    }
    const size_t h_off = ((size_t)K + (size_t)nb * 4 + (size_t)Rr * bpr * 4 + 15) & ~(size_t)15;
    const size_t lds = h_off + (size_t)K * 4;
    if (lds > GEMV_LDS_BUDGET || wgs > 0x7FFFFFFF) return hipErrorNotSupported;
    const dim3 grid((unsigned)wgs), block(64 * TILE_WAVES);
    const RmsArgs a{R, H, gamma, eps, nullptr};
    switch ((R ? 2 : 0) | (gamma ? 4 : 0)) {
        case 0: launch_rms_tile<1>(grid, block, lds, stream, grp, X, K, Rr, a); break;
        case 2: launch_rms_tile<3>(grid, block, lds, stream, grp, X, K, Rr, a); break;
        case 4: launch_rms_tile<5>(grid, block, lds, stream, grp, X, K, Rr, a); break;
        default: launch_rms_tile<7>(grid, block, lds, stream, grp, X, K, Rr, a); break;
    }
    return hipGetLastError();
}

// RMS norm + the gate/up pair of a SwiGLU MLP + the SwiGLU itself, one launch
// (bs = 1): every workgroup runs the norm's passes as above, then streams the
// same R rows of gate and of up as one run of steps, and its epilogue writes
// the rows' gate and up outputs (when Yg / Yu are given) and
// S = silu(gate) * up with the SwiGLU producer's arithmetic (act_device.h).
// Rows are computed exactly as by launch_gemv_rms_group on (gate, up), so Yg,
// Yu and h are those bits, and S is the producer's fp32 value of them.  R
// divides N, so every tile is whole, with R * K/256 a multiple of 8 (whole
// steps) and about N / CUs rows (one tile per CU); hipErrorNotSupported when
// no such R exists, or as launch_gemv_rms_group.
hipError_t launch_gemv_rms_swiglu(const uint8_t* Wg, const uint8_t* Wu, float* Yg, float* Yu, float* S, int64_t N,
                                  const float* X, const float* R, float* H, const float* gamma, float eps, int64_t K,
                                  hipStream_t stream) {
    clear_launch_error();
    const int64_t bpr = K / QK_K, nb = K / QK8_1;
    if (bpr < 8 || K > RMS_ONE_BATCH_K || N < 1 || N >= ((int64_t)1 << 30)) return hipErrorNotSupported;
    const int64_t g = 8 / std::gcd<int64_t, int64_t>(bpr, 8);
    const int64_t cus = device_cu_count();
    int64_t Rr = 0;
    // the epilogue parks 2R row sums over the K bytes of activation codes
    for (int64_t r = g * (((N + cus - 1) / cus + g - 1) / g); r <= N && 8 * r <= K; r += g) {
        if (N % r == 0) {
            Rr = r;
            break;
        }
    }
    if (Rr == 0 || Rr * bpr * BLOCK_BYTES >= ((int64_t)1 << 31)) return hipErrorNotSupported;
    GemvGroup grp{};
    for (int i = 0; i < GEMV_GROUP_MAX; ++i) {
        grp.W[i] = i == 1 ? Wu : Wg;
        grp.Y[i] = i == 1 ? Yu : Yg;
        grp.ldy_m[i] = N;
        grp.N[i] = (int)N;
        grp.tile_end[i] = (int)(N / Rr);
    }
    const size_t h_off = ((size_t)K + (size_t)nb * 4 + (size_t)2 * Rr * bpr * 4 + 15) & ~(size_t)15;
    const size_t lds = h_off + (size_t)K * 4;
    if (lds > GEMV_LDS_BUDGET) return hipErrorNotSupported;
    const dim3 grid((unsigned)(N / Rr)), block(64 * TILE_WAVES);
    const RmsArgs a{R, H, gamma, eps, S};
    switch ((R ? 2 : 0) | (gamma ? 4 : 0)) {
        case 0: launch_rms_tile<1 | 64>(grid, block, lds, stream, grp, X, K, Rr, a); break;
        case 2: launch_rms_tile<3 | 64>(grid, block, lds, stream, grp, X, K, Rr, a); break;
        case 4: launch_rms_tile<5 | 64>(grid, block, lds, stream, grp, X, K, Rr, a); break;
        default: launch_rms_tile<7 | 64>(grid, block, lds, stream, grp, X, K, Rr, a); break;
    }
    return hipGetLastError();
}

hipError_t launch_gemv(const uint8_t* W, const int8_t* aqs, const uint32_t* ads, float* Y, int64_t K, int64_t N,
                       int64_t M, int64_t ldy_m, int64_t ldy_n, int32_t* dbg, hipStream_t stream) {
    clear_launch_error();
    return dispatch_cols(W, aqs, ads, nullptr, 0, 0, Y, K, N, M, ldy_m, ldy_n, dbg, stream);
}

hipError_t launch_gemv_fused(const uint8_t* W, const float* X, int64_t sc, int64_t sk, float* Y, int64_t K, int64_t N,
                             int64_t M, int64_t ldy_m, int64_t ldy_n, int32_t* dbg, hipStream_t stream) {
    clear_launch_error();
    return dispatch_cols(W, nullptr, nullptr, X, sc, sk, Y, K, N, M, ldy_m, ldy_n, dbg, stream);
}

}  // namespace iq4xs
