// gemv.hip -- IQ4_XS x Q8_1 GEMV / small-batch GEMV (1..8 activation columns)
// for gfx950, wave64.
//
// Semantics: vec_dot_iq4_xs_q8_1 (real_stock_dp4a_comparator.hip:145-166)
// summed over every 32-weight sub-block of a row (:325-360):
//   y[n] = sum_kb fp16(W.d) * fp16(ds.d) * (float)(sumi_kb * (ls_kb - 32)).
// The int32 sumi of every sub-block is exact (bit-identical to the
// reference); only the fp32 summation order differs.
//
// MI355X mapping.  Each wave owns R consecutive weight rows and streams them
// end to end.  Lane l handles sub-block (l & 7) of super-block column
// b = (l >> 3) + 8i, so one load instruction of the wave covers 8 whole
// consecutive super-blocks (1088 contiguous bytes of one row): fully used
// 128-byte lines straight from HBM, no LDS staging.  The codebook lookup is
// v_perm_b32 on the table held in four SGPR constants, the dot is
// v_dot4_i32_i8, the per-sub-block scale is applied in fp32, and the 64
// partial sums of a row are reduced across the wave once at the end.  The
// 32 Q8_1 codes of a lane are loaded once per super-block column and reused
// for all R rows; they are read from L2 (the whole activation vector is at
// most 8 x 17 KB).
#include "iq4xs_device.h"
#include "iq4xs_internal.h"

namespace iq4xs {

template <int C, int R, bool kDebug>
__global__ __launch_bounds__(256) void gemv_iq4xs_kernel(const uint8_t* __restrict__ W,
                                                         const int8_t* __restrict__ aqs,
                                                         const uint32_t* __restrict__ ads, float* __restrict__ Y,
                                                         int64_t K, int64_t N, int64_t ldy_m, int64_t ldy_n,
                                                         int32_t* __restrict__ dbg) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t row0 = wave * R;
    if (row0 >= N) return;
    const int ib = lane & 7;
    const int slot = lane >> 3;
    const int64_t bpr = K / QK_K;
    const int64_t nb = K / QK8_1;
    const int64_t row_bytes = bpr * BLOCK_BYTES;

    const uint8_t* wrow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t rr = (row0 + r < N) ? row0 + r : N - 1;  // tail rows re-read the last row, never stored
        wrow[r] = W + rr * row_bytes + 8 + 16 * ib;
    }

    float acc[R][C];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < C; ++c) acc[r][c] = 0.0f;

    for (int64_t b = slot; b < bpr; b += 8) {
        v4i a0[C], a1[C];
        float dx[C];
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const v4i* p = reinterpret_cast<const v4i*>(aqs + c * K + b * QK_K + ib * QK8_1);
            a0[c] = p[0];
            a1[c] = p[1];
            dx[c] = half_bits_to_float(ads[c * nb + b * 8 + ib] & 0xFFFFu);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t* qp = wrow[r] + b * BLOCK_BYTES;  // qs of sub-block ib
            const uint8_t* hp = qp - 8 - 16 * ib;           // super-block header
            const v4i w = *reinterpret_cast<const v4i_a8*>(qp);
            const uint32_t h0 = *reinterpret_cast<const uint32_t*>(hp);
            const uint32_t h1 = *reinterpret_cast<const uint32_t*>(hp + 4);
            const int ls = subblock_ls(h0, h1, ib) - 32;
            const float dw = half_bits_to_float(h0 & 0xFFFFu);
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) decode_codes((uint32_t)w[j], lo[j], hi[j]);
#pragma unroll
            for (int c = 0; c < C; ++c) {
                int s = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    s = dot4(lo[j], (uint32_t)a0[c][j], s);
                    s = dot4(hi[j], (uint32_t)a1[c][j], s);
                }
                s *= ls;
                acc[r][c] += (dw * dx[c]) * (float)s;
                if (kDebug && row0 + r < N) dbg[((int64_t)c * N + row0 + r) * nb + b * 8 + ib] = s;
            }
        }
    }

#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const float v = wave_sum(acc[r][c]);
            if (lane == 0 && row0 + r < N) Y[c * ldy_m + (row0 + r) * ldy_n] = v;
        }
}

template <int C, int R>
static hipError_t launch_gemv_cr(const uint8_t* W, const int8_t* aqs, const uint32_t* ads, float* Y, int64_t K,
                                 int64_t N, int64_t ldy_m, int64_t ldy_n, int32_t* dbg, hipStream_t stream) {
    const int64_t waves = (N + R - 1) / R;
    const int64_t grid = (waves + 3) / 4;
    if (grid > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
    if (dbg)
        hipLaunchKernelGGL((gemv_iq4xs_kernel<C, R, true>), dim3((unsigned)grid), dim3(256), 0, stream, W, aqs, ads,
                           Y, K, N, ldy_m, ldy_n, dbg);
    else
        hipLaunchKernelGGL((gemv_iq4xs_kernel<C, R, false>), dim3((unsigned)grid), dim3(256), 0, stream, W, aqs, ads,
                           Y, K, N, ldy_m, ldy_n, dbg);
    return hipGetLastError();
}

hipError_t launch_gemv(const uint8_t* W, const int8_t* aqs, const uint32_t* ads, float* Y, int64_t K, int64_t N,
                       int64_t M, int64_t ldy_m, int64_t ldy_n, int32_t* dbg, hipStream_t stream) {
    switch (M) {
        case 1: return launch_gemv_cr<1, 2>(W, aqs, ads, Y, K, N, ldy_m, ldy_n, dbg, stream);
        case 2: return launch_gemv_cr<2, 2>(W, aqs, ads, Y, K, N, ldy_m, ldy_n, dbg, stream);
        case 3: return launch_gemv_cr<3, 2>(W, aqs, ads, Y, K, N, ldy_m, ldy_n, dbg, stream);
        case 4: return launch_gemv_cr<4, 2>(W, aqs, ads, Y, K, N, ldy_m, ldy_n, dbg, stream);
        case 5: return launch_gemv_cr<5, 2>(W, aqs, ads, Y, K, N, ldy_m, ldy_n, dbg, stream);
        case 6: return launch_gemv_cr<6, 2>(W, aqs, ads, Y, K, N, ldy_m, ldy_n, dbg, stream);
        case 7: return launch_gemv_cr<7, 2>(W, aqs, ads, Y, K, N, ldy_m, ldy_n, dbg, stream);
        case 8: return launch_gemv_cr<8, 2>(W, aqs, ads, Y, K, N, ldy_m, ldy_n, dbg, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace iq4xs
