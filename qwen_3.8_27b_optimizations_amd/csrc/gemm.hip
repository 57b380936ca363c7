// gemm.hip -- IQ4_XS x Q8_1 prefill GEMM on gfx950 int8 MFMA.
//
// Semantics: the reference GEMM (real_stock_dp4a_comparator.hip:374-443):
//   Y[n,m] = sum_kb fp16(W.d) * fp16(ds[m,kb].d) * (float)(sumi[n,m,kb] * (ls-32))
// where sumi is the exact int32 dot of a 32-weight sub-block with the
// matching Q8_1 block.
//
// MI355X mapping.  A workgroup (4 waves) owns a 64-row x 64-token output
// tile and walks K one 256-weight super-block at a time:
//   1. the 64 weight rows' super-blocks are decoded (v_perm codebook lookup,
//      decode_codes_x)
//      straight into int8 LDS tiles, the per-sub-block weight scales
//      d*(ls-32) into a float table;
//   2. the 64 tokens' Q8_1 codes are copied to LDS, their d into a table;
//   3. each wave issues one v_mfma_i32_32x32x32_i8 per 32-wide sub-block --
//      K=32 is exactly one sub-block, so the MFMA result IS the reference's
//      int32 sumi -- and folds it into fp32 accumulators with the two scales.
// LDS rows are 256 bytes; the 16-byte chunk index is XORed with (row & 15)
// so the 32 lanes that read one k-chunk of 32 different rows hit 16
// distinct chunk positions (no bank conflicts from the 256-byte row stride).
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

template <bool kDebug>
__global__ __launch_bounds__(256) void gemm_iq4xs_mfma_kernel(const uint8_t* __restrict__ W,
                                                              const int8_t* __restrict__ aqs,
                                                              const uint32_t* __restrict__ ads,
                                                              float* __restrict__ Y, int64_t K, int64_t N,
                                                              int64_t M, int64_t ldy_m, int64_t ldy_n,
                                                              int32_t* __restrict__ dbg) {
    __shared__ __attribute__((aligned(16))) int8_t sW[GEMM_BN * 256];
    __shared__ __attribute__((aligned(16))) int8_t sX[GEMM_BM * 256];
    __shared__ __attribute__((aligned(16))) float sA[8][GEMM_BN];
    __shared__ __attribute__((aligned(16))) float sB[8][GEMM_BM];
    __shared__ int sL[kDebug ? 8 : 1][GEMM_BN];  // ls - 32, only for the debug export

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wn = wave & 1, wm = wave >> 1;
    const int64_t n0 = (int64_t)blockIdx.x * GEMM_BN;
    const int64_t m0 = (int64_t)blockIdx.y * GEMM_BM;
    const int64_t bpr = K / QK_K, nb = K / QK8_1, row_bytes = bpr * BLOCK_BYTES;

    float acc[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.0f;

    for (int64_t kb = 0; kb < bpr; ++kb) {
        __syncthreads();
        // 1. weights: 64 rows x 8 sub-blocks, two (row, sub-block) pairs per thread
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const int p = tid + 256 * it;
            const int r = p >> 3, s = p & 7;
            const int64_t n = (n0 + r < N) ? n0 + r : N - 1;
            const uint8_t* blk = W + n * row_bytes + kb * BLOCK_BYTES;
            const uint2 h = *reinterpret_cast<const uint2*>(blk);
            const v4i w = *reinterpret_cast<const v4i_a8*>(blk + 8 + 16 * s);
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) decode_codes_x((uint32_t)w[j], lo[j], hi[j]);
            *reinterpret_cast<v4i*>(sW + lds_swz(r, 2 * s)) = v4i{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3]};
            *reinterpret_cast<v4i*>(sW + lds_swz(r, 2 * s + 1)) = v4i{(int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
            sA[s][r] = half_bits_to_float(h.x & 0xFFFFu) * (float)(subblock_ls(h.x, h.y, s) - 32);
            if (kDebug) sL[s][r] = subblock_ls(h.x, h.y, s) - 32;
        }
        // 2. activations: 64 tokens x 16 chunks of 16 codes, four per thread
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int p = tid + 256 * it;
            const int r = p >> 4, c = p & 15;
            const int64_t m = (m0 + r < M) ? m0 + r : M - 1;
            *reinterpret_cast<v4i*>(sX + lds_swz(r, c)) =
                *reinterpret_cast<const v4i*>(aqs + m * K + kb * QK_K + 16 * c);
        }
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const int p = tid + 256 * it;
            const int r = p >> 3, s = p & 7;
            const int64_t m = (m0 + r < M) ? m0 + r : M - 1;
            sB[s][r] = half_bits_to_float(ads[m * nb + kb * 8 + s] & 0xFFFFu);
        }
        __syncthreads();

        // 3. one MFMA per sub-block, fp32 scale epilogue
        const int ra = 32 * wn + (lane & 31);
        const int rb = 32 * wm + (lane & 31);
#pragma unroll 2
        for (int s = 0; s < 8; ++s) {
            const int ch = 2 * s + (lane >> 5);
            const v4i a = *reinterpret_cast<const v4i*>(sW + lds_swz(ra, ch));
            const v4i b = *reinterpret_cast<const v4i*>(sX + lds_swz(rb, ch));
            const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, v16i{}, 0, 0, 0);
            const float bx = sB[s][rb];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int i = 32 * wn + mfma_c_row(e, lane);
                acc[e] += (sA[s][i] * bx) * (float)c[e];
                if (kDebug) {
                    const int64_t n = n0 + i, m = m0 + rb;
                    if (n < N && m < M) dbg[(m * N + n) * nb + kb * 8 + s] = c[e] * sL[s][i];
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

hipError_t launch_gemm(const uint8_t* W, const int8_t* aqs, const uint32_t* ads, float* Y, int64_t K, int64_t N,
                       int64_t M, int64_t ldy_m, int64_t ldy_n, int32_t* dbg, hipStream_t stream) {
    const int64_t gx = (N + GEMM_BN - 1) / GEMM_BN;
    const int64_t gy = (M + GEMM_BM - 1) / GEMM_BM;
    if (gx > 0x7FFFFFFF || gy > 65535) return hipErrorInvalidConfiguration;
    if (dbg)
        hipLaunchKernelGGL(gemm_iq4xs_mfma_kernel<true>, dim3((unsigned)gx, (unsigned)gy), dim3(256), 0, stream, W,
                           aqs, ads, Y, K, N, M, ldy_m, ldy_n, dbg);
    else
        hipLaunchKernelGGL(gemm_iq4xs_mfma_kernel<false>, dim3((unsigned)gx, (unsigned)gy), dim3(256), 0, stream, W,
                           aqs, ads, Y, K, N, M, ldy_m, ldy_n, dbg);
    return hipGetLastError();
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
    hipLaunchKernelGGL(probe_mfma_kernel, dim3(1), dim3(64), 0, stream, A, B, C);
    return hipGetLastError();
}

}  // namespace iq4xs
