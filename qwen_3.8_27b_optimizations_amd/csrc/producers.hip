// producers.hip -- ops that write a mul_mat activation, fused with its Q8_1
// quantisation, on gfx950.
//
// The reference's kernels take fp32 activations and quantise them in a
// separate launch (real_stock_dp4a_comparator.hip:230-306); in the model the
// activation is written just before by RMS_NORM + MUL (ahead of the attention
// and FFN projections) or by SWIGLU (ahead of ffn_down), ops the reference
// profiles at benchmarks/profiling/BOTTLENECK-TABLE.md:24,26,30.  Fusing the
// quantiser into them removes the fp32 round trip through HBM and one launch
// per projection group.  The Q8_1 output is the planar workspace the GEMV and
// GEMM read (codes [M][K], ds [M][K/32]).
//
// The fp32 values are defined exactly, reduction order included, so that
// the Q8_1 blocks match a CPU restatement bit for bit:
//   rms norm: h = x (+ r); ss = sum (double)(h*h) -- thread t of 1024 owns
//     4-float vectors t, t+1024, ... and adds their squares in that order,
//     then a 64-lane xor butterfly per wave (lane 0 kept) and a pairwise
//     tree over the 16 wave sums ((w0 + w1) + (w2 + w3)) + ...;
//     mean = (float)(ss / K); scale = 1/sqrtf(mean + eps);
//     y = (h * scale) * gamma.
//   swiglu: y = silu(g) * u, silu(g) = g / (1 + exp(-g)), exp by Cody-Waite
//     reduction and a degree-7 Taylor polynomial in fused multiply-adds.
// No floating-point contraction is allowed in this file: every expression
// rounds as written (division and sqrt are IEEE, the HIP default).
#include "iq4xs_device.h"
#include "iq4xs_internal.h"
#include "act_device.h"
#include "q8_1_block.h"
#include "rms_device.h"

#pragma clang fp contract(off)

namespace iq4xs {

// exp_cody_waite, silu and swiglu: act_device.h (shared with the GEMV's SwiGLU epilogue).

// One 32-element block by the 8-lane group of lane L: values y at j, j+8,
// j+16, j+24 (j = q8_lane_elem(L)) -> codes, ds and the fp16 code pairs
// (word p = elements p, p + 16) of the block in the planar workspace.
__device__ inline void store_block8(const Q8Block8& b, int8_t* q, uint32_t* ds, uint32_t* hq, int j) {
    q[0] = (int8_t)b.q0;
    q[8] = (int8_t)b.q1;
    q[16] = (int8_t)b.q2;
    q[24] = (int8_t)b.q3;
    hq[j] = codes_to_half2(b.q0, b.q2);
    hq[j + 8] = codes_to_half2(b.q1, b.q3);
    if (j == 0) *ds = b.ds;
}

// y = silu(g) * u over M rows of K; 8 lanes per 32-element block.
__global__ __launch_bounds__(256) void swiglu_q8_1_kernel(const float* __restrict__ G, const float* __restrict__ U,
                                                          int64_t n_blocks, int8_t* __restrict__ qs,
                                                          uint32_t* __restrict__ ds, uint32_t* __restrict__ hq) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t blk = t >> 3;
    if (blk >= n_blocks) return;  // whole 8-lane groups leave together
    const int j = q8_lane_elem((int)(t & 7));
    const int64_t e = blk * QK8_1 + j;
    float y[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        y[i] = swiglu(G[e + 8 * i], U[e + 8 * i]);
    }
    store_block8(quantize_block8(y[0], y[1], y[2], y[3]), qs + e, ds + blk, hq + blk * 16, j);
}

// One work-group of RMS_THREADS threads (16 waves) per row, with the
// arithmetic of rms_device.h.  Pass 1 forms h (writing it to H when asked)
// and reduces its sum of squares; pass 2 quantises y block by block, 8 lanes
// per block.  A thread's loads for up to RMS_BATCH vectors are issued before
// any of its stores, so the row streams in one or two round trips even though
// H may alias X or R.  With kLds (K <= RMS_LDS_MAX) h is staged in LDS for
// pass 2; otherwise pass 2 re-reads it (from H, or recomputes x + r).
constexpr int64_t RMS_LDS_MAX = 32768;  // up to 128 KB of LDS per row

template <bool kLds, bool kRes, bool kGain>
__global__ __launch_bounds__(RMS_THREADS) void rms_norm_q8_1_kernel(const float* X, const float* R, float* H,
                                                                    const float* __restrict__ gamma, float eps,
                                                                    int64_t K, int8_t* __restrict__ qs,
                                                                    uint32_t* __restrict__ ds,
                                                                    uint32_t* __restrict__ hq) {
    extern __shared__ float sh[];  // kLds: h[K]
    __shared__ double part[RMS_WAVES];
    const int64_t m = blockIdx.x;
    const int t = threadIdx.x;
    const float* x = X + m * K;
    const float* r = kRes ? R + m * K : nullptr;
    float* h = H ? H + m * K : nullptr;

    double acc = 0.0;
    for (int64_t k0 = 4 * t; k0 < K; k0 += 4 * RMS_THREADS * RMS_BATCH) {
        RmsBatch b;
        rms_load<kRes>(b, x, r, k0, K);
        acc = rms_accumulate<kRes, kLds>(b, h, sh, k0, K, acc);
    }
    // pass 2's gains: this thread's first block is fetched now (clamped, so
    // unconditional), each next one an iteration ahead
    const int64_t nb = K / QK8_1;
    const int j = q8_lane_elem(t & 7);
    constexpr int STEP = RMS_THREADS / 8;
    const int64_t b0 = t >> 3;
    float gcur[4];
    if (kGain) {
        const int64_t e = (b0 < nb ? b0 : nb - 1) * QK8_1 + j;
#pragma unroll
        for (int i = 0; i < 4; ++i) gcur[i] = gamma[e + 8 * i];
    }
    const float scale = rms_scale(rms_reduce(acc, part, t), K, eps);

    const float* src = kLds ? sh : (h ? h : x);
    for (int64_t b = b0; b < nb; b += STEP) {  // uniform per 8-lane group
        const int64_t e = b * QK8_1 + j;
        float gnext[4];
        if (kGain) {
            const int64_t bn = b + STEP < nb ? b + STEP : nb - 1;
#pragma unroll
            for (int i = 0; i < 4; ++i) gnext[i] = gamma[bn * QK8_1 + j + 8 * i];
        }
        float y[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v = src[e + 8 * i];
            if (!kLds && !h && kRes) v = v + r[e + 8 * i];
            y[i] = rms_y<kGain>(v, scale, kGain ? gcur[i] : 0.0f);
        }
        store_block8(quantize_block8(y[0], y[1], y[2], y[3]), qs + m * K + e, ds + m * nb + b,
                     hq + (m * nb + b) * 16, j);
        if (kGain) {
#pragma unroll
            for (int i = 0; i < 4; ++i) gcur[i] = gnext[i];
        }
    }
}

template <bool kLds>
void launch_rms(bool res, bool gain, dim3 grid, dim3 block, size_t lds, hipStream_t stream, const float* X,
                const float* R, float* H, const float* gamma, float eps, int64_t K, int8_t* qs, uint32_t* ds,
                uint32_t* hq) {
    if (res && gain)
        hipLaunchKernelGGL((rms_norm_q8_1_kernel<kLds, true, true>), grid, block, lds, stream, X, R, H, gamma, eps, K,
                           qs, ds, hq);
    else if (res)
        hipLaunchKernelGGL((rms_norm_q8_1_kernel<kLds, true, false>), grid, block, lds, stream, X, R, H, gamma, eps, K,
                           qs, ds, hq);
    else if (gain)
        hipLaunchKernelGGL((rms_norm_q8_1_kernel<kLds, false, true>), grid, block, lds, stream, X, R, H, gamma, eps, K,
                           qs, ds, hq);
    else
        hipLaunchKernelGGL((rms_norm_q8_1_kernel<kLds, false, false>), grid, block, lds, stream, X, R, H, gamma, eps,
                           K, qs, ds, hq);
}

hipError_t launch_swiglu_q8_1(const float* G, const float* U, int64_t K, int64_t M, int8_t* qs, uint32_t* ds,
                              uint32_t* hq, hipStream_t stream) {
    clear_launch_error();
    const int64_t n_blocks = (K / QK8_1) * M;
    const int64_t grid = (n_blocks * 8 + 255) / 256;
    if (grid > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(swiglu_q8_1_kernel, dim3((unsigned)grid), dim3(256), 0, stream, G, U, n_blocks, qs, ds, hq);
    return hipGetLastError();
}

hipError_t launch_rms_norm_q8_1(const float* X, const float* R, float* H, const float* gamma, float eps, int64_t K,
                                int64_t M, int8_t* qs, uint32_t* ds, uint32_t* hq, hipStream_t stream) {
    clear_launch_error();
    if (M > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
    const dim3 grid((unsigned)M), block(RMS_THREADS);
    const size_t lds = (size_t)K * sizeof(float);
    if (K <= RMS_LDS_MAX) {
        if (lds > 65536) {  // beyond the default dynamic-LDS limit of a launch
            const int cap = (int)(RMS_LDS_MAX * sizeof(float));
            const void* fns[4] = {reinterpret_cast<const void*>(&rms_norm_q8_1_kernel<true, false, false>),
                                  reinterpret_cast<const void*>(&rms_norm_q8_1_kernel<true, false, true>),
                                  reinterpret_cast<const void*>(&rms_norm_q8_1_kernel<true, true, false>),
                                  reinterpret_cast<const void*>(&rms_norm_q8_1_kernel<true, true, true>)};
            for (const void* f : fns) {
                const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, cap);
                if (e != hipSuccess) return e;
            }
        }
        launch_rms<true>(R != nullptr, gamma != nullptr, grid, block, lds, stream, X, R, H, gamma, eps, K, qs, ds, hq);
    } else {
        launch_rms<false>(R != nullptr, gamma != nullptr, grid, block, 0, stream, X, R, H, gamma, eps, K, qs, ds, hq);
    }
    return hipGetLastError();
}

}  // namespace iq4xs
