// compat.hip -- kernels behind the reference's remaining standalone entry
// points: its FP64 comparators and the padded Q8_1 layout of its cooperative
// GEMV.  None of these is on the hot path; they exist so that every entry
// point of kernels/matmul_iq4xs that a test or bench binds has a drop-in here.
//
// FP64 comparators.  Each output is a double accumulation, in the exact loop
// order of the reference, of w * x with w = (double)(fp16 d) * (double)
// (float(ls) - 32) * (double)kvalue and x the fp32 activation:
//   stock GEMV / GEMM (stock_hip_comparator.hip:9-94): one sequential sum per
//     output over super-blocks b, sub-blocks ib, j < 16 (low nibble, then
//     high nibble) -- the order of ref_cpu.cpp:12-106, which it mirrors;
//   gfx1100 GEMV (impl_gemv_gfx1100.hip:6-93): 8 partial sums per row (one
//     per sub-block index ib, over all super-blocks), then added in ib order.
// Products and sums are rounded separately (no contraction in this file), as
// in ref_cpu.cpp, so the stock kernels reproduce its outputs bit for bit.
// These are O(N*M*K) comparators, one thread per output (the order forbids a
// parallel reduction); they are not tuned.
#include "iq4xs_device.h"
#include "iq4xs_internal.h"

#pragma clang fp contract(off)

namespace iq4xs {

// kvalues_iq4nl[i] from the packed table
__device__ inline int kvalue(int i) {
    const uint32_t w = i < 4 ? KV0 : i < 8 ? KV1 : i < 12 ? KV2 : KV3;
    return (int)(int8_t)(w >> (8 * (i & 3)));
}

__device__ inline double subblock_dl(const uint8_t* blk, int ib) {
    const v2u h = *reinterpret_cast<const v2u*>(blk);
    const float d = half_bits_to_float(h.x & 0xFFFFu);
    const int ls = subblock_ls(h.x, h.y, ib);
    return (double)d * (double)((float)ls - 32.0f);
}

// acc += sum over one sub-block: j = 0..15, weight j then weight j + 16.
// x(k) returns the activation of element k of the sub-block.
template <typename XF>
__device__ inline double subblock_fp64(const uint8_t* blk, int ib, double acc, XF x) {
    const double dl = subblock_dl(blk, ib);
    const uint8_t* qs = blk + 8 + 16 * ib;
    for (int j = 0; j < 16; ++j) {
        const uint8_t q = qs[j];
        const double wl = dl * (double)kvalue(q & 0x0F);
        const double wh = dl * (double)kvalue(q >> 4);
        const double pl = wl * (double)x(j);
        acc = acc + pl;
        const double ph = wh * (double)x(j + 16);
        acc = acc + ph;
    }
    return acc;
}

__global__ __launch_bounds__(256) void stock_fp64_kernel(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                                          float* __restrict__ Y, int64_t K, int64_t N, int64_t M) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= N * M) return;
    const int64_t n = t / M, m = t - n * M;
    const int64_t bpr = K / QK_K;
    const uint8_t* row = W + n * bpr * BLOCK_BYTES;
    double acc = 0.0;
    for (int64_t b = 0; b < bpr; ++b) {
        const uint8_t* blk = row + b * BLOCK_BYTES;
        for (int ib = 0; ib < 8; ++ib) {
            const int64_t k0 = b * QK_K + ib * 32;
            acc = subblock_fp64(blk, ib, acc, [&](int k) { return X[(k0 + k) * M + m]; });
        }
    }
    Y[n * M + m] = (float)acc;
}

// 8 lanes per row, lane = sub-block index; partials added in lane order.
__global__ __launch_bounds__(256) void gfx1100_fp64_kernel(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                                            float* __restrict__ y, int64_t K, int64_t N) {
    __shared__ double part[256];
    const int tid = threadIdx.x, ib = tid & 7;
    const int64_t row = (int64_t)blockIdx.x * 32 + (tid >> 3);
    double s = 0.0;
    if (row < N) {
        const int64_t bpr = K / QK_K;
        const uint8_t* r = W + row * bpr * BLOCK_BYTES;
        for (int64_t b = 0; b < bpr; ++b) {
            const float* xs = x + b * QK_K + ib * 32;
            s = subblock_fp64(r + b * BLOCK_BYTES, ib, s, [&](int k) { return xs[k]; });
        }
    }
    part[tid] = s;
    __syncthreads();
    if (row < N && ib == 0) {
        double acc = 0.0;
        for (int t = 0; t < 8; ++t) acc = acc + part[tid + t];
        y[row] = (float)acc;
    }
}

// 64-byte padded Q8_1 blocks (ds at byte 0, codes at 16..47;
// impl_gemv_dp4a_gfx1100.hip:60-66) -> the planar workspace of one column
// (codes, ds and fp16 code pairs).
__global__ __launch_bounds__(256) void coop_to_planar_kernel(const uint8_t* __restrict__ coop, int64_t nb,
                                                             int8_t* __restrict__ qs, uint32_t* __restrict__ ds,
                                                             uint32_t* __restrict__ hq) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t b = t >> 1;
    if (b >= nb) return;
    const int half = (int)(t & 1);
    const uint8_t* src = coop + b * 64;
    const v4i lo = *reinterpret_cast<const v4i*>(src + 16);  // elements 0..15
    const v4i hi = *reinterpret_cast<const v4i*>(src + 32);  // elements 16..31
    *reinterpret_cast<v4i*>(qs + b * QK8_1 + 16 * half) = half ? hi : lo;
    // this thread's 8 pair words: elements p, p + 16 for p = 8 * half .. + 7
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int p = 8 * half + i;
        const int a = (int8_t)((uint32_t)lo[p >> 2] >> (8 * (p & 3)));
        const int c = (int8_t)((uint32_t)hi[p >> 2] >> (8 * (p & 3)));
        w[i] = codes_to_half2(a, c);
    }
    v4i* o = reinterpret_cast<v4i*>(hq + b * 16 + 8 * half);
    o[0] = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    o[1] = v4i{(int)w[4], (int)w[5], (int)w[6], (int)w[7]};
    if (half == 0) ds[b] = *reinterpret_cast<const uint32_t*>(src);
}

static hipError_t grid_of(int64_t threads, dim3& g) {
    const int64_t n = (threads + 255) / 256;
    if (n > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
    g = dim3((unsigned)n);
    return hipSuccess;
}

hipError_t launch_stock_fp64(const uint8_t* W, const float* X, float* Y, int64_t K, int64_t N, int64_t M,
                             hipStream_t stream) {
    clear_launch_error();
    dim3 g;
    if (grid_of(N * M, g) != hipSuccess) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(stock_fp64_kernel, g, dim3(256), 0, stream, W, X, Y, K, N, M);
    return hipGetLastError();
}

hipError_t launch_gfx1100_fp64(const uint8_t* W, const float* x, float* y, int64_t K, int64_t N, hipStream_t stream) {
    clear_launch_error();
    dim3 g;
    if (grid_of(N * 8, g) != hipSuccess) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(gfx1100_fp64_kernel, g, dim3(256), 0, stream, W, x, y, K, N);
    return hipGetLastError();
}

hipError_t launch_coop_to_planar(const uint8_t* coop, int64_t nb, int8_t* qs, uint32_t* ds, uint32_t* hq,
                                 hipStream_t stream) {
    clear_launch_error();
    dim3 g;
    if (grid_of(nb * 2, g) != hipSuccess) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(coop_to_planar_kernel, g, dim3(256), 0, stream, coop, nb, qs, ds, hq);
    return hipGetLastError();
}

}  // namespace iq4xs
