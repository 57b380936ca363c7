// quantize_q8_1.hip -- fp32 activations -> Q8_1 on gfx950.
//
// Semantics: real_stock_dp4a_comparator.hip:230-264 (device quantiser) and
// :278-306 (batched over columns).  Per 32-element block:
//   amax = max|x|, sum = sum x (pairwise tree: x[t]+x[t+16], then +8, +4,
//   +2, +1 -- the reference's xor butterfly seen from lane 0), d = amax/127
//   (IEEE division), q = amax ? (int8)roundf(x/d) : 0, ds = rtz-half2(d, sum).
//
// MI355X mapping:
//   layout MK (X[m*K+k], ggml src1 and bs=1 vectors): eight lanes per block,
//     four elements and four divisions per lane, tree finished with DPP
//     steps (quantize_q8_1_rows_kernel);
//   layout KM (X[k*M+m], standalone API): one lane per block, lanes walk
//     consecutive columns m so each of the 32 loads of a wave covers 64
//     consecutive floats; the tree is evaluated in registers.
#include "iq4xs_device.h"
#include "iq4xs_internal.h"
#include "q8_1_block.h"

namespace iq4xs {

__device__ inline void quantize_block_regs(const float (&x)[32], uint32_t (&q)[8], uint32_t& ds) {
    float a[16], s[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) {
        a[t] = fmaxf(fabsf(x[t]), fabsf(x[t + 16]));
        s[t] = x[t] + x[t + 16];
    }
#pragma unroll
    for (int w = 8; w > 0; w >>= 1) {
#pragma unroll
        for (int t = 0; t < w; ++t) {
            a[t] = fmaxf(a[t], a[t + w]);
            s[t] = s[t] + s[t + w];
        }
    }
    const float amax = a[0];
    const float d = div127(amax);
    int c[32];
    round_codes(x, amax, d, c);
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = pack_codes4(c[4 * j], c[4 * j + 1], c[4 * j + 2], c[4 * j + 3]);
    ds = float_to_half_bits_rtz(d) | (float_to_half_bits_rtz(s[0]) << 16);
}

template <int kLayout>
__global__ __launch_bounds__(256) void quantize_q8_1_kernel(const float* __restrict__ X, int64_t K, int64_t M,
                                                            int8_t* __restrict__ qs, uint32_t* __restrict__ ds,
                                                            uint32_t* __restrict__ hq,
                                                            block_q8_1* __restrict__ blocks) {
    const int64_t nb = K / QK8_1;
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= nb * M) return;
    int64_t m, ib;
    float x[32];
    if (kLayout == LAYOUT_MK) {
        m = g / nb;
        ib = g - m * nb;
        const v4f* p = reinterpret_cast<const v4f*>(X + m * K + ib * QK8_1);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const v4f v = p[j];
            x[4 * j + 0] = v.x;
            x[4 * j + 1] = v.y;
            x[4 * j + 2] = v.z;
            x[4 * j + 3] = v.w;
        }
    } else {
        ib = g / M;
        m = g - ib * M;
        const float* p = X + ib * QK8_1 * M + m;
#pragma unroll
        for (int t = 0; t < 32; ++t) x[t] = p[(int64_t)t * M];
    }
    uint32_t q[8], dsw;
    quantize_block_regs(x, q, dsw);
    if (qs != nullptr) {
        v4i* o = reinterpret_cast<v4i*>(qs + m * K + ib * QK8_1);
        o[0] = v4i{(int)q[0], (int)q[1], (int)q[2], (int)q[3]};
        o[1] = v4i{(int)q[4], (int)q[5], (int)q[6], (int)q[7]};
        ds[m * nb + ib] = dsw;
        // fp16 pairs: word p holds elements p and p + 16
        v4i* h = reinterpret_cast<v4i*>(hq + (m * nb + ib) * 16);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            uint32_t pw[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int p = 4 * w + i;
                pw[i] = codes_to_half2((int8_t)(q[p >> 2] >> (8 * (p & 3))), (int8_t)(q[4 + (p >> 2)] >> (8 * (p & 3))));
            }
            h[w] = v4i{(int)pw[0], (int)pw[1], (int)pw[2], (int)pw[3]};
        }
    }
    if (blocks != nullptr) {
        uint32_t* o = reinterpret_cast<uint32_t*>(blocks + m * nb + ib);
        o[0] = dsw;
#pragma unroll
        for (int j = 0; j < 8; ++j) o[1 + j] = q[j];
    }
}

// Planar workspace -> 36-byte ggml blocks (debug export for bit-exact checks).
__global__ __launch_bounds__(256) void planar_to_blocks_kernel(const int8_t* __restrict__ qs,
                                                               const uint32_t* __restrict__ ds, int64_t K, int64_t M,
                                                               block_q8_1* __restrict__ blocks) {
    const int64_t nb = K / QK8_1;
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= nb * M) return;
    const int64_t m = g / nb, ib = g - m * nb;
    const uint32_t* src = reinterpret_cast<const uint32_t*>(qs + m * K + ib * QK8_1);
    uint32_t* o = reinterpret_cast<uint32_t*>(blocks + g);
    o[0] = ds[g];
#pragma unroll
    for (int j = 0; j < 8; ++j) o[1 + j] = src[j];
}

// Row-contiguous layout (ggml src1, bs=1 vectors): eight lanes per block
// (quantize_block8); whole 8-lane groups are always active together.
__global__ __launch_bounds__(256) void quantize_q8_1_rows_kernel(const float* __restrict__ X, int64_t K, int64_t M,
                                                                 int8_t* __restrict__ qs, uint32_t* __restrict__ ds,
                                                                 uint32_t* __restrict__ hq,
                                                                 block_q8_1* __restrict__ blocks) {
    const int64_t nb = K / QK8_1;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t blk = t >> 3;
    if (blk >= nb * M) return;
    const int j = q8_lane_elem((int)(t & 7));
    const int64_t m = blk / nb, ib = blk - m * nb;
    const float* p = X + m * K + ib * QK8_1 + j;
    const Q8Block8 b = quantize_block8(p[0], p[8], p[16], p[24]);
    if (qs != nullptr) {
        int8_t* o = qs + m * K + ib * QK8_1 + j;
        o[0] = (int8_t)b.q0;
        o[8] = (int8_t)b.q1;
        o[16] = (int8_t)b.q2;
        o[24] = (int8_t)b.q3;
        hq[blk * 16 + j] = codes_to_half2(b.q0, b.q2);  // elements j, j + 16
        hq[blk * 16 + j + 8] = codes_to_half2(b.q1, b.q3);  // elements j + 8, j + 24
        if (j == 0) ds[blk] = b.ds;
    }
    if (blocks != nullptr) {
        int8_t* o = blocks[blk].qs + j;
        o[0] = (int8_t)b.q0;
        o[8] = (int8_t)b.q1;
        o[16] = (int8_t)b.q2;
        o[24] = (int8_t)b.q3;
        if (j == 0) blocks[blk].ds = b.ds;
    }
}

hipError_t launch_quantize(const float* X, int64_t K, int64_t M, int layout, int8_t* qs, uint32_t* ds, uint32_t* hq,
                           block_q8_1* blocks, hipStream_t stream) {
    clear_launch_error();
    const int64_t total = (K / QK8_1) * M;
    if (layout == LAYOUT_MK) {
        const int64_t grid = (total * 8 + 255) / 256;
        if (grid > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
        hipLaunchKernelGGL(quantize_q8_1_rows_kernel, dim3((unsigned)grid), dim3(256), 0, stream, X, K, M, qs, ds,
                           hq, blocks);
        return hipGetLastError();
    }
    const int64_t grid = (total + 255) / 256;
    if (grid > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(quantize_q8_1_kernel<LAYOUT_KM>, dim3((unsigned)grid), dim3(256), 0, stream, X, K, M, qs, ds,
                       hq, blocks);
    return hipGetLastError();
}

hipError_t launch_planar_to_blocks(const int8_t* qs, const uint32_t* ds, int64_t K, int64_t M, block_q8_1* blocks,
                                   hipStream_t stream) {
    clear_launch_error();
    const int64_t total = (K / QK8_1) * M;
    const int64_t grid = (total + 255) / 256;
    if (grid > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(planar_to_blocks_kernel, dim3((unsigned)grid), dim3(256), 0, stream, qs, ds, K, M, blocks);
    return hipGetLastError();
}

}  // namespace iq4xs
