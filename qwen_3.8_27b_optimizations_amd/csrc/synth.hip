// synth.hip -- seeded synthetic IQ4_XS weights and fp32 activations made on
// the device, so multi-GB benchmark inputs never cross PCIe.
//
// Recipe (counter-based; block g / element i are independent):
//   draw(seed, stream, ctr) = mix64(mix64(seed ^ stream*0xD1B54A32D192ED03) ^ ctr)
//   with mix64 the splitmix64 finaliser (Steele, Lea, Flood, OOPSLA 2014).
//   Weights, block g, stream 1:
//     draw 18g    : d = rtz-fp16((float)(r >> 40) * (0.015/2^24) + 0.005)
//     draw 18g+1  : 6-bit scales, ls_ib = (r >> 6*ib) & 63
//     draw 18g+2+w: qs bytes 8w..8w+7 (little-endian), w = 0..15
//   Activations, element i: Box-Muller on draws i of streams 2 and 3; with
//   outliers, x20 where draw i of stream 4 is 0 mod 100.
// Weights are bit-identical to any other implementation of this recipe;
// activations depend on the device's double-precision log/cos.
#include "iq4xs_device.h"
#include "iq4xs_internal.h"

namespace iq4xs {

__device__ inline uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ inline uint64_t draw(uint64_t seed, uint64_t stream, uint64_t ctr) {
    return mix64(mix64(seed ^ (stream * 0xD1B54A32D192ED03ull)) ^ ctr);
}

__device__ inline float synth_d(uint64_t r0) {
#pragma clang fp contract(off)
    const float t = (float)(uint32_t)(r0 >> 40) * 8.94069671630859375e-10f;
    return t + 0.005f;
}

__global__ __launch_bounds__(256) void fill_weights_kernel(uint8_t* __restrict__ W, int64_t n_blocks, uint64_t seed,
                                                           int64_t first_block) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_blocks) return;
    const uint64_t g = (uint64_t)(first_block + i);
    uint32_t* out = reinterpret_cast<uint32_t*>(W + i * BLOCK_BYTES);  // 136 = 34 dwords, 4-byte aligned
    const uint32_t d = float_to_half_bits_rtz(synth_d(draw(seed, 1, g * 18 + 0)));
    const uint64_t r1 = draw(seed, 1, g * 18 + 1);
    uint32_t sh = 0, sl = 0;
#pragma unroll
    for (int ib = 0; ib < 8; ++ib) {
        const uint32_t ls = (uint32_t)(r1 >> (6 * ib)) & 63u;
        sl |= (ls & 0xFu) << (4 * ib);
        sh |= (ls >> 4) << (2 * ib);
    }
    out[0] = d | (sh << 16);
    out[1] = sl;
#pragma unroll 4
    for (int w = 0; w < 16; ++w) {
        const uint64_t r = draw(seed, 1, g * 18 + 2 + (uint64_t)w);
        out[2 + 2 * w] = (uint32_t)r;
        out[3 + 2 * w] = (uint32_t)(r >> 32);
    }
}

__global__ __launch_bounds__(256) void fill_activations_kernel(float* __restrict__ x, int64_t n, uint64_t seed,
                                                               int outliers) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const double u1 = (double)((draw(seed, 2, (uint64_t)i) >> 11) + 1) * 0x1.0p-53;
    const double u2 = (double)(draw(seed, 3, (uint64_t)i) >> 11) * 0x1.0p-53;
    float v = (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925286766559 * u2));
    if (outliers && draw(seed, 4, (uint64_t)i) % 100 == 0) v *= 20.0f;
    x[i] = v;
}

hipError_t launch_fill_weights(uint8_t* W, int64_t n_blocks, uint64_t seed, int64_t first_block, hipStream_t stream) {
    clear_launch_error();
    const int64_t grid = (n_blocks + 255) / 256;
    if (grid > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(fill_weights_kernel, dim3((unsigned)grid), dim3(256), 0, stream, W, n_blocks, seed,
                       first_block);
    return hipGetLastError();
}

hipError_t launch_fill_activations(float* x, int64_t n, uint64_t seed, int outliers, hipStream_t stream) {
    clear_launch_error();
    const int64_t grid = (n + 255) / 256;
    if (grid > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(fill_activations_kernel, dim3((unsigned)grid), dim3(256), 0, stream, x, n, seed, outliers);
    return hipGetLastError();
}

}  // namespace iq4xs
