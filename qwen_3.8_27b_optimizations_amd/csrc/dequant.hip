// dequant.hip -- IQ4_XS super-blocks -> fp32 weights on gfx950.
//
// Semantics (kernels/demo_iq4xs_dequant/ref_cpu.cpp:6-27, impl.hip:14-48):
//   dl = fp16(d) * (float(ls) - 32)             (exact in fp32)
//   y[32*ib + j]      = dl * float(kvalues_iq4nl[qs[16*ib + j] & 15])
//   y[32*ib + j + 16] = dl * float(kvalues_iq4nl[qs[16*ib + j] >> 4])
// Two IEEE fp32 multiplies per output, no contraction possible, so the
// outputs are bit-identical to the reference's CPU dequantiser.
//
// MI355X mapping.  The op moves 136 bytes in and 1024 bytes out per
// super-block: it is bound by HBM writes.  Each thread takes 8 qs bytes of a
// sub-block (16 codes: outputs 8 consecutive low-nibble weights and the 8
// matching high-nibble weights) and writes them as four 16-byte stores, so a
// wave writes 2 KB of contiguous output per store instruction pair; 16 threads
// share a super-block and read its 8-byte header.  Codes are decoded with the
// same v_perm lookup as the GEMV/GEMM (decode_codes_x).
#include "iq4xs_device.h"
#include "iq4xs_internal.h"

namespace iq4xs {

__global__ __launch_bounds__(256) void dequant_iq4xs_kernel(const uint8_t* __restrict__ src, float* __restrict__ dst,
                                                            int64_t n_blocks) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t b = t >> 4;
    if (b >= n_blocks) return;
    const int p = (int)(t & 15);
    const int ib = p >> 1, h = p & 1;  // sub-block, half (qs bytes 8h .. 8h+7 of the sub-block)
    const uint8_t* blk = src + b * BLOCK_BYTES;
    const v2u hd = *reinterpret_cast<const v2u*>(blk);
    const v2u q = *reinterpret_cast<const v2u*>(blk + 8 + 16 * ib + 8 * h);
    const float dl = half_bits_to_float(hd.x & 0xFFFFu) * (float)(subblock_ls(hd.x, hd.y, ib) - 32);
    uint32_t lo[2], hi[2];
    decode_codes_x(q.x, lo[0], hi[0]);
    decode_codes_x(q.y, lo[1], hi[1]);
    float* y = dst + b * QK_K + 32 * ib + 8 * h;
    v4f out[4];
#pragma unroll
    for (int w = 0; w < 2; ++w) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            out[w][k] = dl * (float)(int8_t)(lo[w] >> (8 * k));
            out[2 + w][k] = dl * (float)(int8_t)(hi[w] >> (8 * k));
        }
    }
    reinterpret_cast<v4f*>(y)[0] = out[0];
    reinterpret_cast<v4f*>(y)[1] = out[1];
    reinterpret_cast<v4f*>(y + 16)[0] = out[2];
    reinterpret_cast<v4f*>(y + 16)[1] = out[3];
}

hipError_t launch_dequant(const uint8_t* src, float* dst, int64_t n_blocks, hipStream_t stream) {
    clear_launch_error();
    const int64_t threads = n_blocks * 16;
    const int64_t grid = (threads + 255) / 256;
    if (grid > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(dequant_iq4xs_kernel, dim3((unsigned)grid), dim3(256), 0, stream, src, dst, n_blocks);
    return hipGetLastError();
}

}  // namespace iq4xs
