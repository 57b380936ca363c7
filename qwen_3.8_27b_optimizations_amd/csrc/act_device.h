// act_device.h -- the SwiGLU activation's arithmetic, shared by the SwiGLU
// producer (producers.hip) and the GEMV epilogue that applies it to a
// gate/up pair (gemv.hip), so that both give the same fp32 values:
//   y = silu(g) * u, silu(g) = g / (1 + exp(-g)),
//   exp by Cody-Waite reduction and a degree-7 Taylor polynomial in fused
//   multiply-adds.
// Every expression rounds as written (no contraction; division is IEEE, the
// HIP default).
#pragma once

#include <hip/hip_runtime.h>

namespace iq4xs {

// exp(x) for x <= 88.72283935546875 (+inf above); inputs below -87 are
// raised to -87 so that no result is subnormal.  ln2 = 0x1.62e4p-1 (16
// significant bits: n * head is exact) + 0x1.7f7d1cp-20.
__device__ inline float exp_cody_waite(float x) {
#pragma clang fp contract(off)
    if (x > 0x1.62e430p+6f) return __builtin_inff();
    x = (x < -87.0f) ? -87.0f : x;  // NaN compares false and passes through
    const float n = __builtin_rintf(x * 0x1.715476p+0f);
    float r = __builtin_fmaf(-n, 0x1.62e400p-1f, x);
    r = __builtin_fmaf(-n, 0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;  // 1/7!
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_ldexpf(p, (int)n);
}

__device__ inline float silu(float g) {
#pragma clang fp contract(off)
    return g / (1.0f + exp_cody_waite(-g));
}

// silu(g) * u, rounded after the product.
__device__ inline float swiglu(float g, float u) {
#pragma clang fp contract(off)
    const float s = silu(g);
    return s * u;
}

}  // namespace iq4xs
