// q8_1_block.h -- device-side Q8_1 quantisation of one 32-element block by
// eight cooperating lanes, shared by the standalone quantiser and the fused
// GEMV prologue.
//
// Semantics (real_stock_dp4a_comparator.hip:230-264): amax = max|x|,
// sum = pairwise tree x[t]+x[t+16], +8, +4, +2, +1; d = amax/127 (IEEE);
// q = amax ? (int8)roundf(x/d) : 0; ds = {rtz-fp16(d), rtz-fp16(sum)}.
//
// Lane L (0..7) of a group holds x[j], x[j+8], x[j+16], x[j+24] with
// j = q8_lane_elem(L) = L for L < 4 and 11 - L for L >= 4: the +16 and +8
// levels of the tree are in-lane, and with lanes 4..7 reversed the +4, +2
// and +1 levels are exactly DPP row_half_mirror (L <-> 7-L), quad_perm xor 2
// and quad_perm xor 1 -- VALU modifiers, no LDS round trip.  Callers keep
// whole, 8-aligned lane groups active together.
#pragma once

#include "iq4xs_device.h"

namespace iq4xs {

__host__ __device__ constexpr int q8_lane_elem(int L) { return L < 4 ? L : 11 - L; }

template <int CTRL>
__device__ inline float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// roundf(x / d) with IEEE semantics (the exact path of round_codes below).
static __device__ __attribute__((noinline)) int round_div_exact(float x, float d) { return (int)roundf(x / d); }

// d = a / 127 rounded exactly as the IEEE division rounds it, without the
// division sequence: q = RN(a * RN(1/127)), the residual a - 127 q (exact in
// one FMA), then RN(q + residual * RN(1/127)).  This equals RN(a / 127) for
// every non-negative binary32 a, denormals included (an exhaustive host check
// is part of the CPU tests); for a = Inf or NaN the residual is NaN and q
// (Inf, NaN) is the quotient.
__host__ __device__ inline float div127(float a) {
    constexpr float R = 1.0f / 127.0f;
    const float q = a * R;
    const float r = __builtin_fmaf(-q, 127.0f, a);
    return r == r ? __builtin_fmaf(r, R, q) : q;
}

// The codes roundf(x[i] / d) of N values of one block with amax a and
// d = div127(a), for |x| <= 127 d.  p = x * rcp(d) lies within 2^-15 of x/d
// (|x/d| <= 128, v_rcp_f32 error <= 1 ulp) and RN(x/d) within 2^-17 of x/d,
// so both round to the same integer unless x/d is within 2^-14 of a
// half-integer.  A lane with any such value -- or any non-finite p, where the
// comparison is false -- takes one branch that recomputes all N by the exact
// division (rare); a = 0 gives zero codes.  The product is clamped before the
// conversion so that the conversion is defined on every lane.
template <int N>
__device__ inline void round_codes(const float (&x)[N], float a, float d, int (&q)[N]) {
    const float r = __builtin_amdgcn_rcpf(d);
    bool slow = false;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const float p = x[i] * r;
        const float ap = fabsf(p);
        const float f = ap - floorf(ap);
        slow |= !(fabsf(f - 0.5f) >= 0x1p-14f);
        const float pc = fminf(fmaxf(p, -128.0f), 128.0f);
        q[i] = a != 0.0f ? (int)(pc + copysignf(0.5f, pc)) : 0;
    }
    if (slow && a != 0.0f) {
#pragma unroll
        for (int i = 0; i < N; ++i) q[i] = round_div_exact(x[i], d);
    }
}

// Four int8 codes (low bytes of c0..c3) as one little-endian word.
__device__ inline uint32_t pack_codes4(int c0, int c1, int c2, int c3) {
    return ((uint32_t)c0 & 0xFFu) | (((uint32_t)c1 & 0xFFu) << 8) | (((uint32_t)c2 & 0xFFu) << 16) |
           ((uint32_t)c3 << 24);
}

struct Q8Block8 {
    int q0, q1, q2, q3;  // codes of x[j], x[j+8], x[j+16], x[j+24]
    uint32_t ds;         // rtz-fp16(d) | rtz-fp16(sum) << 16 (identical in all 8 lanes)
};

__device__ inline Q8Block8 quantize_block8(float x0, float x1, float x2, float x3) {
    float a = fmaxf(fmaxf(fabsf(x0), fabsf(x2)), fmaxf(fabsf(x1), fabsf(x3)));
    float s = (x0 + x2) + (x1 + x3);
    a = fmaxf(a, dpp_f32<0x141>(a));  // row_half_mirror: element t with t + 4
    s = s + dpp_f32<0x141>(s);
    a = fmaxf(a, dpp_f32<0x4E>(a));   // quad_perm [2,3,0,1]: t with t + 2
    s = s + dpp_f32<0x4E>(s);
    a = fmaxf(a, dpp_f32<0xB1>(a));   // quad_perm [1,0,3,2]: t with t + 1
    s = s + dpp_f32<0xB1>(s);
    const float d = div127(a);
    const float x[4] = {x0, x1, x2, x3};
    int q[4];
    round_codes(x, a, d, q);
    return Q8Block8{q[0], q[1], q[2], q[3], float_to_half_bits_rtz(d) | (float_to_half_bits_rtz(s) << 16)};
}

// The same block held by four cooperating lanes (an aligned quad), eight
// consecutive elements each: lane L holds x[8L .. 8L+7].  amax is the max
// over the quad (DPP quad_perm xor 2, xor 1; max is exact in any order), so
// d and every code are those of quantize_block8; the block sum is not formed.
// Returns the eight codes as bytes, x[8L] in the lowest, and rtz-fp16(d).
struct Q8Quad {
    uint32_t q_lo, q_hi;  // codes of x[8L .. 8L+3], x[8L+4 .. 8L+7]
    uint32_t d_bits;      // rtz-fp16(d) (identical in the four lanes)
};

__device__ inline Q8Quad quantize_quad8(const float (&x)[8]) {
    float a = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
    a = fmaxf(a, fmaxf(fmaxf(fabsf(x[4]), fabsf(x[5])), fmaxf(fabsf(x[6]), fabsf(x[7]))));
    a = fmaxf(a, dpp_f32<0x4E>(a));  // quad_perm [2,3,0,1]
    a = fmaxf(a, dpp_f32<0xB1>(a));  // quad_perm [1,0,3,2]
    const float d = div127(a);
    int q[8];
    round_codes(x, a, d, q);
    return Q8Quad{pack_codes4(q[0], q[1], q[2], q[3]), pack_codes4(q[4], q[5], q[6], q[7]), float_to_half_bits_rtz(d)};
}

}  // namespace iq4xs
