// rms_device.h -- the fp32/fp64 arithmetic of the RMS-norm producer, shared by
// its own kernel (producers.hip) and by the GEMV prologue that fuses it
// (gemv.hip), so that both give the same bits by construction.
//
// Order (a work-group of RMS_THREADS threads per row):
//   h = x (+ r); thread t owns 4-float vectors t, t+1024, ... and adds the
//   squares of their elements, as doubles, in that order; a 64-lane xor
//   butterfly per wave (lane 0 kept) and a pairwise tree over the 16 wave
//   sums ((w0 + w1) + (w2 + w3)) + ... give ss;
//   mean = (float)(ss / K); scale = 1/sqrtf(mean + eps); y = (h * scale) * gamma.
// No contraction: every expression rounds as written.
#pragma once

#include "iq4xs_device.h"

namespace iq4xs {

constexpr int RMS_THREADS = 1024;
constexpr int RMS_WAVES = RMS_THREADS / 64;
constexpr int RMS_BATCH = 2;  // two rounds reach K = 8192 (rms at decode shapes); four measured 8 % slower
// one pass-1 batch of a thread covers K up to this
constexpr int64_t RMS_ONE_BATCH_K = 4 * (int64_t)RMS_THREADS * RMS_BATCH;

struct RmsBatch {
    v4f v[RMS_BATCH];
    v4f w[RMS_BATCH];
};

// Pass-1 loads of the batch whose first vector starts at k0 (= 4t + a
// multiple of 4 * RMS_THREADS * RMS_BATCH); indices past K are clamped, so
// every load is unconditional.
template <bool kRes>
__device__ inline void rms_load(RmsBatch& b, const float* x, const float* r, int64_t k0, int64_t K) {
#pragma unroll
    for (int u = 0; u < RMS_BATCH; ++u) {
        const int64_t k = k0 + 4 * RMS_THREADS * u < K ? k0 + 4 * RMS_THREADS * u : K - 4;
        b.v[u] = *reinterpret_cast<const v4f*>(x + k);
        if (kRes) b.w[u] = *reinterpret_cast<const v4f*>(r + k);
    }
}

// Pass-1 arithmetic of a loaded batch: h = x (+ r), stored to h (global, when
// non-null) and to sh (LDS, with kLds), its squares added to acc.
template <bool kRes, bool kLds>
__device__ inline double rms_accumulate(RmsBatch& b, float* h, float* sh, int64_t k0, int64_t K, double acc) {
#pragma clang fp contract(off)
#pragma unroll
    for (int u = 0; u < RMS_BATCH; ++u) {
        const int64_t k = k0 + 4 * RMS_THREADS * u;
        if (k < K) {
            if (kRes) b.v[u] = v4f{b.v[u].x + b.w[u].x, b.v[u].y + b.w[u].y, b.v[u].z + b.w[u].z, b.v[u].w + b.w[u].w};
            if (h) *reinterpret_cast<v4f*>(h + k) = b.v[u];
            if (kLds) *reinterpret_cast<v4f*>(sh + k) = b.v[u];
            const float s0 = b.v[u].x * b.v[u].x, s1 = b.v[u].y * b.v[u].y, s2 = b.v[u].z * b.v[u].z,
                        s3 = b.v[u].w * b.v[u].w;
            acc = acc + (double)s0;
            acc = acc + (double)s1;
            acc = acc + (double)s2;
            acc = acc + (double)s3;
        }
    }
    return acc;
}

// A double moved across lanes by one DPP control (both halves).
template <int kCtrl>
__device__ inline double dpp_f64(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)b, kCtrl, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(b >> 32), kCtrl, 0xF, 0xF, false);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// The work-group's sum of squares from every thread's acc (part: RMS_WAVES
// doubles of LDS).  Contains the __syncthreads that also orders pass 1's
// stores before pass 2's reads.
//
// The wave sum is the xor butterfly acc += acc[lane ^ o], o = 32, 16, ..., 1.
// o = 32 and 16 cross DPP rows and go through ds_bpermute; the other four
// steps are DPP moves: row_ror:8 is lane ^ 8 within a row; row_ror:4 reads
// lane (i + 4) mod 16, which differs from i ^ 4 by 8, and after the o = 8
// step every lane holds the same value as its lane ^ 8 (a + b = b + a
// exactly), so it reads the value lane ^ 4 holds; quad_perm [2,3,0,1] and
// [1,0,3,2] are lane ^ 2 and lane ^ 1.  Every lane therefore adds the same
// two doubles as the shuffle butterfly: the same bits, without four of its
// six LDS round trips.
__device__ inline double rms_reduce(double acc, double* part, int t) {
#pragma clang fp contract(off)
    acc = acc + __shfl_xor(acc, 32, 64);
    acc = acc + __shfl_xor(acc, 16, 64);
    acc = acc + dpp_f64<0x128>(acc);  // row_ror:8
    acc = acc + dpp_f64<0x124>(acc);  // row_ror:4
    acc = acc + dpp_f64<0x4E>(acc);   // quad_perm [2,3,0,1]
    acc = acc + dpp_f64<0xB1>(acc);   // quad_perm [1,0,3,2]
    if ((t & 63) == 0) part[t >> 6] = acc;
    __syncthreads();
    double p[RMS_WAVES];
#pragma unroll
    for (int i = 0; i < RMS_WAVES; ++i) p[i] = part[i];
#pragma unroll
    for (int n = RMS_WAVES / 2; n > 0; n >>= 1) {
#pragma unroll
        for (int i = 0; i < n; ++i) p[i] = p[2 * i] + p[2 * i + 1];
    }
    return p[0];
}

__device__ inline float rms_scale(double ss, int64_t K, float eps) {
#pragma clang fp contract(off)
    const float mean = (float)(ss / (double)K);
    return 1.0f / __builtin_sqrtf(mean + eps);
}

// y of one element: (h * scale) * gamma, or h * scale without a gain
template <bool kGain>
__device__ inline float rms_y(float h, float scale, float g) {
#pragma clang fp contract(off)
    const float sc = h * scale;
    return kGain ? sc * g : sc;
}

}  // namespace iq4xs
