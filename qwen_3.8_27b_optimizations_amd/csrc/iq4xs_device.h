// iq4xs_device.h -- IQ4_XS / Q8_1 formats and the register-level arithmetic
// shared by every gfx950 kernel of this library.
//
// Formats (byte-compatible with ggml):
//   block_iq4_xs  kernels/common/block_iq4_xs.h:10-19   136 B / 256 weights
//   block_q8_1    real_stock_dp4a_comparator.hip:22-26   36 B / 32 activations
//
// Inside the library, quantised activations live in a "planar" Q8_1 buffer:
//   qs : int8   [M][K]      (256-byte aligned)
//   ds : uint32 [M][K/32]   ({trunc-fp16 d, trunc-fp16 sum}, ggml's ds word)
// so that a lane reads its 32 codes with two aligned 16-byte loads.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace iq4xs {

constexpr int QK_K = 256;
constexpr int QK8_1 = 32;
constexpr int BLOCK_BYTES = 136;
constexpr int Q8_1_BYTES = 36;

struct __attribute__((packed)) block_iq4_xs {
    uint16_t d;
    uint16_t scales_h;
    uint8_t scales_l[4];
    uint8_t qs[128];
};
static_assert(sizeof(block_iq4_xs) == BLOCK_BYTES, "block_iq4_xs is 136 bytes");

struct block_q8_1 {
    uint32_t ds;
    int8_t qs[QK8_1];
};
static_assert(sizeof(block_q8_1) == Q8_1_BYTES, "block_q8_1 is 36 bytes");

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
// 16-byte vector whose address is only known to be 8-byte aligned (the qs of
// every other 136-byte super-block); gfx950 loads it with one dwordx4.
typedef int v4i_a8 __attribute__((ext_vector_type(4), aligned(8)));

// Byte offset of the planar ds array inside a Q8_1 workspace of M columns.
__host__ __device__ inline size_t planar_ds_offset(int64_t K, int64_t M) {
    return ((size_t)(K * M) + 255u) & ~(size_t)255u;
}
// The same codes as fp16 values (exact: |q| <= 127), for the matrix-core GEMM:
// hq [M][K/32][16] uint32 at the next 256-byte boundary, word p of a block
// holding the fp16 codes of elements p (low half) and p + 16 (high half).
__host__ __device__ inline size_t planar_hq_offset(int64_t K, int64_t M) {
    return (planar_ds_offset(K, M) + (size_t)M * (size_t)(K / QK8_1) * 4u + 255u) & ~(size_t)255u;
}
__host__ __device__ inline size_t planar_bytes(int64_t K, int64_t M) {
    return planar_hq_offset(K, M) + (size_t)M * (size_t)K * 2u;
}

// Two int8 codes as an fp16 pair word (lo | hi << 16), exactly.
__device__ inline uint32_t codes_to_half2(int lo, int hi) {
    const _Float16 a = (_Float16)(short)lo, b = (_Float16)(short)hi;
    return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// Exact binary16 -> binary32 (hardware conversion; fp16 denormals are kept).
__device__ inline float half_bits_to_float(uint32_t h) {
    union {
        uint16_t u;
        _Float16 f;
    } v;
    v.u = (uint16_t)h;
    return (float)v.f;
}

// binary32 -> binary16 rounding toward zero, |x| < 2^-24 -> signed zero,
// |x| >= 65536 / Inf / NaN -> signed Inf.  This is the encoder the reference
// uses for Q8_1 ds (real_stock_dp4a_comparator.hip:43-62); written here as
// integer field arithmetic.
__host__ __device__ inline uint32_t float_to_half_bits_rtz(float f) {
    const uint32_t x = __builtin_bit_cast(uint32_t, f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int e = (int)((x >> 23) & 0xFFu) - 112;  // rebias 127 -> 15
    const uint32_t m10 = (x >> 13) & 0x3FFu;
    // selects, not branches: the subnormal shift 1 - e is clamped to 31, which
    // also gives the signed zero of e < -10 ((m10 | 0x400) < 2^11)
    const uint32_t sub = (m10 | 0x400u) >> (1 - e < 0 ? 0 : (1 - e > 31 ? 31 : 1 - e));
    const uint32_t mag = e >= 31 ? 0x7C00u : (e > 0 ? ((uint32_t)e << 10) | m10 : sub);
    return sign | mag;
}

// 6-bit scale of sub-block ib from the first 8 bytes of a super-block
// (h0 = d | scales_h << 16, h1 = scales_l[0..3]); ref_cpu.cpp:28-31.
__device__ inline int subblock_ls(uint32_t h0, uint32_t h1, int ib) {
    const uint32_t lo = (h1 >> (4 * ib)) & 0xFu;
    const uint32_t hi = (h0 >> (16 + 2 * ib)) & 0x3u;
    return (int)(lo | (hi << 4));
}

// kvalues_iq4nl (kernels/common/block_iq4_xs.h:22-24) as four little-endian
// byte quadruples: entries 0-3, 4-7, 8-11, 12-15.
constexpr uint32_t KV0 = 0xBFAD9881u;  // -127 -104  -83  -65
constexpr uint32_t KV1 = 0xF6EADDCFu;  //  -49  -35  -22  -10
constexpr uint32_t KV2 = 0x26190D01u;  //    1   13   25   38
constexpr uint32_t KV3 = 0x71594535u;  //   53   69   89  113

// Eight 4-bit codes in one dword (byte i = codes 2i, 2i+1 as lo|hi<<4) ->
// lo: 4 int8 codebook values of the low nibbles, hi: of the high nibbles.
// v_perm_b32 selects bytes of {S0:S1}: selectors 0-3 pick S1, 4-7 pick S0, so
// one perm looks up the 3 low index bits in half of the table and a third
// perm chooses between the two halves with bit 3.
__device__ inline void decode_codes(uint32_t q, uint32_t& lo, uint32_t& hi) {
    const uint32_t ia = q & 0x07070707u;
    const uint32_t ib = (q >> 4) & 0x07070707u;
    const uint32_t la = __builtin_amdgcn_perm(KV1, KV0, ia);
    const uint32_t ua = __builtin_amdgcn_perm(KV3, KV2, ia);
    const uint32_t lb = __builtin_amdgcn_perm(KV1, KV0, ib);
    const uint32_t ub = __builtin_amdgcn_perm(KV3, KV2, ib);
    const uint32_t sa = ((q >> 1) & 0x04040404u) | 0x03020100u;
    const uint32_t sb = ((q >> 5) & 0x04040404u) | 0x03020100u;
    lo = __builtin_amdgcn_perm(ua, la, sa);
    hi = __builtin_amdgcn_perm(ub, lb, sb);
}

__device__ inline int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Cheaper exact decode through the v_perm_b32 selector "specials": selector
// bytes 8-11 return 0x00/0xFF from the sign bit of table byte 1/3/5/7, 12
// returns 0x00 and 13-15 return 0xFF.  With the raw 4-bit code n as the
// selector of table A and n^8 as the selector of table B, exactly one lookup
// hits its table and the other yields a known special byte; the tables below
// are the (unique) pair for which A(n) ^ B(n^8) == kvalues_iq4nl[n] for all n.
// Five index ops + four perms + two xors decode eight codes (vs thirteen ops
// with the two-level lookup above).
constexpr uint32_t KXA0 = 0x40529881u, KXA1 = 0x091522cfu;
constexpr uint32_t KXB0 = 0x26190dfeu, KXB1 = 0x8ea6ba35u;

__device__ inline void decode_codes_x(uint32_t q, uint32_t& lo, uint32_t& hi) {
    const uint32_t nl = q & 0x0F0F0F0Fu;
    const uint32_t xl = (q ^ 0x08080808u) & 0x0F0F0F0Fu;
    const uint32_t t = q >> 4;
    const uint32_t nh = t & 0x0F0F0F0Fu;
    const uint32_t xh = (t ^ 0x08080808u) & 0x0F0F0F0Fu;
    lo = __builtin_amdgcn_perm(KXA1, KXA0, nl) ^ __builtin_amdgcn_perm(KXB1, KXB0, xl);
    hi = __builtin_amdgcn_perm(KXA1, KXA0, nh) ^ __builtin_amdgcn_perm(KXB1, KXB0, xh);
}

// fp32 sum over the 64 lanes of a wave (DPP inside rows of 16, then one
// readlane per row); the result is wave-uniform.
__device__ inline float wave_sum_dpp(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, true));
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (r0 + r1) + (r2 + r3);
}

// Integer dot of one 32-weight sub-block: 16 qs bytes (w) against the 32
// Q8_1 codes of the matching activation block (a = bytes 0-15, b = 16-31).
// Weight j (j<16) is the low nibble of qs byte j, weight j+16 its high nibble
// (ref_cpu.cpp:35-46).
__device__ inline int subblock_dot(const v4i& w, const v4i& a, const v4i& b) {
    int s = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t lo, hi;
        decode_codes((uint32_t)w[j], lo, hi);
        s = dot4(lo, (uint32_t)a[j], s);
        s = dot4(hi, (uint32_t)b[j], s);
    }
    return s;
}

// Full-wave (64-lane) sum; every lane receives the total.
__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

}  // namespace iq4xs
