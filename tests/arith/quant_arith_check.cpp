// Exhaustive host check of two pieces of the Q8_1 quantiser's device
// arithmetic, compiled from the library's own headers:
//   * div127(a) == a / 127.0f (IEEE division, round to nearest) for every
//     non-negative binary32 a (2^31 patterns: zero, denormals, normals, Inf, NaN);
//   * float_to_half_bits_rtz(f) == the oracle's truncating fp16 encoder
//     (orc_fp32_to_fp16_trunc, the restatement of the reference's
//     real_stock_dp4a_comparator.hip:43-62) for all 2^32 binary32 patterns.
// usage: quant_arith_check <liboracle_iq4xs.so>; prints the mismatch counts,
// exit status 0 when both are zero.
#include <dlfcn.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <cmath>

#include "q8_1_block.h"

int main(int argc, char** argv) {
    if (argc < 2) return 2;
    void* h = dlopen(argv[1], RTLD_NOW);
    if (!h) {
        fprintf(stderr, "%s\n", dlerror());
        return 2;
    }
    typedef uint16_t (*enc_t)(float);
    const enc_t enc = reinterpret_cast<enc_t>(dlsym(h, "orc_fp32_to_fp16_trunc"));
    if (!enc) return 2;
    long long bad_div = 0, bad_rtz = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : bad_div, bad_rtz)
    for (long long hi = 0; hi < 65536; ++hi) {
        for (uint32_t lo = 0; lo < 65536; ++lo) {
            const uint32_t u = (uint32_t)(hi << 16) | lo;
            float f;
            memcpy(&f, &u, 4);
            if (iq4xs::float_to_half_bits_rtz(f) != enc(f)) ++bad_rtz;
            if (u < 0x80000000u) {
                const float ref = f / 127.0f, got = iq4xs::div127(f);
                uint32_t rb, gb;
                memcpy(&rb, &ref, 4);
                memcpy(&gb, &got, 4);
                if (std::isnan(ref) ? !std::isnan(got) : rb != gb) ++bad_div;
            }
        }
    }
    printf("div127 mismatches %lld, rtz mismatches %lld\n", bad_div, bad_rtz);
    return (bad_div || bad_rtz) ? 1 : 0;
}
