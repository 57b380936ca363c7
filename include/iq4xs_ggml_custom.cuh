// iq4xs_ggml_custom.cuh -- drop-in for the reference patch's two ggml headers
// custom_gfx1100/gemm_iq4xs.cuh (patches/0001-gfx1100-mul-mat-custom.patch:56-155)
// and custom_gfx1100/gemv_iq4xs.cuh (patch:156-281).
//
// The patch's hooks in mmq.cu (patch:299-306) and mmvq.cu (patch:327-334)
// call custom_gemm_iq4xs_can_handle / _dispatch and custom_gemv_iq4xs_can_handle
// / _dispatch with ggml's own types (ggml_type, const block_iq4_xs*,
// hipStream_t).  The inline functions below have exactly those parameter
// types and forward to the C entry points of libiq4xs_mi355x.so, which carry
// the same names with C types (int, const void*, void*).  In C++ these are
// distinct overloads: the hooks' calls match the forwarders exactly, and the
// forwarders reach the C symbols through explicit casts, so the hook bodies
// stay as the patch wrote them.  A hook falls back to stock ggml on any
// non-zero return, as before.
//
// Include it where ggml_type and block_iq4_xs are declared (ggml-cuda's
// common.cuh brings in ggml.h and ggml-common.h), in place of either header.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "iq4xs_mi355x.h"

// patch:274-277: IQ4_XS, one column, any K % 256 == 0 and any N (the patch's
// K/N whitelist is dropped).
inline bool custom_gemv_iq4xs_can_handle(int64_t K, int64_t N, int64_t M, ggml_type type) {
    return ::custom_gemv_iq4xs_can_handle(K, N, M, static_cast<int>(type));
}

// patch:278-280: y[N] = W x on ggml's src0 / src1 / dst; stream-ordered, no
// host synchronisation.
inline hipError_t custom_gemv_iq4xs_dispatch(const block_iq4_xs* W, const float* x, float* y, int64_t K, int64_t N,
                                             hipStream_t stream) {
    return static_cast<hipError_t>(
        ::custom_gemv_iq4xs_dispatch(static_cast<const void*>(W), x, y, K, N, static_cast<void*>(stream)));
}

// patch:148-151: IQ4_XS, any M >= 1, K % 256 == 0, any N.
inline bool custom_gemm_iq4xs_can_handle(int64_t K, int64_t N, int64_t M, ggml_type type) {
    return ::custom_gemm_iq4xs_can_handle(K, N, M, static_cast<int>(type));
}

// patch:152-154: ggml layout, X[m*K + k] -> Y[m*N + n].
inline hipError_t custom_gemm_iq4xs_dispatch(const block_iq4_xs* W, const float* X, float* Y, int64_t K, int64_t N,
                                             int64_t M, hipStream_t stream) {
    return static_cast<hipError_t>(
        ::custom_gemm_iq4xs_dispatch(static_cast<const void*>(W), X, Y, K, N, M, static_cast<void*>(stream)));
}
