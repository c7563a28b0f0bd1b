// common.hpp - device helpers shared by the gfx950 kernels of libjules_hip.
//
// Every translation unit of the library is compiled with -ffp-contract=off:
// the activation helpers below perform the same IEEE-754 operations in the
// same order as the reference's AVX-512 helpers as g++ compiles them, so a
// multiply and an add are fused exactly where written as an fma.  Those fmas
// include the ones g++ makes at its default -ffp-contract=fast: it expands
// _mm512_add/sub/mul_ps into generic vector arithmetic and fuses a product
// into the adds and subtracts that consume it when those are its only uses
// (marked "contracted" below).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "jules_hip.h"

namespace jh {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// ---- activation epilogue ---------------------------------------------------

// fast_exp_zmm of reference FusedKernels.h:90-133, one lane, as its two
// factors: clamp to [-88,88], r = x*log2(e), floor split, degree-6 Horner in
// fma, 2^floor from exponent bits.  The result is scale*poly.
struct ExpParts {
    float scale, poly;
};
__device__ __forceinline__ ExpParts fast_exp_parts(float x) {
    x = (x < 88.0f) ? x : 88.0f;
    x = (x > -88.0f) ? x : -88.0f;
    const float r = x * 1.4426950408889634f;
    const float ri = floorf(r);
    const float rf = r - ri;
    float p = __builtin_fmaf(0.000154040f, rf, 0.001333356f);
    p = __builtin_fmaf(p, rf, 0.009614425f);
    p = __builtin_fmaf(p, rf, 0.055495506f);
    p = __builtin_fmaf(p, rf, 0.240226507f);
    p = __builtin_fmaf(p, rf, 0.693147180f);
    p = __builtin_fmaf(p, rf, 1.0f);
    const int e = ((int)ri + 127) << 23;
    return ExpParts{__int_as_float(e), p};
}

__device__ __forceinline__ float fast_exp(float x) {
    const ExpParts e = fast_exp_parts(x);
    return e.scale * e.poly;
}

// fast_tanh_zmm, reference FusedKernels.h:137-143: (e-1)/(e+1) with
// e = exp(2x); both the subtract and the add are contracted.
__device__ __forceinline__ float fast_tanh(float x) {
    const ExpParts e = fast_exp_parts(2.0f * x);
    return __fdiv_rn(__builtin_fmaf(e.scale, e.poly, -1.0f), __builtin_fmaf(e.scale, e.poly, 1.0f));
}

// sigmoid_zmm, reference FusedKernels.h:146-152: 1/(1+exp(0-x)), the add
// contracted
__device__ __forceinline__ float sigmoid(float x) {
    const ExpParts e = fast_exp_parts(0.0f - x);
    return __fdiv_rn(1.0f, __builtin_fmaf(e.scale, e.poly, 1.0f));
}

// gelu_zmm, reference FusedKernels.h:155-164; x + 0.044715*x^3 contracted
__device__ __forceinline__ float gelu(float x) {
    const float x3 = x * (x * x);
    const float inner = 0.7978845608f * __builtin_fmaf(0.044715f, x3, x);
    const float t = fast_tanh(inner);
    return 0.5f * (x * (1.0f + t));
}

// The epilogue switch of the reference's vector path (FusedKernels.h:408-414)
// plus SiLU = x*sigmoid(x).  ACT is a template parameter so the switch folds.
template <int ACT>
__device__ __forceinline__ float activate(float x) {
    if constexpr (ACT == JH_ACT_RELU) return (x > 0.0f) ? x : 0.0f;  // maxps(x,0)
    else if constexpr (ACT == JH_ACT_SIGMOID) return sigmoid(x);
    else if constexpr (ACT == JH_ACT_TANH) return fast_tanh(x);
    else if constexpr (ACT == JH_ACT_GELU) return gelu(x);
    else if constexpr (ACT == JH_ACT_SILU) return x * sigmoid(x);
    else return x;
}

// ---- bf16 ---------------------------------------------------------------------

// two fp32 -> packed bf16x2, round to nearest even (v_cvt_pk_bf16_f32 on gfx950)
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2_t v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float bf16_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

}  // namespace jh

// Dispatch a runtime activation code to a template instantiation.
#define JH_DISPATCH_ACT(act, ACTC, ...)                                  \
    switch (act) {                                                      \
    case JH_ACT_NONE: { constexpr int ACTC = JH_ACT_NONE; __VA_ARGS__; } break;       \
    case JH_ACT_RELU: { constexpr int ACTC = JH_ACT_RELU; __VA_ARGS__; } break;       \
    case JH_ACT_SIGMOID: { constexpr int ACTC = JH_ACT_SIGMOID; __VA_ARGS__; } break; \
    case JH_ACT_TANH: { constexpr int ACTC = JH_ACT_TANH; __VA_ARGS__; } break;       \
    case JH_ACT_GELU: { constexpr int ACTC = JH_ACT_GELU; __VA_ARGS__; } break;       \
    case JH_ACT_SILU: { constexpr int ACTC = JH_ACT_SILU; __VA_ARGS__; } break;       \
    default: break;                                                     \
    }
