// gxx_activation_probe.cpp - what g++ makes of the reference's AVX-512
// activation and tiled-GEMM sequences.  TEST INFRASTRUCTURE ONLY.
//
// The reference kernels cannot be compiled here (their headers include
// <cblas.h>), and their exact bits depend on the compiler: g++ fuses a
// product into the adds and subtracts that consume it (C++ defaults to
// -ffp-contract=fast), also through _mm512_add_ps / _mm512_sub_ps /
// _mm512_mul_ps, which GCC's headers define as generic vector arithmetic.
// This file issues the intrinsic sequences of
//   fast_exp_zmm / fast_tanh_zmm / sigmoid_zmm / gelu_zmm / relu_zmm
//     (include/jules/Kernel/FusedKernels.h:81-170),
//   the tiled kernel's loops and epilogue switch (:378-458), and
//   fusedGelu (:606-627)
// in the order the reference issues them, and tests/test_oracle.py builds it
// with the flags of benchmarks/bench_kernel.cpp:15-19 (plus -mavx512bw, which
// GCC 11 needs for those headers) and no -ffp-contract option, then compares
// the oracle's restatement with it bit for bit.  It needs an AVX-512F host.
#include <immintrin.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>

namespace {

enum { NONE = 0, RELU = 1, SIGMOID = 2, TANH = 3, GELU = 4 };

inline __m512 splat(float v) { return _mm512_set1_ps(v); }

// exp(x): clamp, 2^r split at floor(r), Horner in explicit fmadds, exponent
// bits times the polynomial (FusedKernels.h:90-133)
inline __m512 v_exp(__m512 x) {
    static const float horner[6] = {0.001333356f, 0.009614425f, 0.055495506f,
                                    0.240226507f, 0.693147180f, 1.0f};
    x = _mm512_max_ps(_mm512_min_ps(x, splat(88.0f)), splat(-88.0f));
    const __m512 r = _mm512_mul_ps(x, splat(1.4426950408889634f));
    const __m512 fl = _mm512_roundscale_ps(r, _MM_FROUND_FLOOR);
    const __m512 frac = _mm512_sub_ps(r, fl);
    __m512 p = splat(0.000154040f);
    for (float c : horner) p = _mm512_fmadd_ps(p, frac, splat(c));
    __m512i bits = _mm512_add_epi32(_mm512_cvttps_epi32(fl), _mm512_set1_epi32(127));
    bits = _mm512_slli_epi32(bits, 23);
    return _mm512_mul_ps(_mm512_castsi512_ps(bits), p);
}

// (e^{2x} - 1) / (e^{2x} + 1)  (:137-143)
inline __m512 v_tanh(__m512 x) {
    const __m512 e = v_exp(_mm512_mul_ps(splat(2.0f), x));
    return _mm512_div_ps(_mm512_sub_ps(e, splat(1.0f)), _mm512_add_ps(e, splat(1.0f)));
}

// 1 / (1 + e^{0 - x})  (:146-152)
inline __m512 v_sigmoid(__m512 x) {
    const __m512 e = v_exp(_mm512_sub_ps(_mm512_setzero_ps(), x));
    return _mm512_div_ps(splat(1.0f), _mm512_add_ps(splat(1.0f), e));
}

// 0.5 * (x * (1 + tanh(c * (x + d * (x * (x * x))))))  (:155-164)
inline __m512 v_gelu(__m512 x) {
    const __m512 cube = _mm512_mul_ps(x, _mm512_mul_ps(x, x));
    const __m512 u = _mm512_mul_ps(splat(0.7978845608f),
                                   _mm512_add_ps(x, _mm512_mul_ps(splat(0.044715f), cube)));
    return _mm512_mul_ps(splat(0.5f), _mm512_mul_ps(x, _mm512_add_ps(splat(1.0f), v_tanh(u))));
}

inline __m512 v_act(int act, __m512 v) {
    switch (act) {
    case RELU: return _mm512_max_ps(v, _mm512_setzero_ps());
    case GELU: return v_gelu(v);
    case SIGMOID: return v_sigmoid(v);
    case TANH: return v_tanh(v);
    default: return v;
    }
}

// the scalar-tail epilogue (:424-430)
inline float s_act(int act, float s) {
    switch (act) {
    case RELU: return std::max(s, 0.0f);
    case GELU: return 0.5f * s * (1.0f + tanhf(0.7978845608f * (s + 0.044715f * s * s * s)));
    case SIGMOID: return 1.0f / (1.0f + expf(-s));
    case TANH: return tanhf(s);
    default: return s;
    }
}

}  // namespace

extern "C" {

int probe_has_avx512f() { return __builtin_cpu_supports("avx512f") ? 1 : 0; }

// the vector-path activation on n elements, n a multiple of 16
void probe_act(int act, float* out, const float* in, int64_t n) {
    for (int64_t i = 0; i + 16 <= n; i += 16)
        _mm512_storeu_ps(out + i, v_act(act, _mm512_loadu_ps(in + i)));
}

// fusedGelu: groups of 16 through the vector helper, the rest through the
// scalar formula
void probe_fused_gelu(float* out, const float* in, int n) {
    for (int g = 0; g < n; g += 16) {
        if (g + 16 <= n) {
            _mm512_storeu_ps(out + g, v_gelu(_mm512_loadu_ps(in + g)));
            continue;
        }
        for (int j = g; j < n; j++) {
            const float x = in[j];
            out[j] = 0.5f * x * (1.0f + tanhf(0.7978845608f * (x + 0.044715f * x * x * x)));
        }
    }
}

// the tiled kernel: C zeroed, tile rows / columns / K slices, 16-wide column
// blocks chained with explicit fmadds and reloaded between K slices, scalar
// columns past the last block with `s += a * b`, the activation applied in
// the slice where tkk + tk >= K
void probe_tiled(const float* A, const float* B, float* C, int M, int N, int K, int tm, int tn,
                 int tk, int act) {
    std::memset(C, 0, sizeof(float) * (size_t)M * N);
    // int index arithmetic as in the reference, so that g++ makes the same
    // vectorisation choices for the scalar columns
    for (int r0 = 0; r0 < M; r0 += tm) {
        const int rows = std::min(tm, M - r0);
        for (int c0 = 0; c0 < N; c0 += tn) {
            const int cols = std::min(tn, N - c0);
            for (int k0 = 0; k0 < K; k0 += tk) {
                const int depth = std::min(tk, K - k0);
                for (int i = 0; i < rows; i++) {
                    int j = 0;
                    for (; j + 15 < cols; j += 16) {
                        __m512 acc = _mm512_loadu_ps(&C[(r0 + i) * N + (c0 + j)]);
                        for (int kk = 0; kk < depth; kk++)
                            acc = _mm512_fmadd_ps(_mm512_set1_ps(A[(r0 + i) * K + (k0 + kk)]),
                                                  _mm512_loadu_ps(&B[(k0 + kk) * N + (c0 + j)]), acc);
                        if (k0 + tk >= K) acc = v_act(act, acc);
                        _mm512_storeu_ps(&C[(r0 + i) * N + (c0 + j)], acc);
                    }
                    for (; j < cols; j++) {
                        float s = C[(r0 + i) * N + (c0 + j)];
                        for (int kk = 0; kk < depth; kk++)
                            s += A[(r0 + i) * K + (k0 + kk)] * B[(k0 + kk) * N + (c0 + j)];
                        if (k0 + tk >= K) s = s_act(act, s);
                        C[(r0 + i) * N + (c0 + j)] = s;
                    }
                }
            }
        }
    }
}

}  // extern "C"
