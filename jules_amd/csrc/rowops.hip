// rowops.hip - row kernels: fusedSoftmax, fusedLayerNorm, fusedCrossEntropyLoss.
//
// Reference: include/jules/Kernel/FusedKernels.h:464-526 (softmax),
// :532-600 (layernorm), :766-854 (cross entropy), AVX-512 branches.  Each
// reference row is processed by one thread as 16-float vectors plus a scalar
// tail; the per-element arithmetic is kept here:
//   softmax  e = fast_exp(x - max) for j < N & ~15, expf(x - max) for the
//            tail; out = e * (1 / sum) for j < N & ~15, e / sum for the tail;
//   layernorm mean = sum / N, var = sum fma(d, d) / N, inv_std =
//            1 / sqrtf(var + eps), out = fma((x - mean) * inv_std, gamma, beta);
//   cross entropy  p = softmax row, loss_i = -logf(p[t] + 1e-10),
//            grad = (p - onehot(t)) / M, loss = sum_i loss_i / M.
// The sums are taken in a different (fixed, tree) order than the reference's
// 16 lane partials, so results match it to rounding, not bit for bit.
//
// All three are HBM-bound.  One wave owns a row; with N <= 4096 the row is
// held in registers (ELEMS elements per lane, element j = lane + 64 * t, so
// every load and store instruction covers 256 contiguous bytes), read from
// HBM once and written once.  Longer rows take three streaming passes, the
// reference's own pass structure.  Four rows per workgroup; the wave
// reductions are a fixed butterfly, so results are deterministic.
#include <cfloat>

#include "common.hpp"
#include "launch.hpp"

namespace jh {
namespace {

constexpr int ROWS_PER_BLOCK = 4;
constexpr int MAX_CACHED = 4096;  // longest row held in registers

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
// max as the reference's _mm512_max_ps(acc, x): acc > x ? acc : x
__device__ __forceinline__ float ref_max(float acc, float x) { return acc > x ? acc : x; }

// exp of the reference: fast_exp on the part of the row that fills whole
// 16-float vectors, libm expf on the tail
__device__ __forceinline__ float row_exp(float d, int j, int nv) {
    return j < nv ? fast_exp(d) : expf(d);
}
__device__ __forceinline__ float row_norm(float e, float inv, float sum, int j, int nv) {
    return j < nv ? e * inv : e / sum;
}

// ---- softmax over one row held in registers ----
template <int ELEMS>
__device__ __forceinline__ float softmax_cached(float (&v)[ELEMS], const float* x, int N,
                                                int lane) {
    const int nv = N & ~15;
    float mx = -FLT_MAX;
#pragma unroll
    for (int t = 0; t < ELEMS; ++t) {
        const int j = lane + 64 * t;
        v[t] = j < N ? x[j] : -FLT_MAX;
        mx = ref_max(mx, v[t]);
    }
    mx = wave_max(mx);
    float s = 0.0f;
#pragma unroll
    for (int t = 0; t < ELEMS; ++t) {
        const int j = lane + 64 * t;
        const float e = j < N ? row_exp(v[t] - mx, j, nv) : 0.0f;
        v[t] = e;
        s += e;
    }
    s = wave_sum(s);
    const float inv = 1.0f / s;
#pragma unroll
    for (int t = 0; t < ELEMS; ++t) v[t] = row_norm(v[t], inv, s, lane + 64 * t, nv);
    return s;
}

template <int ELEMS>
__global__ __launch_bounds__(256) void softmax_kernel(float* __restrict__ out,
                                                      const float* __restrict__ in, int M, int N) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
    if (row >= M) return;
    const float* x = in + (int64_t)row * N;
    float* y = out + (int64_t)row * N;
    float v[ELEMS];
    softmax_cached<ELEMS>(v, x, N, lane);
#pragma unroll
    for (int t = 0; t < ELEMS; ++t) {
        const int j = lane + 64 * t;
        if (j < N) y[j] = v[t];
    }
}

// rows longer than MAX_CACHED: max pass, exp + sum pass (e stored in out),
// normalize pass - the reference's passes 1a, 1b, 2
__global__ __launch_bounds__(256) void softmax_stream_kernel(float* out, const float* in, int M,
                                                             int N) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
    if (row >= M) return;
    const float* x = in + (int64_t)row * N;
    float* y = out + (int64_t)row * N;
    const int nv = N & ~15;
    float mx = -FLT_MAX;
    for (int j = lane; j < N; j += 64) mx = ref_max(mx, x[j]);
    mx = wave_max(mx);
    float s = 0.0f;
    for (int j = lane; j < N; j += 64) {
        const float e = row_exp(x[j] - mx, j, nv);
        y[j] = e;
        s += e;
    }
    s = wave_sum(s);
    const float inv = 1.0f / s;
    for (int j = lane; j < N; j += 64) y[j] = row_norm(y[j], inv, s, j, nv);
}

// ---- layernorm ----
template <int ELEMS>
__global__ __launch_bounds__(256) void layernorm_kernel(float* __restrict__ out,
                                                        const float* __restrict__ in,
                                                        const float* __restrict__ gamma,
                                                        const float* __restrict__ beta, int M,
                                                        int N, float eps) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
    if (row >= M) return;
    const float* x = in + (int64_t)row * N;
    float* y = out + (int64_t)row * N;
    float v[ELEMS];
    float s = 0.0f;
#pragma unroll
    for (int t = 0; t < ELEMS; ++t) {
        const int j = lane + 64 * t;
        v[t] = j < N ? x[j] : 0.0f;
        s += v[t];
    }
    const float mean = wave_sum(s) / (float)N;
    float q = 0.0f;
#pragma unroll
    for (int t = 0; t < ELEMS; ++t) {
        const int j = lane + 64 * t;
        const float d = v[t] - mean;
        q = j < N ? __builtin_fmaf(d, d, q) : q;
    }
    const float var = wave_sum(q) / (float)N;
    const float inv_std = 1.0f / sqrtf(var + eps);
#pragma unroll
    for (int t = 0; t < ELEMS; ++t) {
        const int j = lane + 64 * t;
        if (j < N) y[j] = __builtin_fmaf((v[t] - mean) * inv_std, gamma[j], beta[j]);
    }
}

__global__ __launch_bounds__(256) void layernorm_stream_kernel(float* out, const float* in,
                                                               const float* __restrict__ gamma,
                                                               const float* __restrict__ beta,
                                                               int M, int N, float eps) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
    if (row >= M) return;
    const float* x = in + (int64_t)row * N;
    float* y = out + (int64_t)row * N;
    float s = 0.0f;
    for (int j = lane; j < N; j += 64) s += x[j];
    const float mean = wave_sum(s) / (float)N;
    float q = 0.0f;
    for (int j = lane; j < N; j += 64) {
        const float d = x[j] - mean;
        q = __builtin_fmaf(d, d, q);
    }
    const float var = wave_sum(q) / (float)N;
    const float inv_std = 1.0f / sqrtf(var + eps);
    for (int j = lane; j < N; j += 64) y[j] = __builtin_fmaf((x[j] - mean) * inv_std, gamma[j], beta[j]);
}

// ---- cross entropy: grad rows and per-row losses (row_loss[M]) ----
// A target outside [0, N) gives a NaN row loss and no onehot subtraction
// (the reference indexes out of bounds).
__device__ __forceinline__ float ce_grad(float p, int j, int t, float fm) {
    return (j == t ? p - 1.0f : p) / fm;
}

template <int ELEMS>
__global__ __launch_bounds__(256) void cross_entropy_kernel(const float* __restrict__ logits,
                                                            const int32_t* __restrict__ targets,
                                                            float* __restrict__ grad,
                                                            float* __restrict__ row_loss, int M,
                                                            int N) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
    if (row >= M) return;
    const float* x = logits + (int64_t)row * N;
    float* g = grad + (int64_t)row * N;
    float v[ELEMS];
    softmax_cached<ELEMS>(v, x, N, lane);
    const int t = targets[row];
    const bool valid = t >= 0 && t < N;
    // p[t]: held by lane t % 64 in slot t / 64
    float pt = 0.0f;
#pragma unroll
    for (int k = 0; k < ELEMS; ++k)
        if (lane + 64 * k == t) pt = v[k];
    pt = wave_sum(pt);  // one lane holds it, the others 0
    const float fm = (float)M;
#pragma unroll
    for (int k = 0; k < ELEMS; ++k) {
        const int j = lane + 64 * k;
        if (j < N) g[j] = ce_grad(v[k], j, valid ? t : -1, fm);
    }
    if (lane == 0) row_loss[row] = valid ? -logf(pt + 1e-10f) : __builtin_nanf("");
}

__global__ __launch_bounds__(256) void cross_entropy_stream_kernel(const float* logits,
                                                                   const int32_t* targets,
                                                                   float* grad, float* row_loss,
                                                                   int M, int N) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
    if (row >= M) return;
    const float* x = logits + (int64_t)row * N;
    float* g = grad + (int64_t)row * N;
    const int nv = N & ~15;
    float mx = -FLT_MAX;
    for (int j = lane; j < N; j += 64) mx = ref_max(mx, x[j]);
    mx = wave_max(mx);
    float s = 0.0f;
    for (int j = lane; j < N; j += 64) {
        const float e = row_exp(x[j] - mx, j, nv);
        g[j] = e;
        s += e;
    }
    s = wave_sum(s);
    const float inv = 1.0f / s;
    const int t = targets[row];
    const bool valid = t >= 0 && t < N;
    float pt = 0.0f;
    for (int j = lane; j < N; j += 64) {
        const float p = row_norm(g[j], inv, s, j, nv);
        if (j == t) pt = p;
        g[j] = ce_grad(p, j, valid ? t : -1, (float)M);
    }
    pt = wave_sum(pt);
    if (lane == 0) row_loss[row] = valid ? -logf(pt + 1e-10f) : __builtin_nanf("");
}

// loss = sum of row_loss in a fixed order / M (one workgroup)
__global__ __launch_bounds__(256) void cross_entropy_reduce_kernel(const float* __restrict__ row_loss,
                                                                   float* __restrict__ loss, int M) {
    __shared__ float part[4];
    float s = 0.0f;
    for (int i = threadIdx.x; i < M; i += 256) s += row_loss[i];
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) loss[0] = ((part[0] + part[1]) + (part[2] + part[3])) / (float)M;
}

// one wave per row: the smallest register-cache size that holds N
template <typename F>
hipError_t by_elems(int N, F&& f) {
    if (N <= 64) return f(std::integral_constant<int, 1>{});
    if (N <= 128) return f(std::integral_constant<int, 2>{});
    if (N <= 256) return f(std::integral_constant<int, 4>{});
    if (N <= 512) return f(std::integral_constant<int, 8>{});
    if (N <= 1024) return f(std::integral_constant<int, 16>{});
    if (N <= 2048) return f(std::integral_constant<int, 32>{});
    return f(std::integral_constant<int, 64>{});
}

}  // namespace

hipError_t launch_softmax(float* out, const float* in, int M, int N, hipStream_t s) {
    const unsigned blocks = (unsigned)((M + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK);
    if (N > MAX_CACHED) {
        hipLaunchKernelGGL(softmax_stream_kernel, dim3(blocks), dim3(256), 0, s, out, in, M, N);
        return hipGetLastError();
    }
    return by_elems(N, [&](auto e) {
        hipLaunchKernelGGL(softmax_kernel<decltype(e)::value>, dim3(blocks), dim3(256), 0, s, out,
                           in, M, N);
        return hipGetLastError();
    });
}

hipError_t launch_layernorm(float* out, const float* in, const float* gamma, const float* beta,
                            int M, int N, float eps, hipStream_t s) {
    const unsigned blocks = (unsigned)((M + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK);
    if (N > MAX_CACHED) {
        hipLaunchKernelGGL(layernorm_stream_kernel, dim3(blocks), dim3(256), 0, s, out, in, gamma,
                           beta, M, N, eps);
        return hipGetLastError();
    }
    return by_elems(N, [&](auto e) {
        hipLaunchKernelGGL(layernorm_kernel<decltype(e)::value>, dim3(blocks), dim3(256), 0, s,
                           out, in, gamma, beta, M, N, eps);
        return hipGetLastError();
    });
}

hipError_t launch_cross_entropy(const float* logits, const int32_t* targets, float* grad,
                                float* loss, float* row_loss, int M, int N, hipStream_t s) {
    const unsigned blocks = (unsigned)((M + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK);
    hipError_t e;
    if (N > MAX_CACHED) {
        hipLaunchKernelGGL(cross_entropy_stream_kernel, dim3(blocks), dim3(256), 0, s, logits,
                           targets, grad, row_loss, M, N);
        e = hipGetLastError();
    } else {
        e = by_elems(N, [&](auto el) {
            hipLaunchKernelGGL(cross_entropy_kernel<decltype(el)::value>, dim3(blocks), dim3(256), 0,
                               s, logits, targets, grad, row_loss, M, N);
            return hipGetLastError();
        });
    }
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(cross_entropy_reduce_kernel, dim3(1), dim3(256), 0, s, row_loss, loss, M);
    return hipGetLastError();
}

}  // namespace jh
