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
// HBM once and written once, four rows per workgroup.  Longer rows get a
// 256-thread workgroup each and three passes over the row (max, sum, write:
// the reference's own pass structure, with the exponentials recomputed in the
// last pass instead of stored); the loads of a pass are unrolled four deep
// and the re-reads of a row mostly hit the MALL.  Reductions are a fixed
// butterfly within a wave and a fixed order across waves, so results are
// deterministic.
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

// ---- rows longer than MAX_CACHED: one 256-thread workgroup per row ----
constexpr int LT = 256;  // threads per long row

// fixed-order reductions over the workgroup (4 waves)
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    __syncthreads();  // red is reused by consecutive reductions
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// f(j) for j = tid, tid + 256, ... < N, four loads in flight
template <typename F>
__device__ __forceinline__ void row_loop(int N, F&& f) {
    int j = threadIdx.x;
    for (; j + 3 * LT < N; j += 4 * LT) {
        f(j);
        f(j + LT);
        f(j + 2 * LT);
        f(j + 3 * LT);
    }
    for (; j < N; j += LT) f(j);
}

// max and sum of exp(x - max) of a long row (reference passes 1a and 1b)
__device__ __forceinline__ void long_row_stats(const float* x, int N, float* red, float* mx_out,
                                               float* s_out) {
    const int nv = N & ~15;
    float mx = -FLT_MAX;
    row_loop(N, [&](int j) { mx = ref_max(mx, x[j]); });
    mx = block_max(mx, red);
    float s = 0.0f;
    row_loop(N, [&](int j) { s += row_exp(x[j] - mx, j, nv); });
    *mx_out = mx;
    *s_out = block_sum(s, red);
}

__global__ __launch_bounds__(LT) void softmax_long_kernel(float* out, const float* in, int N) {
    __shared__ float red[4];
    const float* x = in + (int64_t)blockIdx.x * N;
    float* y = out + (int64_t)blockIdx.x * N;
    const int nv = N & ~15;
    float mx, s;
    long_row_stats(x, N, red, &mx, &s);
    const float inv = 1.0f / s;
    row_loop(N, [&](int j) { y[j] = row_norm(row_exp(x[j] - mx, j, nv), inv, s, j, nv); });
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

__global__ __launch_bounds__(LT) void layernorm_long_kernel(float* out, const float* in,
                                                           const float* __restrict__ gamma,
                                                           const float* __restrict__ beta, int N,
                                                           float eps) {
    __shared__ float red[4];
    const float* x = in + (int64_t)blockIdx.x * N;
    float* y = out + (int64_t)blockIdx.x * N;
    float s = 0.0f;
    row_loop(N, [&](int j) { s += x[j]; });
    const float mean = block_sum(s, red) / (float)N;
    float q = 0.0f;
    row_loop(N, [&](int j) {
        const float d = x[j] - mean;
        q = __builtin_fmaf(d, d, q);
    });
    const float var = block_sum(q, red) / (float)N;
    const float inv_std = 1.0f / sqrtf(var + eps);
    row_loop(N, [&](int j) { y[j] = __builtin_fmaf((x[j] - mean) * inv_std, gamma[j], beta[j]); });
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

__global__ __launch_bounds__(LT) void cross_entropy_long_kernel(const float* logits,
                                                               const int32_t* targets, float* grad,
                                                               float* row_loss, int M, int N) {
    __shared__ float red[4];
    const int row = blockIdx.x;
    const float* x = logits + (int64_t)row * N;
    float* g = grad + (int64_t)row * N;
    const int nv = N & ~15;
    float mx, s;
    long_row_stats(x, N, red, &mx, &s);
    const float inv = 1.0f / s;
    const int t = targets[row];
    const bool valid = t >= 0 && t < N;
    const float fm = (float)M;
    float pt = 0.0f;
    row_loop(N, [&](int j) {
        const float p = row_norm(row_exp(x[j] - mx, j, nv), inv, s, j, nv);
        if (j == t) pt = p;
        g[j] = ce_grad(p, j, valid ? t : -1, fm);
    });
    pt = block_sum(pt, red);  // one thread holds it, the others 0
    if (threadIdx.x == 0) row_loss[row] = valid ? -logf(pt + 1e-10f) : __builtin_nanf("");
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
        hipLaunchKernelGGL(softmax_long_kernel, dim3(M), dim3(LT), 0, s, out, in, N);
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
        hipLaunchKernelGGL(layernorm_long_kernel, dim3(M), dim3(LT), 0, s, out, in, gamma, beta, N,
                           eps);
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
        if (M > 0)
            hipLaunchKernelGGL(cross_entropy_long_kernel, dim3(M), dim3(LT), 0, s, logits, targets,
                               grad, row_loss, M, N);
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
