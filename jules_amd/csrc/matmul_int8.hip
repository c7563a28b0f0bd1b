// matmul_int8.hip - int8 x int8 GEMM with the semantics of matmulInt8's
// scalar path (reference include/jules/Kernel/FusedKernels.h:1046-1066):
//   C[i,j] = float(sum_k A[i,k] * B[k,j]) * (scale_A * scale_B)  [+ bias[j]]
// and its W8A8 form with per-token activation scales sA[i] and per-channel
// weight scales sB[j] (the scale product rounded to fp32 per element):
//   C[i,j] = float(sum_k A[i,k] * B[k,j]) * (sA[i] * sB[j])    [+ bias[j]]
// int32 accumulation is exact (|sum| <= 127*128*K < 2^31 for K <= 131072), so
// any summation order gives the reference's integer; the epilogue is one fp32
// multiply by the fp32-rounded scale product, then one add of bias.
//
// Not on the decode hot path (that is W8A16); a plain LDS-tiled SIMT kernel,
// 64x64 outputs per 256-thread block, 4x4 per thread, v_dot4-free so that the
// packed byte layout of B ([K,N], row-major) needs no transposition.
#include "common.hpp"
#include "launch.hpp"

namespace jh {
namespace {

constexpr int BM = 64, BN = 64, BK = 32;

__global__ __launch_bounds__(256) void matmul_int8_kernel(
    const int8_t* __restrict__ A, const int8_t* __restrict__ B, float* __restrict__ C,
    int M, int N, int K, float scale_a, float scale_b, const float* __restrict__ row_scale,
    const float* __restrict__ col_scale, const float* __restrict__ bias) {
    __shared__ int As[BK][BM + 1];
    __shared__ int Bs[BK][BN + 1];
    const int tid = threadIdx.x;
    const int tx = tid & 15, ty = tid >> 4;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    int acc[4][4] = {};
    for (int k0 = 0; k0 < K; k0 += BK) {
        for (int e = tid; e < BM * BK; e += 256) {
            const int m = e / BK, k = e % BK;
            As[k][m] = (m0 + m < M && k0 + k < K) ? (int)A[(int64_t)(m0 + m) * K + k0 + k] : 0;
        }
        for (int e = tid; e < BK * BN; e += 256) {
            const int k = e / BN, n = e % BN;
            Bs[k][n] = (k0 + k < K && n0 + n < N) ? (int)B[(int64_t)(k0 + k) * N + n0 + n] : 0;
        }
        __syncthreads();
#pragma unroll 8
        for (int k = 0; k < BK; ++k) {
            int a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = As[k][ty + 16 * i];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = Bs[k][tx + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] += a[i] * b[j];
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + ty + 16 * i;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + tx + 16 * j;
            if (n >= N) continue;
            // the scale product is rounded to fp32 first, then one multiply
            const float sc = (row_scale ? row_scale[m] : scale_a) * (col_scale ? col_scale[n] : scale_b);
            float c = (float)acc[i][j] * sc;
            if (bias) c = c + bias[n];
            C[(int64_t)m * N + n] = c;
        }
    }
}

}  // namespace

hipError_t launch_matmul_int8(const int8_t* A, const int8_t* B, float* C, int M, int N, int K,
                              float scale_a, float scale_b, const float* bias, hipStream_t s) {
    // per-tensor scales: scale_a * scale_b rounded to fp32 first, FusedKernels.h:1061
    dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
    hipLaunchKernelGGL(matmul_int8_kernel, grid, dim3(256), 0, s, A, B, C, M, N, K, scale_a, scale_b,
                       nullptr, nullptr, bias);
    return hipGetLastError();
}

hipError_t launch_matmul_w8a8(const int8_t* A, const int8_t* B, float* C, int M, int N, int K,
                              const float* scale_a, const float* scale_b, const float* bias,
                              hipStream_t s) {
    dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
    hipLaunchKernelGGL(matmul_int8_kernel, grid, dim3(256), 0, s, A, B, C, M, N, K, 1.0f, 1.0f,
                       scale_a, scale_b, bias);
    return hipGetLastError();
}

}  // namespace jh
