// mlp.hip - 2-layer MLP forward + softmax cross entropy + backward on gfx950.
//
// Reference: interleavedMLPForwardBackward (include/jules/Kernel/
// InterleavedAutodiff.h:55-441):
//   h = X W1 + b1, a = relu(h)                               :144-166
//   o = a W2 + b2 -> output                                  :168-176
//   p = softmax(o) per row, loss = sum_i -log(p[t_i] + 1e-10) / M,
//   dO = (p - onehot(t)) / M                                 :178-197
//   dW2 = a^T dO, db2 = colsum(dO)                           :207-221
//   dA = dO W2^T, dH = dA * (h > 0)                          :223-247
//   dW1 = X^T dH, db1 = colsum(dH), dX = dH W1^T             :249-267
// The reference runs this tile by tile on the CPU so that h and a stay in
// cache between the forward and the backward of a tile.  Here the five
// products are whole-matrix fp32 MFMA GEMMs and the intermediates (a, dO,
// dH) go to a caller workspace in HBM: at the shapes where the GPU pays off
// they are a few per cent of the GEMM traffic, and whole-matrix GEMMs keep
// the MFMA pipes full where tile-sized ones would not.
//
// relu'(h) is read from a: a > 0 exactly when h > 0, so h is not stored.
// The loss and dO come from the fused cross-entropy row kernel (rowops.hip),
// which computes the same formula.  db1/db2 are column sums in a fixed order
// (row chunks, then the chunks in order), so every result is deterministic.
//
// GEMM: C[M,N] = op(A)[M,K] op(B)[K,N] with v_mfma_f32_32x32x2_f32.  A 128x128
// output tile per 256-thread workgroup (4 waves, 64x64 each = 2x2 MFMA
// blocks), K in slices of 16 staged through LDS ([k][m] and [k][n], padded
// rows), the next slice's global loads in registers while the current one is
// multiplied, one barrier per slice.  op(A) = A^T and op(B) = B^T only change
// which dimension the global loads run along; the LDS layout is the same.
// Out-of-range elements are loaded as 0 (any summation order is allowed
// here: the reference's products are BLAS calls).
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"

namespace jh {
namespace {

typedef float f32x16_mfma_t __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 16;
constexpr int GT = 256;              // threads per GEMM workgroup
constexpr int LDA_S = BM + 1;        // LDS row pitch (floats)
constexpr int LDB_S = BN + 1;
constexpr int PA = BM * BK / GT;     // A elements per thread per slice (8)
constexpr int PB = BK * BN / GT;

// BLAS sgemm epilogue: alpha * acc + beta * C, with C not read when
// beta = 0 (so NaNs in an uninitialised C never propagate), and acc itself
// when alpha = 1 and beta = 0
__device__ __forceinline__ float alpha_beta(float acc, float alpha, float beta, const float* c) {
    const float v = alpha * acc;
    return beta == 0.0f ? v : v + beta * *c;
}

template <bool TA, bool TB, int EPI>
__global__ __launch_bounds__(GT, 2) void gemm_f32_mfma_kernel(
    const float* __restrict__ A, int lda, const float* __restrict__ B, int ldb,
    float* __restrict__ C, int ldc, int M, int N, int K, const float* __restrict__ bias,
    const float* __restrict__ mask, int ldm, int kc, float* __restrict__ part, float alpha,
    float beta) {
    __shared__ float As[2][BK * LDA_S];
    __shared__ float Bs[2][BK * LDB_S];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;  // 64x64 quadrant of the tile
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    // this workgroup's K range (split-K: blockIdx.z of gridDim.z)
    const int kb = blockIdx.z * kc, ke = min(K, kb + kc);

    float ra[PA], rb[PB];
    // element e of a slice: along the dimension contiguous in memory
    auto gload = [&](int k0) {
#pragma unroll
        for (int p = 0; p < PA; ++p) {
            const int e = tid + p * GT;
            const int m = TA ? (e & (BM - 1)) : (e >> 4);
            const int k = TA ? (e >> 7) : (e & (BK - 1));
            const int gm = m0 + m, gk = k0 + k;
            const bool ok = gm < M && gk < ke;
            const int64_t off = TA ? (int64_t)gk * lda + gm : (int64_t)gm * lda + gk;
            const float v = A[ok ? off : 0];  // branch-free: element 0, then dropped
            ra[p] = ok ? v : 0.0f;
        }
#pragma unroll
        for (int p = 0; p < PB; ++p) {
            const int e = tid + p * GT;
            const int n = TB ? (e >> 4) : (e & (BN - 1));
            const int k = TB ? (e & (BK - 1)) : (e >> 7);
            const int gn = n0 + n, gk = k0 + k;
            const bool ok = gn < N && gk < ke;
            const int64_t off = TB ? (int64_t)gn * ldb + gk : (int64_t)gk * ldb + gn;
            const float v = B[ok ? off : 0];
            rb[p] = ok ? v : 0.0f;
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int p = 0; p < PA; ++p) {
            const int e = tid + p * GT;
            const int m = TA ? (e & (BM - 1)) : (e >> 4);
            const int k = TA ? (e >> 7) : (e & (BK - 1));
            As[buf][k * LDA_S + m] = ra[p];
        }
#pragma unroll
        for (int p = 0; p < PB; ++p) {
            const int e = tid + p * GT;
            const int n = TB ? (e >> 4) : (e & (BN - 1));
            const int k = TB ? (e & (BK - 1)) : (e >> 7);
            Bs[buf][k * LDB_S + n] = rb[p];
        }
    };

    f32x16_mfma_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int nk = (ke - kb + BK - 1) / BK;
    gload(kb);
    sstore(0);
    __syncthreads();
    const int lr = lane & 31, lk = lane >> 5;  // MFMA operand: row/col lr, k lk
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload(kb + (kt + 1) * BK);
        const float* as = As[buf];
        const float* bs = Bs[buf];
#pragma unroll
        for (int kk = 0; kk < BK; kk += 2) {
            float a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) a[i] = as[(kk + lk) * LDA_S + wm * 64 + i * 32 + lr];
#pragma unroll
            for (int j = 0; j < 2; ++j) b[j] = bs[(kk + lk) * LDB_S + wn * 64 + j * 32 + lr];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) sstore(buf ^ 1);
        __syncthreads();
    }

    // 32x32 accumulator layout: register r of lane l holds row
    // 8*(r/4) + 4*(l/32) + r%4, column l%32
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + wn * 64 + j * 32 + lr;
            if (n >= N) continue;
            if (part) {  // split-K: raw partial sums, epilogue in the reduction
                float* pz = part + (int64_t)blockIdx.z * M * N;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
                    if (m < M) pz[(int64_t)m * N + n] = acc[i][j][r];
                }
                continue;
            }
            float bn = 0.0f;
            if constexpr (EPI == 1 || EPI == 2) bn = bias[n];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
                if (m >= M) continue;
                float v = acc[i][j][r];
                if constexpr (EPI == 1) {
                    v = v + bn;
                } else if constexpr (EPI == 2) {
                    v = v + bn;
                    v = v > 0.0f ? v : 0.0f;
                } else if constexpr (EPI == 3) {
                    v = mask[(int64_t)m * ldm + n] > 0.0f ? v : 0.0f;
                } else if constexpr (EPI == 4) {
                    v = alpha_beta(v, alpha, beta, C + (int64_t)m * ldc + n);
                }
                C[(int64_t)m * ldc + n] = v;
            }
        }
}

// Split-K reduction: C = epilogue(sum over z of part[z], in z order).
template <int EPI>
__global__ void splitk_reduce_kernel(const float* __restrict__ part, int S, int M, int N,
                                     float* __restrict__ C, int ldc, const float* __restrict__ bias,
                                     const float* __restrict__ mask, int ldm, float alpha,
                                     float beta) {
    const int64_t total = (int64_t)M * N, stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
        const int m = (int)(e / N), n = (int)(e - (int64_t)m * N);
        float v = part[e];
        for (int z = 1; z < S; ++z) v += part[(int64_t)z * total + e];
        if constexpr (EPI == 1) {
            v = v + bias[n];
        } else if constexpr (EPI == 2) {
            v = v + bias[n];
            v = v > 0.0f ? v : 0.0f;
        } else if constexpr (EPI == 3) {
            v = mask[(int64_t)m * ldm + n] > 0.0f ? v : 0.0f;
        } else if constexpr (EPI == 4) {
            v = alpha_beta(v, alpha, beta, C + (int64_t)m * ldc + n);
        }
        C[(int64_t)m * ldc + n] = v;
    }
}

// C = beta * C (alpha * op(A) op(B) vanishes: K = 0 or alpha = 0); beta = 0
// writes zeros without reading C, as BLAS does
__global__ void scale_c_kernel(float* __restrict__ C, int ldc, int M, int N, float beta) {
    const int64_t total = (int64_t)M * N, stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
        const int m = (int)(e / N), n = (int)(e - (int64_t)m * N);
        float* c = C + (int64_t)m * ldc + n;
        *c = beta == 0.0f ? 0.0f : beta * *c;
    }
}

// Column sums in a fixed order: partial[s][n] sums rows [s*R, (s+1)*R) in
// row order, then out[n] sums the partials in s order.
__global__ void colsum_partial_kernel(const float* __restrict__ X, int M, int N, int ld, int R,
                                      float* __restrict__ part) {
    const int n = blockIdx.x * blockDim.x + threadIdx.x;
    const int s = blockIdx.y;
    if (n >= N) return;
    const int r0 = s * R, r1 = min(M, r0 + R);
    float acc = 0.0f;
    int m = r0;
    // 8 loads in flight, added in row order
    for (; m + 8 <= r1; m += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = X[(int64_t)(m + u) * ld + n];
#pragma unroll
        for (int u = 0; u < 8; ++u) acc += v[u];
    }
    for (; m < r1; ++m) acc += X[(int64_t)m * ld + n];
    part[(int64_t)s * N + n] = acc;
}

__global__ void colsum_final_kernel(const float* __restrict__ part, int S, int N,
                                    float* __restrict__ out) {
    const int n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= N) return;
    float acc = part[n];
    for (int s = 1; s < S; ++s) acc += part[(int64_t)s * N + n];
    out[n] = acc;
}

__global__ void fill_kernel(float* __restrict__ p, int64_t n, float v) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = v;
}

enum { EPI_NONE = 0, EPI_BIAS = 1, EPI_BIAS_RELU = 2, EPI_MASK = 3, EPI_ALPHA_BETA = 4 };

// Split-K plan: a GEMM with fewer than 128 output tiles gets its K range
// split (at least 4 slices per split) so that about 256 workgroups run; the
// partial sums go to the workspace and a reduction applies the epilogue.
struct KPlan {
    int S;   // splits
    int kc;  // K elements per split, a multiple of BK
};

KPlan kplan(int M, int N, int K) {
    // 64-bit: M, N, K may be anywhere up to INT_MAX
    const int64_t tiles = ((int64_t)M + BM - 1) / BM * (((int64_t)N + BN - 1) / BN);
    const int max_s = K / (4 * BK);
    if (tiles <= 0 || tiles >= 128 || max_s < 2) return {1, K};
    int S = (int)((256 + tiles - 1) / tiles);
    if (S > max_s) S = max_s;
    const int64_t kc = (((int64_t)K + S - 1) / S + BK - 1) / BK * BK;
    return {(int)(((int64_t)K + kc - 1) / kc), (int)kc};
}

size_t kplan_floats(int M, int N, int K) {
    const KPlan p = kplan(M, N, K);
    return p.S > 1 ? (size_t)p.S * M * N : 0;
}

template <bool TA, bool TB, int EPI>
hipError_t gemm(const float* A, int lda, const float* B, int ldb, float* C, int ldc, int M, int N,
                int K, const float* bias, const float* mask, int ldm, float* part, hipStream_t s,
                float alpha = 1.0f, float beta = 0.0f) {
    const KPlan p = kplan(M, N, K);
    const dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM, p.S);
    hipLaunchKernelGGL((gemm_f32_mfma_kernel<TA, TB, EPI>), grid, dim3(GT), 0, s, A, lda, B, ldb, C,
                       ldc, M, N, K, bias, mask, ldm, p.kc, p.S > 1 ? part : nullptr, alpha, beta);
    if (p.S > 1) {
        int64_t b = ((int64_t)M * N + 255) / 256;
        if (b > 2048) b = 2048;
        hipLaunchKernelGGL(splitk_reduce_kernel<EPI>, dim3((unsigned)b), dim3(256), 0, s, part, p.S,
                           M, N, C, ldc, bias, mask, ldm, alpha, beta);
    }
    return hipGetLastError();
}

constexpr int COLSUM_ROWS = 256;  // rows per partial column sum
constexpr int COLSUM_MAX_CHUNKS = 64;

int colsum_chunks(int M, int* rows) {
    int S = (M + COLSUM_ROWS - 1) / COLSUM_ROWS;
    if (S > COLSUM_MAX_CHUNKS) S = COLSUM_MAX_CHUNKS;
    if (S < 1) S = 1;
    *rows = (M + S - 1) / S;
    return S;
}

hipError_t colsum(const float* X, int M, int N, float* part, float* out, hipStream_t s) {
    int R;
    const int S = colsum_chunks(M, &R);
    hipLaunchKernelGGL(colsum_partial_kernel, dim3((N + 255) / 256, S), dim3(256), 0, s, X, M, N, N,
                       R, part);
    hipLaunchKernelGGL(colsum_final_kernel, dim3((N + 255) / 256), dim3(256), 0, s, part, S, N, out);
    return hipGetLastError();
}

hipError_t fill(float* p, int64_t n, float v, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    int64_t b = (n + 255) / 256;
    if (b > 4096) b = 4096;
    hipLaunchKernelGGL(fill_kernel, dim3((unsigned)b), dim3(256), 0, s, p, n, v);
    return hipGetLastError();
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

}  // namespace

// workspace: a [M,N1], dH [M,N1], dO [M,N2], per-row losses [M], column-sum
// partials [chunks, max(N1,N2)], each 256-byte aligned
size_t mlp_workspace_size(int M, int K1, int N1, int N2) {
    (void)K1;
    int R;
    const int S = colsum_chunks(M, &R);
    const size_t mn1 = (size_t)M * N1 * sizeof(float), mn2 = (size_t)M * N2 * sizeof(float);
    // split-K partials of the five products (only skinny ones split)
    size_t kp = kplan_floats(M, N1, K1);
    kp = std::max(kp, kplan_floats(M, N2, N1));
    kp = std::max(kp, kplan_floats(N1, N2, M));
    kp = std::max(kp, kplan_floats(M, N1, N2));
    kp = std::max(kp, kplan_floats(K1, N1, M));
    kp = std::max(kp, kplan_floats(M, K1, N1));
    return 2 * align256(mn1) + align256(mn2) + align256((size_t)M * sizeof(float)) +
           align256((size_t)S * (N1 > N2 ? N1 : N2) * sizeof(float)) + align256(kp * sizeof(float));
}

// fusedMLPForward (reference FusedKernels.h:659-760): output = relu(X W1 +
// b1) W2 + b2, the forward half of the step below.  workspace: the hidden
// activations [M,N1], then split-K partials
size_t mlp_forward_workspace_size(int M, int K1, int N1, int N2) {
    (void)K1;
    const size_t kp = std::max(kplan_floats(M, N1, K1), kplan_floats(M, N2, N1));
    return align256((size_t)M * N1 * sizeof(float)) + align256(kp * sizeof(float));
}

hipError_t launch_mlp_forward(const float* X, const float* W1, const float* b1, const float* W2,
                              const float* b2, float* output, int M, int K1, int N1, int N2,
                              void* ws, hipStream_t s) {
    if (M == 0) return hipSuccess;
    float* act = static_cast<float*>(ws);
    float* kpart = reinterpret_cast<float*>(static_cast<char*>(ws) +
                                            align256((size_t)M * N1 * sizeof(float)));
    hipError_t e;
    if ((e = gemm<false, false, EPI_BIAS_RELU>(X, K1, W1, N1, act, N1, M, N1, K1, b1, nullptr, 0, kpart, s)))
        return e;
    return gemm<false, false, EPI_BIAS>(act, N1, W2, N2, output, N2, M, N2, N1, b2, nullptr, 0, kpart, s);
}

hipError_t launch_mlp_forward_backward(const float* X, const float* W1, const float* b1,
                                       const float* W2, const float* b2, const int32_t* targets,
                                       float* output, float* dW1, float* db1, float* dW2, float* db2,
                                       float* dX, float* loss, int M, int K1, int N1, int N2,
                                       void* ws, hipStream_t s) {
    if (M == 0) {
        // no rows: zero gradients, loss 0/0 (the reference divides its
        // empty sum by M)
        hipError_t e = fill(dW1, (int64_t)K1 * N1, 0.0f, s);
        if (e == hipSuccess) e = fill(db1, N1, 0.0f, s);
        if (e == hipSuccess) e = fill(dW2, (int64_t)N1 * N2, 0.0f, s);
        if (e == hipSuccess) e = fill(db2, N2, 0.0f, s);
        if (e == hipSuccess) e = fill(loss, 1, __builtin_nanf(""), s);
        return e;
    }
    char* w = static_cast<char*>(ws);
    const size_t mn1 = align256((size_t)M * N1 * sizeof(float));
    const size_t mn2 = align256((size_t)M * N2 * sizeof(float));
    float* act = reinterpret_cast<float*>(w);
    float* dH = reinterpret_cast<float*>(w + mn1);
    float* dO = reinterpret_cast<float*>(w + 2 * mn1);
    float* row_loss = reinterpret_cast<float*>(w + 2 * mn1 + mn2);
    float* part = reinterpret_cast<float*>(w + 2 * mn1 + mn2 + align256((size_t)M * sizeof(float)));
    int R;
    const int S = colsum_chunks(M, &R);
    float* kpart = reinterpret_cast<float*>(reinterpret_cast<char*>(part) +
                                            align256((size_t)S * (N1 > N2 ? N1 : N2) * sizeof(float)));

    hipError_t e;
    // forward
    if ((e = gemm<false, false, EPI_BIAS_RELU>(X, K1, W1, N1, act, N1, M, N1, K1, b1, nullptr, 0, kpart, s)))
        return e;
    if ((e = gemm<false, false, EPI_BIAS>(act, N1, W2, N2, output, N2, M, N2, N1, b2, nullptr, 0, kpart, s)))
        return e;
    // loss and dO
    if ((e = launch_cross_entropy(output, targets, dO, loss, row_loss, M, N2, s))) return e;
    // layer 2 gradients
    if ((e = gemm<true, false, EPI_NONE>(act, N1, dO, N2, dW2, N2, N1, N2, M, nullptr, nullptr, 0, kpart, s)))
        return e;
    if ((e = colsum(dO, M, N2, part, db2, s))) return e;
    // dH = (dO W2^T) * (a > 0)
    if ((e = gemm<false, true, EPI_MASK>(dO, N2, W2, N2, dH, N1, M, N1, N2, nullptr, act, N1, kpart, s)))
        return e;
    // layer 1 gradients
    if ((e = gemm<true, false, EPI_NONE>(X, K1, dH, N1, dW1, N1, K1, N1, M, nullptr, nullptr, 0, kpart, s)))
        return e;
    if ((e = colsum(dH, M, N1, part, db1, s))) return e;
    if (dX && (e = gemm<false, true, EPI_NONE>(dH, N1, W1, N1, dX, K1, M, K1, N1, nullptr, nullptr, 0, kpart, s)))
        return e;
    return hipSuccess;
}

// blasMatmul / cblas_sgemm (reference FusedKernels.h:633-644): the MFMA GEMM
// above with the sgemm epilogue.  Skinny products split K into a per-stream
// library buffer (the entry point has no workspace argument).
hipError_t launch_sgemm(bool transA, bool transB, int M, int N, int K, float alpha, const float* A,
                        int lda, const float* B, int ldb, float beta, float* C, int ldc,
                        hipStream_t s) {
    if (M == 0 || N == 0) return hipSuccess;
    if (K == 0 || alpha == 0.0f) {
        int64_t b = ((int64_t)M * N + 255) / 256;
        if (b > 4096) b = 4096;
        hipLaunchKernelGGL(scale_c_kernel, dim3((unsigned)b), dim3(256), 0, s, C, ldc, M, N, beta);
        return hipGetLastError();
    }
    float* part = nullptr;
    const size_t pf = kplan_floats(M, N, K);
    if (pf) {
        void* ws = nullptr;
        const hipError_t e = stream_workspace(pf * sizeof(float), s, &ws);
        if (e != hipSuccess) return e;
        part = static_cast<float*>(ws);
    }
    auto run = [&](auto ta, auto tb) {
        return gemm<decltype(ta)::value, decltype(tb)::value, EPI_ALPHA_BETA>(
            A, lda, B, ldb, C, ldc, M, N, K, nullptr, nullptr, 0, part, s, alpha, beta);
    };
    using F = std::false_type;
    using T = std::true_type;
    if (transA) return transB ? run(T{}, T{}) : run(T{}, F{});
    return transB ? run(F{}, T{}) : run(F{}, F{});
}

}  // namespace jh
