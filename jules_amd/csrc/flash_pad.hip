// flash_pad.hip - flash attention for head dims the kernels are not built
// for (1 <= D <= 128, D not 64 or 128), and the per-stream workspace shared
// by the entry points that take none.
//
// The reference's flashAttention (include/jules/Kernel/FlashAttention.h:
// 130-309) accepts any head_dim.  The MFMA kernels here are built for 64 and
// 128; other sizes are zero-padded to the next of the two.  Zero columns
// change neither the scores Q K^T, nor the log-sum-exp, nor the real columns
// of O (padded V columns only produce padded O columns), nor, in the
// backward, the real columns of dQ, dK and dV (rowsum(dO * O) is unchanged;
// the padded gradient columns come out as zeros).  The caller's scale is
// used as given (its default is 1/sqrt(D) of the real D).
#include <map>
#include <mutex>

#include "common.hpp"
#include "launch.hpp"

namespace jh {

// One workspace per (device, stream), kept for the process: calls on one
// stream run in order and may share it, calls on other streams get their
// own.  A larger need replaces it once the stream is done with the old one.
hipError_t stream_workspace(size_t need, hipStream_t s, void** ws) {
    static std::mutex mu;
    static std::map<std::pair<int, hipStream_t>, std::pair<void*, size_t>> cache;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(mu);
    auto& slot = cache[{dev, s}];
    if (slot.second < need) {
        if (slot.first) {
            if ((e = hipStreamSynchronize(s)) != hipSuccess) return e;
            (void)hipFree(slot.first);
        }
        slot = {nullptr, 0};
        void* p = nullptr;
        if ((e = hipMalloc(&p, need)) != hipSuccess) return e;
        slot = {p, need};
    }
    *ws = slot.first;
    return hipSuccess;
}

namespace {

// dst[r][c] = c < D ? src[r][c] : 0 over [rows][Dp]
template <typename T>
__global__ void pad_rows_kernel(T* __restrict__ dst, const T* __restrict__ src, int64_t rows, int D,
                                int Dp) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * Dp) return;
    const int64_t r = i / Dp;
    const int c = (int)(i % Dp);
    dst[i] = c < D ? src[r * D + c] : T(0);
}
// dst[r][c] = src[r][c] for c < D, over [rows][D]
template <typename T>
__global__ void unpad_rows_kernel(T* __restrict__ dst, const T* __restrict__ src, int64_t rows, int D,
                                  int Dp) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * D) return;
    const int64_t r = i / D;
    const int c = (int)(i % D);
    dst[i] = src[r * Dp + c];
}

inline size_t a256(size_t n) { return (n + 255) & ~size_t(255); }

// element size: fp32 moved as uint32_t, bf16 as uint16_t
template <typename T>
hipError_t pad(void* dst, const void* src, int64_t rows, int D, int Dp, hipStream_t s) {
    const int64_t n = rows * Dp;
    hipLaunchKernelGGL(pad_rows_kernel<T>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                       static_cast<T*>(dst), static_cast<const T*>(src), rows, D, Dp);
    return hipGetLastError();
}
template <typename T>
hipError_t unpad(void* dst, const void* src, int64_t rows, int D, int Dp, hipStream_t s) {
    const int64_t n = rows * D;
    hipLaunchKernelGGL(unpad_rows_kernel<T>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                       static_cast<T*>(dst), static_cast<const T*>(src), rows, D, Dp);
    return hipGetLastError();
}

}  // namespace

int flash_padded_dim(int D) { return D <= 64 ? 64 : 128; }

hipError_t launch_flash_fwd_padded(int dtype, int causal, float scale, const void* Q, const void* K,
                                   const void* V, void* O, float* lse, int B, int H, int S, int D,
                                   hipStream_t s) {
    const int Dp = flash_padded_dim(D);
    const int64_t rows = (int64_t)B * H * S;
    const size_t es = dtype == JH_BF16 ? 2 : 4;
    const size_t one = a256((size_t)rows * Dp * es);
    void* ws = nullptr;
    hipError_t e = stream_workspace(4 * one, s, &ws);
    if (e != hipSuccess) return e;
    char* w = static_cast<char*>(ws);
    void *Qp = w, *Kp = w + one, *Vp = w + 2 * one, *Op = w + 3 * one;
    auto padf = dtype == JH_BF16 ? pad<uint16_t> : pad<uint32_t>;
    if ((e = padf(Qp, Q, rows, D, Dp, s)) || (e = padf(Kp, K, rows, D, Dp, s)) ||
        (e = padf(Vp, V, rows, D, Dp, s)))
        return e;
    if ((e = launch_flash_fwd(dtype, causal, scale, Qp, Kp, Vp, Op, lse, B, H, S, Dp, s))) return e;
    return dtype == JH_BF16 ? unpad<uint16_t>(O, Op, rows, D, Dp, s) : unpad<uint32_t>(O, Op, rows, D, Dp, s);
}

hipError_t launch_flash_bwd_padded(int dtype, int causal, float scale, const void* Q, const void* K,
                                   const void* V, const void* O, const void* dO, const float* lse,
                                   void* dQ, void* dK, void* dV, int B, int H, int S, int D,
                                   void* bwd_ws, hipStream_t s) {
    const int Dp = flash_padded_dim(D);
    const int64_t rows = (int64_t)B * H * S;
    const size_t es = dtype == JH_BF16 ? 2 : 4;
    const size_t one = a256((size_t)rows * Dp * es);
    void* ws = nullptr;
    hipError_t e = stream_workspace(8 * one, s, &ws);
    if (e != hipSuccess) return e;
    char* w = static_cast<char*>(ws);
    void* p[8];
    for (int i = 0; i < 8; ++i) p[i] = w + i * one;  // Q K V O dO dQ dK dV
    auto padf = dtype == JH_BF16 ? pad<uint16_t> : pad<uint32_t>;
    auto unpadf = dtype == JH_BF16 ? unpad<uint16_t> : unpad<uint32_t>;
    const void* src[5] = {Q, K, V, O, dO};
    for (int i = 0; i < 5; ++i)
        if ((e = padf(p[i], src[i], rows, D, Dp, s))) return e;
    if ((e = launch_flash_bwd(dtype, causal, scale, p[0], p[1], p[2], p[3], p[4], lse, p[5], p[6], p[7],
                              B, H, S, Dp, bwd_ws, s)))
        return e;
    if ((e = unpadf(dQ, p[5], rows, D, Dp, s)) || (e = unpadf(dK, p[6], rows, D, Dp, s)) ||
        (e = unpadf(dV, p[7], rows, D, Dp, s)))
        return e;
    return hipSuccess;
}

}  // namespace jh
