// pjrt_ops.hip - fp32 kernels for the StableHLO ops the ROCm PJRT executor
// runs itself (pjrt.cpp); custom_call targets go to the kernel registry.
//
// Semantics follow the reference's CPU interpreter (lib/PJRT.cpp):
//   binary  :606-630  out[i] = f(a[i] or 0 past a's end, b[i] or 0), n = max
//   unary   :632-648, with the per-op formulas of :225-266
//   transpose :726-801 (rank 2 always swaps the two dimensions, :768-777)
//   reduce  :805-857  sum over the reduced dimensions, each output summed in
//                     increasing input order (one thread per output keeps
//                     that order, so results equal the reference's loop)
// Shapes and strides are computed by the caller; rank <= 8.
#include "common.hpp"
#include "launch.hpp"

namespace jh {
namespace {

template <int OP>
__device__ __forceinline__ float binop(float a, float b) {
    if constexpr (OP == PJ_ADD) return a + b;
    else if constexpr (OP == PJ_SUB) return a - b;
    else if constexpr (OP == PJ_MUL) return a * b;
    else if constexpr (OP == PJ_DIV) return b != 0.0f ? a / b : 0.0f;
    else if constexpr (OP == PJ_MAX) return (a < b) ? b : a;  // std::max(a, b)
    else return (b < a) ? b : a;                              // std::min(a, b)
}

template <int OP>
__device__ __forceinline__ float unop(float a) {
    if constexpr (OP == PJ_NEG) return -a;
    else if constexpr (OP == PJ_RELU) return a > 0.0f ? a : 0.0f;
    else if constexpr (OP == PJ_SIGMOID) return 1.0f / (1.0f + expf(-a));
    else if constexpr (OP == PJ_TANH) return tanhf(a);
    else if constexpr (OP == PJ_EXP) return expf(a);
    else return a > 0.0f ? logf(a) : -__builtin_huge_valf();
}

template <int OP>
__global__ void binary_kernel(const float* __restrict__ a, int64_t na, const float* __restrict__ b,
                              int64_t nb, float* __restrict__ out, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const float x = i < na ? a[i] : 0.0f;
        const float y = i < nb ? b[i] : 0.0f;
        out[i] = binop<OP>(x, y);
    }
}

template <int OP>
__global__ void unary_kernel(const float* __restrict__ a, float* __restrict__ out, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = unop<OP>(a[i]);
}

// out flat index -> out multi-index (out_stride) -> input offset (in_step[d]
// = input stride of the input dimension that output dimension d walks)
__global__ void transpose_kernel(const float* __restrict__ in, float* __restrict__ out, int64_t n,
                                 PjIndexMap map) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t f = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; f < n; f += stride) {
        int64_t rem = f, off = 0;
        for (int d = 0; d < map.rank; ++d) {
            const int64_t q = rem / map.out_stride[d];
            rem -= q * map.out_stride[d];
            off += q * map.in_step[d];
        }
        out[f] = in[off];
    }
}

// One thread per output: `base` from the kept dimensions (out_stride /
// in_step as in transpose over the kept dims), then the reduced dimensions
// walked in row-major order (red_stride: strides of the reduced index space,
// red_step: their input strides), i.e. increasing input offset.
__global__ void reduce_kernel(const float* __restrict__ in, float* __restrict__ out, int64_t n_out,
                              int64_t n_red, PjIndexMap keep, PjIndexMap red) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < n_out; o += stride) {
        int64_t rem = o, base = 0;
        for (int d = 0; d < keep.rank; ++d) {
            const int64_t q = rem / keep.out_stride[d];
            rem -= q * keep.out_stride[d];
            base += q * keep.in_step[d];
        }
        float s = 0.0f;
        for (int64_t r = 0; r < n_red; ++r) {
            int64_t rr = r, off = base;
            for (int d = 0; d < red.rank; ++d) {
                const int64_t q = rr / red.out_stride[d];
                rr -= q * red.out_stride[d];
                off += q * red.in_step[d];
            }
            s = s + in[off];
        }
        out[o] = s;
    }
}

unsigned grid_for(int64_t n) {
    int64_t b = (n + 255) / 256;
    if (b > 8192) b = 8192;
    return (unsigned)(b < 1 ? 1 : b);
}

}  // namespace

hipError_t launch_pj_binary(int op, const float* a, int64_t na, const float* b, int64_t nb,
                            float* out, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    switch (op) {
#define JH_PJ_B(OPC)                                                                           \
    case OPC:                                                                                  \
        hipLaunchKernelGGL(binary_kernel<OPC>, dim3(grid_for(n)), dim3(256), 0, s, a, na, b, nb, out, n); \
        break;
        JH_PJ_B(PJ_ADD) JH_PJ_B(PJ_SUB) JH_PJ_B(PJ_MUL) JH_PJ_B(PJ_DIV) JH_PJ_B(PJ_MAX) JH_PJ_B(PJ_MIN)
#undef JH_PJ_B
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_pj_unary(int op, const float* a, float* out, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    switch (op) {
#define JH_PJ_U(OPC)                                                                      \
    case OPC:                                                                             \
        hipLaunchKernelGGL(unary_kernel<OPC>, dim3(grid_for(n)), dim3(256), 0, s, a, out, n); \
        break;
        JH_PJ_U(PJ_NEG) JH_PJ_U(PJ_RELU) JH_PJ_U(PJ_SIGMOID) JH_PJ_U(PJ_TANH) JH_PJ_U(PJ_EXP) JH_PJ_U(PJ_LOG)
#undef JH_PJ_U
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_pj_transpose(const float* in, float* out, int64_t n, const PjIndexMap& map,
                               hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(transpose_kernel, dim3(grid_for(n)), dim3(256), 0, s, in, out, n, map);
    return hipGetLastError();
}

hipError_t launch_pj_reduce(const float* in, float* out, int64_t n_out, int64_t n_red,
                            const PjIndexMap& keep, const PjIndexMap& red, hipStream_t s) {
    if (n_out <= 0) return hipSuccess;
    hipLaunchKernelGGL(reduce_kernel, dim3(grid_for(n_out)), dim3(256), 0, s, in, out, n_out, n_red,
                       keep, red);
    return hipGetLastError();
}

}  // namespace jh
