// calib.hip - roofline calibrations (no counterpart in the reference): the
// MFMA rate the part sustains, and the HBM read rate a plain streaming read
// attains.
//
// A stream of independent v_mfma_f32_32x32x16_bf16 on random bf16 operands
// held in registers.  It measures the MFMA rate the part sustains under load:
// the engine clock drops under the power limit as MFMA activity rises
// (measured: ~93% MFMA busy at ~1.7 GHz instead of 2.4 GHz), so this is the
// clock-adjusted peak that the hot-path kernels' MFMA rates are compared with,
// next to the published 2516.6 TFLOP/s.  Operands come from a hash of
// (wave, lane, index), uniform in [-1, 1) at bf16 precision, so the
// multipliers toggle like they do on real data (all-zero operands run faster).
#include "common.hpp"
#include "launch.hpp"

namespace jh {
namespace {

__device__ __forceinline__ uint32_t mix32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352dU;
    x ^= x >> 15;
    x *= 0x846ca68bU;
    x ^= x >> 16;
    return x;
}

// 4 waves, 16 MFMAs per iteration into 8 accumulators (two uses each, never
// back to back)
__global__ __launch_bounds__(256, 1) void mfma_ceiling_kernel(float* __restrict__ out, int iters) {
    const int lane = threadIdx.x & 63;
    const uint32_t wid = blockIdx.x * 4 + (threadIdx.x >> 6);
    bf16x8_t a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        u32x4_t ua, ub;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t h0 = mix32((wid * 64 + lane) * 32 + i * 8 + 2 * w);
            const uint32_t h1 = mix32((wid * 64 + lane) * 32 + i * 8 + 2 * w + 1);
            const float s = 1.0f / 32768.0f;
            ua[w] = pack_bf16x2((float)(h0 & 0xffff) * s - 1.0f, (float)(h1 & 0xffff) * s - 1.0f);
            ub[w] = pack_bf16x2((float)(h0 >> 16) * s - 1.0f, (float)(h1 >> 16) * s - 1.0f);
        }
        a[i] = __builtin_bit_cast(bf16x8_t, ua);
        b[i] = __builtin_bit_cast(bf16x8_t, ub);
    }
    f32x16_t acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2 * r + i], b[j], acc[i][j], 0, 0, 0);
    }
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) t += acc[i][j][e];
    out[(int64_t)blockIdx.x * 256 + threadIdx.x] = t;
}

// HBM read floor: each lane reads 16-byte chunks of `buf` (grid-stride) and
// xors them; one 4-byte result per lane keeps the loads live.  The loads run
// as a ring of R = 8 per lane: the load of round t + R is issued as round t's
// data is consumed, so 8 stay in flight without the drain between batches.
// 256 workgroups of 256 lanes measured fastest for 64 MiB: 11.1 us (6.0 TB/s)
// against 11.5 us for batches of 8 and for LDS-DMA streams of 16-48 loads
// in flight per wave; 512 and 1024 workgroups, or rings of 16 and 24, were
// slower.
__global__ __launch_bounds__(256) void hbm_read_kernel(const u32x4_t* __restrict__ buf, int64_t n16,
                                                       uint32_t* __restrict__ out) {
    constexpr int R = 8;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t rounds = n16 / stride;  // chunks i0 + t * stride, t < rounds, exist for every lane
    u32x4_t acc = {0u, 0u, 0u, 0u};
    int64_t t = 0;
    if (rounds >= R) {
        u32x4_t v[R];
#pragma unroll
        for (int r = 0; r < R; ++r) v[r] = __builtin_nontemporal_load(buf + i0 + r * stride);
        for (; t + 2 * R <= rounds; t += R) {  // loads rounds t + R .. t + 2R - 1
#pragma unroll
            for (int r = 0; r < R; ++r) {
                acc ^= v[r];
                v[r] = __builtin_nontemporal_load(buf + i0 + (t + R + r) * stride);
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) acc ^= v[r];  // rounds t .. t + R - 1
        t += R;
    }
    for (; t < rounds; ++t) acc ^= buf[i0 + t * stride];
    if (i0 + rounds * stride < n16) acc ^= buf[i0 + rounds * stride];  // the partial last round
    out[i0] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

}  // namespace

hipError_t launch_hbm_read(const void* buf, int64_t bytes, uint32_t* out, int workgroups,
                           hipStream_t s) {
    hipLaunchKernelGGL(hbm_read_kernel, dim3(workgroups), dim3(256), 0, s,
                       static_cast<const u32x4_t*>(buf), bytes / 16, out);
    return hipGetLastError();
}

hipError_t launch_mfma_ceiling(float* out, int workgroups, int iters, hipStream_t s) {
    hipLaunchKernelGGL(mfma_ceiling_kernel, dim3(workgroups), dim3(256), 0, s, out, iters);
    return hipGetLastError();
}

}  // namespace jh
