// w8a16_packed.hip - W8A16 decode GEMM + bias + activation on a packed weight
// layout, for gfx950.
//
//   y[m,j] = act(scale[j] * sum_k x[m,k] * W[k,j] + bias[j])
//
// Same operation and argument meaning as w8a16.hip (jules_hip_w8a16_gemm_bias_act),
// but W is first repacked once (w8a16_pack_kernel, at weight-load time) into
// the order the kernel consumes it.  The row-major kernel has to split K
// across workgroups (a workgroup owning a column strip over all of K would
// read 32-byte pieces of 8 KiB-apart rows, which HBM serves at a fraction of
// its rate) and pays a cross-workgroup reduction at the end of the launch.
// Here a workgroup owns 32 output columns over all of K and reduces its own
// tile in LDS: the launch has no cross-workgroup traffic.
//
// Packed layout.  Column tile c (32 columns) and k-step s (32 rows) form one
// 1 KiB block at Wp + (s * tiles + c) * 1024; inside it lane l's 16 bytes
// are, for kg = l / 16 and j = l % 16,
//   bytes 0..7:  W[32 s + 8 kg + i][32 c + j]       i = 0..7
//   bytes 8..15: W[32 s + 8 kg + i][32 c + 16 + j]
// i.e. exactly the B operands of the two v_mfma_f32_16x16x32_bf16 of that
// k-step (column j and column 16 + j, k = 8 kg .. 8 kg + 7).  Rows past K and
// columns past N are zero.  ksteps = ceil(K / 32), tiles = ceil(N / 32).
// Blocks are k-step-major, and wave w of every workgroup takes k-steps in
// adjacent pairs, 2w, 2w + 1, 2w + 8, 2w + 9, ...: at any moment the whole
// grid reads one contiguous window of W, the access pattern of a plain
// streaming read, and one x load of a pair covers whole 128-byte lines of x.
//
// Per workgroup (4 waves), each wave issues the weight loads of the k-steps 6
// ahead before it converts the current pair, so 6 to 8 steps (24-32 KiB per
// CU) are in flight; more in flight was measured slower.  Each step
// converts the lane's 16 weight bytes to bf16 in registers (int8 is exact in
// bf16) and issues two MFMAs with x (M padded to 16 rows) as the A operand.
// For M <= 8 one x load serves two k-steps (see XP below).  The 4 wave
// partials are summed in LDS in wave order (deterministic); every thread then
// finishes one output (two for M > 8): scale, bias, activation, bf16 store.
#include "common.hpp"
#include "launch.hpp"

namespace jh {
namespace {

constexpr int PK_COLS = 32;     // columns per tile (one workgroup)
constexpr int PK_KSTEP = 32;    // rows per k-step
constexpr int PK_WAVES = 4;
constexpr int PK_THREADS = PK_WAVES * 64;
constexpr int PK_DEPTH = 6;     // k-steps of weight loads issued ahead per wave
// W loads use the default cache policy: the nontemporal hint measured ~1 %
// slower on this read stream
constexpr uint32_t kOOBp = 0x80000000u;  // past every buffer range used: loads return 0
// byte offset of block (tile c, k-step s)
__host__ __device__ __forceinline__ int64_t pk_block(int c, int s, int tiles) {
    return ((int64_t)s * tiles + c) * 1024;
}

__global__ __launch_bounds__(256) void w8a16_pack_kernel(const int8_t* __restrict__ W, int K, int N,
                                                        int ksteps, int tiles,
                                                        int8_t* __restrict__ Wp) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // 16-byte chunk
    const int64_t total = (int64_t)tiles * ksteps * 64;
    if (i >= total) return;
    const int lane = (int)(i & 63);
    const int64_t blk = i >> 6;
    const int s = (int)(blk % ksteps), c = (int)(blk / ksteps);
    const int kg = lane >> 4, j = lane & 15;
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        uint32_t v = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int byte = 4 * q + b;
            const int k = PK_KSTEP * s + 8 * kg + (byte & 7);
            const int col = PK_COLS * c + 16 * (byte >> 3) + j;
            const uint32_t e = (k < K && col < N) ? (uint32_t)(uint8_t)W[(int64_t)k * N + col] : 0u;
            v |= e << (8 * b);
        }
        w[q] = v;
    }
    *reinterpret_cast<u32x4_t*>(Wp + pk_block(c, s, tiles) + lane * 16) =
        u32x4_t{w[0], w[1], w[2], w[3]};
}

// Workgroup barrier ordering LDS only (global loads stay in flight).
__device__ __forceinline__ void pk_lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int ACT, bool XP>
__global__ __launch_bounds__(PK_THREADS, 1) void w8a16_packed_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ Wp, int M, int N, int K, int ksteps,
    const float* __restrict__ scale, const float* __restrict__ bias, uint16_t* __restrict__ y) {
    __shared__ f32x4_t red[PK_WAVES * 2 * 64];  // 8 KiB: [wave][half][lane]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tile = blockIdx.x;
    const int n0 = tile * PK_COLS;
    const int j = lane & 15, kg = lane >> 4;

    // The epilogue gives every thread one output of rows 0-7 (and one of rows
    // 8-15 when M > 8): half eh = tid / 128 (columns 16 eh .. 16 eh + 15),
    // row em = (tid / 16) % 8, column ej = tid % 16.  Its scale and bias are
    // loaded now so their latency is off the tail.
    const int eh = tid >> 7, em = (tid >> 4) & 7, ej = tid & 15;
    const int ecol = n0 + 16 * eh + ej;
    const float esc = scale[min(ecol, N - 1)];
    const float ebi = bias ? bias[min(ecol, N - 1)] : 0.0f;

    // this wave's k-steps, in adjacent pairs: s(t) = 8 (t / 2) + 2 wave + t % 2
    // for t < n (every s < ksteps exactly once over the 4 waves)
    const int tiles = gridDim.x;
    const int full = ksteps >> 3, rest = ksteps & 7;
    const int n = 2 * full + min(max(rest - 2 * wave, 0), 2);
    auto kstep = [&](int t) { return 2 * PK_WAVES * (t >> 1) + 2 * wave + (t & 1); };
    const __amdgpu_buffer_rsrc_t xsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(x), 0, (uint32_t)M * (uint32_t)K * 2u, 0x00020000);

    f32x4_t acc[2] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
    // XP (M <= 8): rows 8..15 of the A operand are padding, so one x load
    // serves two k-steps: lanes j < 8 fetch row j of step t, lanes j >= 8 row
    // j - 8 of step t + 1; step t keeps the low lanes (the high ones zeroed),
    // step t + 1 gets the high lanes' data moved down by a DPP row shift.
    // step t lives in slot t % RING: PK_DEPTH steps ahead plus the pair (or
    // step) being converted
    constexpr int STEP = XP ? 2 : 1;
    constexpr int RING = PK_DEPTH + STEP;
    constexpr int XSLOTS = XP ? RING / 2 : RING;
    u32x4_t wr[RING], xr[XSLOTS];
    auto wload = [&](int t, int d) {
        const bool live = t < n;
        const __amdgpu_buffer_rsrc_t wsrc = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<int8_t*>(Wp) + (live ? pk_block(tile, kstep(t), tiles) : 0), 0,
            live ? 1024u : 0u, 0x00020000);
        wr[d] = __builtin_amdgcn_raw_buffer_load_b128(wsrc, lane * 16, 0, 0);
    };
    // x fragment of local step t, row r, into slot xd.  Range-checked buffer
    // loads stand in for every bounds test: steps past n are past the weight
    // range, x rows past M and k past K get an out-of-range offset; all
    // return 0.
    auto xload = [&](int t, int r, int xd) {
        const int kb = PK_KSTEP * kstep(t) + 8 * kg;
        const uint32_t xo = (r < M && t < n && kb < K) ? (uint32_t)(r * K + kb) * 2u : kOOBp;
        xr[xd] = __builtin_amdgcn_raw_buffer_load_b128(xsrc, xo, 0, 0);
    };
    auto issue = [&](int t, int d) {  // XP: t and d even, issues steps t and t + 1
        wload(t, d);
        if constexpr (XP) {
            wload(t + 1, d + 1);
            xload(j < 8 ? t : t + 1, j & 7, d / 2);
        } else {
            xload(t, j, d);
        }
    };
    auto mfma2 = [&](const u32x4_t& xa4, int d) {
        const bf16x8_t xa = __builtin_bit_cast(bf16x8_t, xa4);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            u32x4_t b;
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const uint32_t dw = wr[d][2 * h + (p >> 1)];
                const int sh = 16 * (p & 1);
                b[p] = pack_bf16x2((float)(int8_t)(dw >> sh), (float)(int8_t)(dw >> (sh + 8)));
            }
            acc[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, __builtin_bit_cast(bf16x8_t, b), acc[h],
                                                             0, 0, 0);
        }
    };
    auto convert = [&](int t, int d) {  // XP: t and d even, converts steps t and t + 1
        if constexpr (XP) {
            const u32x4_t xv = xr[d / 2];
            u32x4_t lo, hi;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                lo[q] = j < 8 ? xv[q] : 0u;
                // row_shl:8 with bound_ctrl: lane j < 8 of each 16-lane row
                // takes lane j + 8, lanes j >= 8 read past the row and get 0
                hi[q] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)xv[q], 0x108, 0xF, 0xF, true);
            }
            if (t < n) mfma2(lo, d);
            if (t + 1 < n) mfma2(hi, d + 1);
        } else {
            if (t < n) mfma2(xr[d], d);
        }
    };
#pragma unroll
    for (int d = 0; d < PK_DEPTH; d += STEP) issue(d, d);
    for (int t0 = 0; t0 < n; t0 += RING) {
#pragma unroll
        for (int d = 0; d < RING; d += STEP) {
            // the steps PK_DEPTH ahead (past n: no traffic) into the slot the
            // previous pair freed, then the current pair
            issue(t0 + d + PK_DEPTH, (d + PK_DEPTH) % RING);
            convert(t0 + d, d);
        }
    }

    // ---- the 4 wave partials of each output, summed in wave order ----
#pragma unroll
    for (int h = 0; h < 2; ++h) red[(wave * 2 + h) * 64 + lane] = acc[h];
    pk_lds_barrier();
    // Output (row m, column 16 eh + ej) sits in component m % 4 of lane
    // 16 (m / 4) + ej of each wave's half-eh accumulator.  Rows past M hold 0;
    // range-checked buffer stores drop them and columns past N without
    // branches (M * N * 2 <= 2^31: every offset fits the 32-bit range).
    const float* redf = reinterpret_cast<const float*>(red);
    const __amdgpu_buffer_rsrc_t ysrc =
        __builtin_amdgcn_make_buffer_rsrc(y, 0, (uint32_t)M * (uint32_t)N * 2u, 0x00020000);
#pragma unroll
    for (int r = 0; r < (XP ? 1 : 2); ++r) {
        const int m = em + 8 * r;
        const int src = ((m >> 2) * 16 + ej) * 4 + (m & 3);
        float sum = redf[eh * 256 + src];
#pragma unroll
        for (int w = 1; w < PK_WAVES; ++w) sum += redf[(w * 2 + eh) * 256 + src];
        float t = sum * esc;
        if (bias) t = t + ebi;
        const uint32_t yo = (m < M && ecol < N) ? (uint32_t)(m * N + ecol) * 2u : kOOBp;
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (__bf16)activate<ACT>(t)),
                                              ysrc, yo, 0, 0);
    }
}

}  // namespace

size_t w8a16_packed_bytes(int K, int N) {
    if (K <= 0 || N <= 0) return 0;
    return (size_t)((N + PK_COLS - 1) / PK_COLS) * (size_t)((K + PK_KSTEP - 1) / PK_KSTEP) * 1024u;
}

hipError_t launch_w8a16_pack(const int8_t* W, int K, int N, int8_t* Wp, hipStream_t s) {
    const int ksteps = (K + PK_KSTEP - 1) / PK_KSTEP, tiles = (N + PK_COLS - 1) / PK_COLS;
    const int64_t chunks = (int64_t)tiles * ksteps * 64;
    hipLaunchKernelGGL(w8a16_pack_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, s, W, K,
                       N, ksteps, tiles, Wp);
    return hipGetLastError();
}

hipError_t launch_w8a16_packed(int act, const uint16_t* x, const int8_t* Wp, const float* scale,
                               const float* bias, uint16_t* y, int M, int N, int K, hipStream_t s) {
    const int ksteps = (K + PK_KSTEP - 1) / PK_KSTEP, tiles = (N + PK_COLS - 1) / PK_COLS;
    hipError_t e = hipSuccess;
    JH_DISPATCH_ACT(act, ACT, {
        if (M <= 8)
            hipLaunchKernelGGL((w8a16_packed_kernel<ACT, true>), dim3(tiles), dim3(PK_THREADS), 0, s, x,
                               Wp, M, N, K, ksteps, scale, bias, y);
        else
            hipLaunchKernelGGL((w8a16_packed_kernel<ACT, false>), dim3(tiles), dim3(PK_THREADS), 0, s, x,
                               Wp, M, N, K, ksteps, scale, bias, y);
        e = hipGetLastError();
    });
    return e;
}

}  // namespace jh
