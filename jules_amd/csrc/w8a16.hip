// w8a16.hip - decode-shaped W8A16 GEMM + bias + activation for gfx950.
//
//   y[m,j] = act(scale[j] * sum_k x[m,k] * W[k,j] + bias[j])
//   x bf16 [M,K] (M <= 16), W int8 [K,N] row-major (W[k*N+j], the indexing of
//   matmulInt8, include/jules/Kernel/FusedKernels.h:1053), scale/bias fp32 [N],
//   y bf16 [M,N].
//
// The kernel is HBM-bound: it streams the K*N weight bytes once and does
// ~M MACs per byte.  Each lane loads 16 consecutive columns of 8 consecutive
// W rows with 16-byte loads straight into registers (no LDS staging), converts
// them in-register to bf16 (one v_cvt_f32_i32 with SDWA byte select + sign
// extension per element, one v_cvt_pk_bf16_f32 per pair; int8 values are
// exact in bf16), and feeds them as the B operand of v_mfma_f32_16x16x32_bf16
// with x as the A operand (M padded to 16 rows).  The MFMA is used as the
// dot-product engine only: doing the 8 MACs per byte with v_dot2c_f32_bf16
// would cost ~4 VALU issues per weight byte on top of the conversion and make
// the kernel VALU-bound above the HBM time; with the MFMA the VALU work is
// ~1.5 issues per byte.  16-byte loads matter: a wave can have at most 63
// vector loads outstanding, so narrower loads cap the bytes in flight per CU.
//
// Work split: a workgroup (8 waves) owns 256 columns and one of KS K-ranges;
// every wave takes its own 32-row k-steps of that range, issuing all of its
// weight loads for 2 k-steps before converting the first.  The 8 wave
// partials are summed in LDS in a fixed tree order and the workgroup stores
// its fp32 partial tile to the workspace.  A second, small kernel sums the KS
// partials of every output in split order and applies scale, bias and the
// activation.  The kernel boundary makes the partials visible; an agent-scope
// release fence per workgroup (an L2 write-back on this part) measured
// several microseconds.  The summation order is fixed, so results are
// deterministic run to run.
#include "common.hpp"
#include "launch.hpp"

namespace jh {
namespace {

constexpr int COLS = 256;       // columns per workgroup: 16 lanes x 16 columns
constexpr int WAVES = 8;
constexpr int THREADS = WAVES * 64;
constexpr int KSTEP = 32;       // rows per MFMA k-step
constexpr int GROUP = 2;        // k-steps whose loads are in flight together

struct Plan {
    int ks;         // number of K splits (partials)
    int steps;      // k-steps per wave
};

inline Plan plan(int K) {
    const int total_steps = (K + KSTEP - 1) / KSTEP;
    // aim for two groups of GROUP k-steps per wave (measured best at
    // K = N = 8192: fewer splits starve the chip, more cost partial traffic);
    // at most 16 splits
    int ks = (total_steps + 2 * WAVES * GROUP - 1) / (2 * WAVES * GROUP);
    if (ks > 16) ks = 16;
    if (ks < 1) ks = 1;
    const int per_split = (total_steps + ks - 1) / ks;
    const int steps = (per_split + WAVES - 1) / WAVES;
    return {ks, steps};
}

__global__ __launch_bounds__(THREADS, 1) void w8a16_partial_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ W, int M, int N, int K, int KS,
    int steps, float* __restrict__ partials) {
    __shared__ f32x4_t red[4 * 16 * 64];  // 4 wave slots x 16 accumulators x 64 lanes

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tile = blockIdx.x, split = blockIdx.y;
    const int n0 = tile * COLS;
    const int lc = lane & 15, lg = lane >> 4;     // column chunk, k group
    const int col0 = n0 + 16 * lc;                // this lane's 16 columns
    const bool col_ok = col0 < N;

    f32x4_t acc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // k-steps of this split: [s0, s1); wave w takes s0 + w + WAVES * t
    const int total_steps = (K + KSTEP - 1) / KSTEP;
    const int per_split = (total_steps + KS - 1) / KS;
    const int s0 = split * per_split;
    const int s1 = min(total_steps, s0 + per_split);

    for (int t0 = 0; t0 < steps; t0 += GROUP) {
        u32x4_t wr[GROUP][8];
        bf16x8_t xa[GROUP];
#pragma unroll
        for (int u = 0; u < GROUP; ++u) {
            const int st = s0 + wave + WAVES * (t0 + u);
            const bool live = (t0 + u < steps) && st < s1;
            const int kb = st * KSTEP + 8 * lg;  // this lane's 8 rows
            // Branch-free loads: an out-of-range lane reads element 0 and the
            // value is dropped by a select, so the compiler can wait on each
            // load separately (vmcnt) instead of draining all of them.
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const bool ok = live && col_ok && kb + r < K;
                const int64_t off = ok ? (int64_t)(kb + r) * N + col0 : 0;
                const u32x4_t v =
                    __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(W + off));
                const u32x4_t z = {0u, 0u, 0u, 0u};
                wr[u][r] = ok ? v : z;
            }
            // A operand: x[m = lane & 15][kb .. kb+7]
            const bool xok = live && lc < M && kb < K;
            const u32x4_t xv =
                *reinterpret_cast<const u32x4_t*>(x + (xok ? (int64_t)lc * K + kb : 0));
            const u32x4_t z = {0u, 0u, 0u, 0u};
            xa[u] = __builtin_bit_cast(bf16x8_t, xok ? xv : z);
        }
#pragma unroll
        for (int u = 0; u < GROUP; ++u) {
            if (t0 + u >= steps) break;
            // column j of the 16: bytes j of the 8 rows -> 8 bf16 (k = kb..kb+7)
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int dw = j >> 2, sh = 8 * (j & 3);
                float f[8];
#pragma unroll
                for (int r = 0; r < 8; ++r) f[r] = (float)(int8_t)(wr[u][r][dw] >> sh);
                u32x4_t b;
                b[0] = pack_bf16x2(f[0], f[1]);
                b[1] = pack_bf16x2(f[2], f[3]);
                b[2] = pack_bf16x2(f[4], f[5]);
                b[3] = pack_bf16x2(f[6], f[7]);
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[u], __builtin_bit_cast(bf16x8_t, b),
                                                                 acc[j], 0, 0, 0);
            }
        }
    }

    // ---- fixed-order tree reduction of the 8 wave partials in LDS ----
    // slot layout red[slot][j][lane]: a wave's 64 lanes write 1 KiB contiguously
    auto put = [&](int slot) {
#pragma unroll
        for (int j = 0; j < 16; ++j) red[(slot * 16 + j) * 64 + lane] = acc[j];
    };
    auto add = [&](int slot) {
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[j] += red[(slot * 16 + j) * 64 + lane];
    };
    if (wave >= 4) put(wave - 4);
    __syncthreads();
    if (wave < 4) add(wave);
    __syncthreads();
    if (wave >= 2 && wave < 4) put(wave - 2);
    __syncthreads();
    if (wave < 2) add(wave);
    __syncthreads();
    if (wave == 1) put(0);
    __syncthreads();
    if (wave != 0) return;
    add(0);
    // 16x16 output layout: lane holds rows 4*lg + i, column n' = lc of
    // MFMA j, i.e. global column col0 + j
    float* part = partials + (int64_t)split * M * N;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = 4 * lg + i;
        if (m < M && col_ok) {
#pragma unroll
            for (int j4 = 0; j4 < 4; ++j4) {
                f32x4_t v = {acc[4 * j4][i], acc[4 * j4 + 1][i], acc[4 * j4 + 2][i], acc[4 * j4 + 3][i]};
                *reinterpret_cast<f32x4_t*>(part + (int64_t)m * N + col0 + 4 * j4) = v;
            }
        }
    }
}

// y = act(scale * sum_p partials[p] + bias): each thread 4 consecutive
// columns of one row, all KS partial loads issued before the first add, the
// sum taken in split order.
template <int ACT>
__global__ __launch_bounds__(256) void w8a16_finalize_kernel(
    const float* __restrict__ partials, const float* __restrict__ scale,
    const float* __restrict__ bias, uint16_t* __restrict__ y, int M, int N, int KS) {
    const int64_t e0 = 4 * ((int64_t)blockIdx.x * 256 + threadIdx.x);
    if (e0 >= (int64_t)M * N) return;
    const int m = (int)(e0 / N), c = (int)(e0 % N);
    f32x4_t part[16];
#pragma unroll
    for (int p = 0; p < 16; ++p)
        if (p < KS) part[p] = *reinterpret_cast<const f32x4_t*>(partials + ((int64_t)p * M + m) * N + c);
    f32x4_t sum = part[0];
#pragma unroll
    for (int p = 1; p < 16; ++p)
        if (p < KS) sum += part[p];
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float t = sum[i] * scale[c + i];
        if (bias) t = t + bias[c + i];
        v[i] = activate<ACT>(t);
    }
    u32x2_t o = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    *reinterpret_cast<u32x2_t*>(y + (int64_t)m * N + c) = o;
}

}  // namespace

size_t w8a16_workspace_size(int M, int N, int K) {
    const Plan p = plan(K);
    return (size_t)p.ks * M * N * sizeof(float);
}

hipError_t launch_w8a16(int act, const uint16_t* x, const int8_t* W, const float* scale,
                        const float* bias, uint16_t* y, int M, int N, int K, void* ws,
                        hipStream_t s) {
    const Plan p = plan(K);
    const int tiles = (N + COLS - 1) / COLS;
    float* partials = static_cast<float*>(ws);
    hipLaunchKernelGGL(w8a16_partial_kernel, dim3(tiles, p.ks), dim3(THREADS), 0, s, x, W, M, N,
                       K, p.ks, p.steps, partials);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t quads = ((int64_t)M * N) / 4;  // N % 16 == 0
    const unsigned blocks = (unsigned)((quads + 255) / 256);
    JH_DISPATCH_ACT(act, ACT, {
        hipLaunchKernelGGL(w8a16_finalize_kernel<ACT>, dim3(blocks), dim3(256), 0, s, partials,
                           scale, bias, y, M, N, p.ks);
        e = hipGetLastError();
    });
    return e;
}

}  // namespace jh
