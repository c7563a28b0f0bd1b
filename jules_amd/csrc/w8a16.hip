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
// ~1.5 issues per byte.
//
// Work split: a workgroup (8 waves) owns 256 columns and one of KS K-ranges;
// every wave takes its own 32-row k-steps of that range, issuing all of its
// weight loads for up to 4 k-steps before converting the first.  The 8 wave
// partials are summed in LDS in a fixed tree order; the workgroup writes its
// fp32 partial tile to the workspace; the last workgroup to finish a column
// tile (agent-scope counter) sums the KS partials in split order, applies
// scale, bias and the activation, and stores bf16.  The summation order is
// fixed, so results are deterministic run to run.
#include "common.hpp"
#include "launch.hpp"

namespace jh {
namespace {

constexpr int COLS = 256;       // columns per workgroup: 16 lanes x 16 columns
constexpr int WAVES = 8;
constexpr int THREADS = WAVES * 64;
constexpr int KSTEP = 32;       // rows per MFMA k-step
constexpr int GROUP = 4;        // k-steps whose loads are in flight together

struct Plan {
    int ks;         // number of K splits (partials)
    int steps;      // k-steps per wave
};

__host__ __device__ inline Plan plan(int K) {
    const int total_steps = (K + KSTEP - 1) / KSTEP;
    // aim for GROUP k-steps per wave; at most 16 splits
    int ks = (total_steps + WAVES * GROUP - 1) / (WAVES * GROUP);
    if (ks > 16) ks = 16;
    if (ks < 1) ks = 1;
    const int per_split = (total_steps + ks - 1) / ks;
    const int steps = (per_split + WAVES - 1) / WAVES;
    return {ks, steps};
}

inline size_t counters_bytes(int N) { return (size_t)((N + COLS - 1) / COLS * 4 + 255) & ~size_t(255); }

template <int ACT>
__global__ __launch_bounds__(THREADS, 1) void w8a16_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ W, const float* __restrict__ scale,
    const float* __restrict__ bias, uint16_t* __restrict__ y, int M, int N, int K, int KS,
    int steps, uint32_t* __restrict__ counters, float* __restrict__ partials) {
    __shared__ float red[4 * 64 * 64];  // 4 wave slots x 64 lanes x 64 accumulators
    __shared__ int last_flag;

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
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                u32x4_t v = {0u, 0u, 0u, 0u};
                if (live && col_ok && kb + r < K)
                    v = __builtin_nontemporal_load(
                        reinterpret_cast<const u32x4_t*>(W + (int64_t)(kb + r) * N + col0));
                wr[u][r] = v;
            }
            // A operand: x[m = lane & 15][kb .. kb+7]
            u32x4_t xv = {0u, 0u, 0u, 0u};
            if (live && lc < M && kb < K)
                xv = *reinterpret_cast<const u32x4_t*>(x + (int64_t)lc * K + kb);
            xa[u] = __builtin_bit_cast(bf16x8_t, xv);
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
    // slot layout: red[slot][e][lane] so a wave's 64 lanes write 64 consecutive floats
    auto put = [&](int slot) {
#pragma unroll
        for (int j = 0; j < 16; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[(slot * 64 + 4 * j + i) * 64 + lane] = acc[j][i];
    };
    auto add = [&](int slot) {
#pragma unroll
        for (int j = 0; j < 16; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[j][i] += red[(slot * 64 + 4 * j + i) * 64 + lane];
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
    if (wave == 0) {
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
        __threadfence();  // release the partial tile at agent scope
        if (lane == 0) {
            const uint32_t prev = __hip_atomic_fetch_add(&counters[tile], 1u, __ATOMIC_ACQ_REL,
                                                         __HIP_MEMORY_SCOPE_AGENT);
            last_flag = (prev == (uint32_t)(KS - 1));
        }
    }
    __syncthreads();
    if (!last_flag) return;
    __threadfence();  // acquire the other workgroups' partials

    // ---- last workgroup of this column tile: sum KS partials in split order ----
    const int ncols = min(COLS, N - n0);
    for (int e = tid; e < M * ncols; e += THREADS) {
        const int m = e / ncols, c = n0 + e % ncols;
        float s = 0.0f;
        for (int p = 0; p < KS; ++p) s += __builtin_nontemporal_load(partials + ((int64_t)p * M + m) * N + c);
        float v = s * scale[c];
        if (bias) v = v + bias[c];
        y[(int64_t)m * N + c] = __builtin_bit_cast(uint16_t, (__bf16)activate<ACT>(v));
    }
    if (tid == 0) counters[tile] = 0u;  // leave the workspace ready for the next call
}

}  // namespace

size_t w8a16_workspace_size(int M, int N, int K) {
    const Plan p = plan(K);
    return counters_bytes(N) + (size_t)p.ks * M * N * sizeof(float);
}

hipError_t launch_w8a16(int act, const uint16_t* x, const int8_t* W, const float* scale,
                        const float* bias, uint16_t* y, int M, int N, int K, void* ws,
                        hipStream_t s) {
    const Plan p = plan(K);
    const int tiles = (N + COLS - 1) / COLS;
    uint32_t* counters = static_cast<uint32_t*>(ws);
    float* partials = reinterpret_cast<float*>(static_cast<char*>(ws) + counters_bytes(N));
    hipError_t e = hipSuccess;
    JH_DISPATCH_ACT(act, ACT, {
        hipLaunchKernelGGL(w8a16_kernel<ACT>, dim3(tiles, p.ks), dim3(THREADS), 0, s, x, W,
                           scale, bias, y, M, N, K, p.ks, p.steps, counters, partials);
        e = hipGetLastError();
    });
    return e;
}

}  // namespace jh
