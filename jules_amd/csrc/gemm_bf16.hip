// gemm_bf16.hip - bf16 fused GEMM + bias + activation on gfx950 MFMA.
//
// C[M,N] (bf16) = act(A[M,K] . B[K,N] + bias[N]), A and B bf16 row-major (the
// reference's layout, FusedKernels.h:378: A[i*K+k], B[k*N+j]), fp32
// accumulation in v_mfma_f32_32x32x16_bf16, epilogue in fp32.
//
// Block tile 256 x 256 x 64, 256 threads = 4 waves in a 2 x 2 grid, each wave
// owning a 128 x 128 sub-tile = 4 x 4 MFMA tiles of 32 x 32 (256 fp32
// accumulators per lane).  At 4096^3 this is 256 workgroups: one per CU.
//
// Operand staging.  The MFMA wants, per lane, 8 consecutive k of one row of
// A and 8 consecutive k of one column of B.  A rows are k-contiguous in HBM;
// B columns are not (B is [K,N] row-major).  Each thread therefore loads an
// 8(k) x 8(n) block of B with eight 16-byte row loads and transposes it in
// registers with 32 v_perm_b32, so that B is stored in LDS n-major with k
// contiguous, exactly like A.  Both LDS tiles are 256 rows x 128 bytes, 16-byte
// chunk c of row r stored at chunk position c ^ ((r ^ (r >> 3)) & 7): the
// MFMA fragment reads (8 consecutive rows, one chunk) and the transposed B
// stores (rows 8 apart, one chunk) then both hit distinct bank groups.
//
// Pipeline: two LDS stages (128 KiB).  Iteration kt issues the HBM loads of
// slice kt+1 into registers, runs the 64 MFMAs of slice kt from LDS, then
// writes slice kt+1 into the other stage; one barrier per slice.
//
// Workgroup order is XCD aware: consecutive workgroup ids land on different
// XCDs (round robin over 8), so ids are remapped so that each XCD's workgroups
// cover a compact 4-row band of output tiles that shares A and B slices in
// that XCD's L2.
#include "common.hpp"
#include "launch.hpp"

namespace jh {
namespace {

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int THREADS = 256;
constexpr int TILE_BYTES = 256 * BK * 2;  // one operand tile in LDS: 32 KiB
constexpr int STAGE_BYTES = 2 * TILE_BYTES;

__device__ __forceinline__ int swz(int row, int chunk) {
    return row * (BK * 2) + ((chunk ^ ((row ^ (row >> 3)) & 7)) << 4);
}

// bf16 GELU for the MFMA path: gelu_tanh(x) = x * sigmoid(2u),
// u = sqrt(2/pi) (x + 0.044715 x^3), with the hardware exp2 and reciprocal.
// The bit-exact fast_exp epilogue of the fp32 path costs ~40 VALU ops per
// element (a correctly rounded divide among them); bf16 output needs 8 bits.
__device__ __forceinline__ float gelu_fast(float x) {
    const float k1 = -2.0f * 0.7978845608f * 1.4426950408889634f;
    const float k2 = k1 * 0.044715f;
    const float x2 = x * x;
    const float t = __builtin_amdgcn_exp2f(x * __builtin_fmaf(k2, x2, k1));
    return x * __builtin_amdgcn_rcpf(1.0f + t);
}

__device__ __forceinline__ float sigmoid_fast(float x) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

template <int ACT>
__device__ __forceinline__ float act_bf16(float x) {
    if constexpr (ACT == JH_ACT_GELU) return gelu_fast(x);
    else if constexpr (ACT == JH_ACT_SILU) return x * sigmoid_fast(x);
    else if constexpr (ACT == JH_ACT_SIGMOID) return sigmoid_fast(x);
    else if constexpr (ACT == JH_ACT_TANH) return 2.0f * sigmoid_fast(2.0f * x) - 1.0f;
    else if constexpr (ACT == JH_ACT_RELU) return (x > 0.0f) ? x : 0.0f;
    else return x;
}

template <int ACT>
__global__ __launch_bounds__(THREADS, 1) void gemm_bf16_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
    const float* __restrict__ bias, uint16_t* __restrict__ C, int M, int N, int K) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * STAGE_BYTES];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    // ---- XCD-aware tile order ----
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    const int nblk = tiles_m * tiles_n;
    int t = blockIdx.x;
    if ((nblk & 7) == 0) t = (t & 7) * (nblk >> 3) + (t >> 3);
    constexpr int GM = 4;
    const int group = t / (GM * tiles_n);
    const int first_m = group * GM;
    const int gsize = min(GM, tiles_m - first_m);
    const int tile_m = first_m + (t % (GM * tiles_n)) % gsize;
    const int tile_n = (t % (GM * tiles_n)) / gsize;
    const int m0 = tile_m * BM, n0 = tile_n * BN;

    // ---- global -> register assignment ----
    const int a_row = tid >> 3, a_chunk = tid & 7;  // rows a_row + 32*i, chunk a_chunk
    const int b_kb = tid >> 5, b_nb = tid & 31;     // 8x8 block: k 8*b_kb.., n 8*b_nb..
    u32x4_t ra[8], rb[8];

    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int gm = m0 + a_row + 32 * i, gk = k0 + a_chunk * 8;
            u32x4_t v = {0u, 0u, 0u, 0u};
            if (gm < M && gk < K) v = *reinterpret_cast<const u32x4_t*>(A + (int64_t)gm * K + gk);
            ra[i] = v;
        }
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int gk = k0 + 8 * b_kb + r, gn = n0 + 8 * b_nb;
            u32x4_t v = {0u, 0u, 0u, 0u};
            if (gk < K && gn < N) v = *reinterpret_cast<const u32x4_t*>(B + (int64_t)gk * N + gn);
            rb[r] = v;
        }
    };

    auto lstore = [&](int stage) {
        uint8_t* As = smem + stage * STAGE_BYTES;
        uint8_t* Bs = As + TILE_BYTES;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            *reinterpret_cast<u32x4_t*>(As + swz(a_row + 32 * i, a_chunk)) = ra[i];
        // 8x8 transpose of 16-bit elements: column j of the loaded block
        // becomes LDS row n = 8*b_nb + j holding k = 8*b_kb .. 8*b_kb+7.
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
            u32x4_t tv;
#pragma unroll
            for (int c = 0; c < 4; ++c)
                tv[c] = __builtin_amdgcn_perm(rb[2 * c + 1][j >> 1], rb[2 * c][j >> 1], sel);
            *reinterpret_cast<u32x4_t*>(Bs + swz(8 * b_nb + j, b_kb)) = tv;
        }
    };

    f32x16_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    const int wm = wave >> 1, wn = wave & 1;
    const int frag_row = lane & 31;
    const int frag_half = lane >> 5;

    auto compute = [&](int stage) {
        const uint8_t* As = smem + stage * STAGE_BYTES;
        const uint8_t* Bs = As + TILE_BYTES;
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int chunk = ks * 2 + frag_half;
            bf16x8_t af[4], bfr[4];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
                af[mt] = *reinterpret_cast<const bf16x8_t*>(
                    As + swz(wm * 128 + mt * 32 + frag_row, chunk));
#pragma unroll
            for (int nt = 0; nt < 4; ++nt)
                bfr[nt] = *reinterpret_cast<const bf16x8_t*>(
                    Bs + swz(wn * 128 + nt * 32 + frag_row, chunk));
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int nt = 0; nt < 4; ++nt)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mt], bfr[nt],
                                                                          acc[mt][nt], 0, 0, 0);
        }
    };

    const int KT = (K + BK - 1) / BK;
    if (KT > 0) {
        gload(0);
        lstore(0);
        __syncthreads();
        for (int kt = 0; kt < KT; ++kt) {
            const int cur = kt & 1;
            const bool more = kt + 1 < KT;
            if (more) gload((kt + 1) * BK);
            compute(cur);
            if (more) lstore(cur ^ 1);
            __syncthreads();
        }
    }

    // ---- epilogue: bias + activation in fp32, bf16 store ----
    // 32x32 MFMA output layout: lane holds column (lane & 31), element e holds
    // row 8*(e/4) + 4*(lane/32) + (e%4).
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
        const int col = n0 + wn * 128 + nt * 32 + frag_row;
        if (col >= N) continue;
        const float bv = bias ? bias[col] : 0.0f;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm * 128 + mt * 32 + 8 * (e >> 2) + 4 * frag_half + (e & 3);
                if (row < M) {
                    const float v = act_bf16<ACT>(acc[mt][nt][e] + bv);
                    C[(int64_t)row * N + col] = __builtin_bit_cast(uint16_t, (__bf16)v);
                }
            }
        }
    }
}

}  // namespace

hipError_t launch_gemm_bf16(int act, const uint16_t* A, const uint16_t* B, const float* bias,
                            uint16_t* C, int M, int N, int K, hipStream_t s) {
    const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    hipError_t e = hipSuccess;
    JH_DISPATCH_ACT(act, ACT, {
        hipLaunchKernelGGL(gemm_bf16_kernel<ACT>, dim3(tiles), dim3(THREADS), 0, s, A, B, bias,
                           C, M, N, K);
        e = hipGetLastError();
    });
    return e;
}

}  // namespace jh
