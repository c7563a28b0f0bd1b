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
// A [M,K] and B [K,N] are row-major (B[k*N+j], FusedKernels.h:1053).  The
// int8 MFMAs want K contiguous in every lane for both operands; A has it, B
// is transposed on the way:
//
// Decode shapes (M <= 16): HBM-bound, the design of the W8A16 kernel.  Each
// lane loads 16 consecutive columns of 16 consecutive B rows with 16-byte
// loads, transposes the 16x16 bytes in registers (v_perm_b32, 4x4 blocks)
// and feeds each column as the B operand of v_mfma_i32_16x16x64_i8 with A as
// the A operand (M padded to 16).  A workgroup owns 256 columns and one of KS
// K-ranges; the 8 wave partials are summed in LDS and the workgroup adds its
// exact int32 partial tile into C, used as int32 scratch, with integer
// atomics (order-free, so the result is deterministic).  C is zeroed before
// and converted in place after (C = float(sum) * scale + bias), three
// launches in all and no workspace.
//
// Larger M: v_mfma_i32_32x32x32_i8 on 128x128 tiles, 4 waves of 64x64, K in
// slices of 64 staged through double-buffered LDS (next slice in registers
// during the current one's MFMAs).  A fragments are ds_read_b128 of a row;
// B fragments come from two ds_read_b64_tr_b8 each (a 16-lane group reads an
// 8-row x 16-column byte block and lane i receives column i).  Row strides
// are padded so both reads are free of bank conflicts.
//
// Shapes whose rows are not 16-byte aligned (K or N not a multiple of 16, or
// misaligned pointers) take a plain LDS-tiled SIMT kernel.
#include "common.hpp"
#include "launch.hpp"

namespace jh {
namespace {

typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x16_t __attribute__((ext_vector_type(16)));
typedef int i32x2_t __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// SIMT fallback: 64x64 outputs per 256-thread block, 4x4 per thread
// ---------------------------------------------------------------------------
constexpr int BM = 64, BN = 64, BK = 32;

__global__ __launch_bounds__(256) void matmul_int8_simt_kernel(
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

// the epilogue of one output element from its exact integer sum
__device__ __forceinline__ float int8_epilogue(int sum, int m, int n, float scale_a, float scale_b,
                                               const float* row_scale, const float* col_scale,
                                               const float* bias) {
    const float sc = (row_scale ? row_scale[m] : scale_a) * (col_scale ? col_scale[n] : scale_b);
    float c = (float)sum * sc;
    if (bias) c = c + bias[n];
    return c;
}

// ---------------------------------------------------------------------------
// Decode shapes (M <= 16)
// ---------------------------------------------------------------------------
constexpr int DCOLS = 256;      // columns per workgroup: 16 lanes x 16 columns
constexpr int DWAVES = 8;
constexpr int DTHREADS = DWAVES * 64;
constexpr int DKSTEP = 64;      // rows per MFMA k-step
constexpr int DMAX_KS = 8;

struct DPlan {
    int ks;     // K splits
    int steps;  // k-steps per wave
};
inline DPlan dplan(int K, int N) {
    const int total = (K + DKSTEP - 1) / DKSTEP;
    const int tiles = (N + DCOLS - 1) / DCOLS;
    // about 256 workgroups in all, at least two k-steps per wave
    int ks = (256 + tiles - 1) / tiles;
    const int max_ks = (total + 2 * DWAVES - 1) / (2 * DWAVES);
    if (ks > max_ks) ks = max_ks;
    if (ks > DMAX_KS) ks = DMAX_KS;
    if (ks < 1) ks = 1;
    const int per_split = (total + ks - 1) / ks;
    return {ks, (per_split + DWAVES - 1) / DWAVES};
}

// 4x4 byte transpose: rows a, b, c, e (4 column bytes each) -> t[j] = byte j
// of a, b, c, e (one column's 4 rows)
__device__ __forceinline__ void transpose4x4(uint32_t a, uint32_t b, uint32_t c, uint32_t e,
                                             uint32_t (&t)[4]) {
    // v_perm_b32(s0, s1, sel): byte i of the result = byte sel_i of {s0:s1}
    // (0-3 select s1, 4-7 select s0)
    const uint32_t ab_lo = __builtin_amdgcn_perm(b, a, 0x05010400u);  // a0 b0 a1 b1
    const uint32_t ab_hi = __builtin_amdgcn_perm(b, a, 0x07030602u);  // a2 b2 a3 b3
    const uint32_t ce_lo = __builtin_amdgcn_perm(e, c, 0x05010400u);  // c0 e0 c1 e1
    const uint32_t ce_hi = __builtin_amdgcn_perm(e, c, 0x07030602u);  // c2 e2 c3 e3
    t[0] = __builtin_amdgcn_perm(ce_lo, ab_lo, 0x05040100u);         // a0 b0 c0 e0
    t[1] = __builtin_amdgcn_perm(ce_lo, ab_lo, 0x07060302u);         // a1 b1 c1 e1
    t[2] = __builtin_amdgcn_perm(ce_hi, ab_hi, 0x05040100u);
    t[3] = __builtin_amdgcn_perm(ce_hi, ab_hi, 0x07060302u);
}

__global__ void int8_zero_kernel(int* __restrict__ c, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) c[i] = 0;
}

__global__ __launch_bounds__(DTHREADS, 1) void int8_decode_kernel(
    const int8_t* __restrict__ A, const int8_t* __restrict__ B, int* __restrict__ Ci, int M, int N,
    int K, int KS, int steps) {
    __shared__ i32x4_t red[DWAVES * 16 * 64];  // 128 KiB: [wave][j][lane]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tile = blockIdx.x, split = blockIdx.y;
    const int n0 = tile * DCOLS;
    const int lc = lane & 15, lg = lane >> 4;  // column chunk, k group
    const int col0 = n0 + 16 * lc;             // this lane's 16 columns
    const bool col_ok = col0 < N;

    i32x4_t acc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = i32x4_t{0, 0, 0, 0};

    const int total = (K + DKSTEP - 1) / DKSTEP;
    const int per_split = (total + KS - 1) / KS;
    const int s0 = split * per_split;
    const int s1 = min(total, s0 + per_split);

    for (int t = 0; t < steps; ++t) {
        const int st = s0 + wave + DWAVES * t;
        if (st >= s1) break;  // wave-uniform
        const int kb = st * DKSTEP + 16 * lg;  // this lane's 16 rows
        // branch-free loads: an out-of-range row reads row 0 and is replaced by zeros
        u32x4_t wr[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const bool ok = col_ok && kb + r < K;
            const int64_t off = ok ? (int64_t)(kb + r) * N + col0 : 0;
            const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(B + off));
            const u32x4_t z = {0u, 0u, 0u, 0u};
            wr[r] = ok ? v : z;
        }
        // A operand: A[m = lane & 15][kb .. kb+15] (zero past M and K; K % 16 == 0)
        const bool aok = lc < M && kb < K;
        const u32x4_t av = *reinterpret_cast<const u32x4_t*>(A + (aok ? (int64_t)lc * K + kb : 0));
        const u32x4_t z = {0u, 0u, 0u, 0u};
        const i32x4_t a = __builtin_bit_cast(i32x4_t, aok ? av : z);
        // column j = 4q + jj of the 16: byte jj of dword q of the 16 rows
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint32_t col[4][4];  // [jj][row block d]
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                uint32_t t4[4];
                transpose4x4(wr[4 * d][q], wr[4 * d + 1][q], wr[4 * d + 2][q], wr[4 * d + 3][q], t4);
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) col[jj][d] = t4[jj];
            }
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                const i32x4_t b = {(int)col[jj][0], (int)col[jj][1], (int)col[jj][2], (int)col[jj][3]};
                acc[4 * q + jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[4 * q + jj], 0, 0, 0);
            }
        }
    }

    // ---- 8 wave partials summed in LDS; wave w then owns accumulators
    // j = 2w, 2w+1 (lane (lc, lg): rows 4 lg .. 4 lg + 3 of column n0 + 16 lc + j) ----
#pragma unroll
    for (int j = 0; j < 16; ++j) red[(wave * 16 + j) * 64 + lane] = acc[j];
    __syncthreads();
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int j = 2 * wave + h;
        i32x4_t r = red[j * 64 + lane];
#pragma unroll
        for (int w = 1; w < DWAVES; ++w) r += red[(w * 16 + j) * 64 + lane];
        const int c = n0 + 16 * lc + j;
        if (c >= N) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 4 * lg + i;
            if (m < M)
                __hip_atomic_fetch_add(Ci + (int64_t)m * N + c, r[i], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// C = float(sum) * scale + bias in place over the int32 sums
__global__ void int8_finish_kernel(float* __restrict__ C, int M, int N, float scale_a,
                                   float scale_b, const float* __restrict__ row_scale,
                                   const float* __restrict__ col_scale, const float* __restrict__ bias) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)M * N) return;
    const int m = (int)(i / N), n = (int)(i % N);
    const int sum = __builtin_bit_cast(int, C[i]);
    C[i] = int8_epilogue(sum, m, n, scale_a, scale_b, row_scale, col_scale, bias);
}

// ---------------------------------------------------------------------------
// Larger M: 128x128 tiles on v_mfma_i32_32x32x32_i8
// ---------------------------------------------------------------------------
constexpr int TM = 128, TN = 128, TK = 64;
constexpr int A_STRIDE = TK + 16;    // 80 bytes: the 16 rows a b128 read serves hit 16 bank groups
constexpr int B_STRIDE = TN + 32;    // 160 bytes: the 8 rows x 2 column groups of a tr8 read are disjoint
constexpr int A_BYTES = TM * A_STRIDE;
constexpr int B_BYTES = TK * B_STRIDE;
constexpr int STAGE_BYTES = A_BYTES + B_BYTES;

typedef __attribute__((address_space(3))) i32x2_t lds_i32x2;

__global__ __launch_bounds__(256, 2) void int8_mfma_kernel(
    const int8_t* __restrict__ A, const int8_t* __restrict__ B, float* __restrict__ C, int M, int N,
    int K, float scale_a, float scale_b, const float* __restrict__ row_scale,
    const float* __restrict__ col_scale, const float* __restrict__ bias) {
    __shared__ __attribute__((aligned(16))) uint8_t sm[2 * STAGE_BYTES];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;  // 64x64 wave tile
    // XCD-aware order: consecutive workgroup ids go to different XCDs; give
    // each XCD a contiguous run of tiles along N for one row band
    const int tiles_n = (N + TN - 1) / TN, tiles_m = (M + TM - 1) / TM;
    const int nt = tiles_m * tiles_n;
    int b = blockIdx.x;
    if ((nt & 7) == 0) b = (b & 7) * (nt >> 3) + (b >> 3);
    const int m0 = (b / tiles_n) * TM, n0 = (b % tiles_n) * TN;

    // global -> register staging: A tile 128 rows x 64 B (thread: rows r, r+64,
    // 16-byte chunk c); B tile 64 rows x 128 B (thread: rows r, r+32, chunk c)
    const int ar = tid >> 2, ac = tid & 3;
    const int br = tid >> 3, bc = tid & 7;
    u32x4_t ga[2], gb[2];
    auto gload = [&](int k0) {
        const u32x4_t z = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int m = m0 + ar + 64 * h, k = k0 + 16 * ac;
            const bool ok = m < M && k < K;
            const u32x4_t v = *reinterpret_cast<const u32x4_t*>(A + (ok ? (int64_t)m * K + k : 0));
            ga[h] = ok ? v : z;
            const int kr = k0 + br + 32 * h, n = n0 + 16 * bc;
            const bool okb = kr < K && n < N;
            const u32x4_t w = *reinterpret_cast<const u32x4_t*>(B + (okb ? (int64_t)kr * N + n : 0));
            gb[h] = okb ? w : z;
        }
    };
    auto lstore = [&](int st) {
        uint8_t* s = sm + st * STAGE_BYTES;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            *reinterpret_cast<u32x4_t*>(s + (ar + 64 * h) * A_STRIDE + 16 * ac) = ga[h];
            *reinterpret_cast<u32x4_t*>(s + A_BYTES + (br + 32 * h) * B_STRIDE + 16 * bc) = gb[h];
        }
    };

    i32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = i32x16_t{};

    // fragment addresses within a stage
    const int fr = lane & 31, kh = lane >> 5;
    // A: row wm*64 + 32 i + fr, bytes 32 ks + 16 kh .. +15
    // B: tr8 group g = lane/16 reads rows 32 ks + 16 kh + 8 half + s/2, bytes
    //    wn*64 + 32 j + 16 (g & 1) + 8 (s & 1); lane s receives column s of the group
    const int s16 = lane & 15, g2 = (lane >> 4) & 1;
    const int nk = (K + TK - 1) / TK;
    gload(0);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int st = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * TK);
        const uint8_t* s = sm + st * STAGE_BYTES;
#pragma unroll
        for (int ks = 0; ks < TK / 32; ++ks) {
            i32x4_t af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = *reinterpret_cast<const i32x4_t*>(s + (wm * 64 + 32 * i + fr) * A_STRIDE + 32 * ks + 16 * kh);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int row = 32 * ks + 16 * kh + (s16 >> 1);
                const int colb = wn * 64 + 32 * j + 16 * g2 + 8 * (s16 & 1);
                const uint8_t* p0 = s + A_BYTES + row * B_STRIDE + colb;
                const i32x2_t lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)(p0));
                const i32x2_t hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)(p0 + 8 * B_STRIDE));
                bf[j] = i32x4_t{lo[0], lo[1], hi[0], hi[1]};
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) {
            lstore(st ^ 1);
            __syncthreads();
        }
    }

    // epilogue: element e of acc[i][j] is row 8(e/4) + 4 kh + e%4 of the
    // 32x32 tile, column fr
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + wn * 64 + 32 * j + fr;
            if (n >= N) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + wm * 64 + 32 * i + 8 * (e >> 2) + 4 * kh + (e & 3);
                if (m < M)
                    C[(int64_t)m * N + n] =
                        int8_epilogue(acc[i][j][e], m, n, scale_a, scale_b, row_scale, col_scale, bias);
            }
        }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

hipError_t launch_int8(const int8_t* A, const int8_t* B, float* C, int M, int N, int K,
                       float scale_a, float scale_b, const float* row_scale, const float* col_scale,
                       const float* bias, hipStream_t s) {
    if (M == 0 || N == 0) return hipSuccess;
    const bool vec = K > 0 && K % 16 == 0 && N % 16 == 0 && aligned16(A) && aligned16(B);
    if (vec && M <= 16) {
        const int64_t mn = (int64_t)M * N;
        int* Ci = reinterpret_cast<int*>(C);
        hipLaunchKernelGGL(int8_zero_kernel, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, s, Ci, mn);
        const DPlan p = dplan(K, N);
        const int tiles = (N + DCOLS - 1) / DCOLS;
        hipLaunchKernelGGL(int8_decode_kernel, dim3(tiles, p.ks), dim3(DTHREADS), 0, s, A, B, Ci, M,
                           N, K, p.ks, p.steps);
        hipLaunchKernelGGL(int8_finish_kernel, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, s, C,
                           M, N, scale_a, scale_b, row_scale, col_scale, bias);
        return hipGetLastError();
    }
    if (vec) {
        const int nt = ((M + TM - 1) / TM) * ((N + TN - 1) / TN);
        hipLaunchKernelGGL(int8_mfma_kernel, dim3(nt), dim3(256), 0, s, A, B, C, M, N, K, scale_a,
                           scale_b, row_scale, col_scale, bias);
        return hipGetLastError();
    }
    dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
    hipLaunchKernelGGL(matmul_int8_simt_kernel, grid, dim3(256), 0, s, A, B, C, M, N, K, scale_a,
                       scale_b, row_scale, col_scale, bias);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_matmul_int8(const int8_t* A, const int8_t* B, float* C, int M, int N, int K,
                              float scale_a, float scale_b, const float* bias, hipStream_t s) {
    // per-tensor scales: scale_a * scale_b rounded to fp32 first, FusedKernels.h:1061
    return launch_int8(A, B, C, M, N, K, scale_a, scale_b, nullptr, nullptr, bias, s);
}

hipError_t launch_matmul_w8a8(const int8_t* A, const int8_t* B, float* C, int M, int N, int K,
                              const float* scale_a, const float* scale_b, const float* bias,
                              hipStream_t s) {
    return launch_int8(A, B, C, M, N, K, 1.0f, 1.0f, scale_a, scale_b, bias, s);
}

}  // namespace jh
