// matmul_int8.hip - int8 x int8 GEMM with the semantics of matmulInt8's
// scalar path (reference include/jules/Kernel/FusedKernels.h:1046-1066):
//   C[i,j] = float(sum_k A[i,k] * B[k,j]) * (scale_A * scale_B)  [+ bias[j]]
// and its W8A8 form with per-token activation scales sA[i] and per-channel
// weight scales sB[j] (the scale product rounded to fp32 per element):
//   C[i,j] = float(sum_k A[i,k] * B[k,j]) * (sA[i] * sB[j])    [+ bias[j]]
// int32 accumulation is exact (|sum| <= 128*128*K < 2^31 for K <= 131071), so
// any summation order gives the reference's integer; the epilogue is one fp32
// multiply by the fp32-rounded scale product, then one add of bias.
//
// A [M,K] and B [K,N] are row-major (B[k*N+j], FusedKernels.h:1053).  The
// int8 MFMAs want K contiguous in every lane for both operands; A has it, B
// is transposed on the way:
//
// Decode shapes (M <= 16): HBM-bound, the W8A16 kernel's design with integer
// arithmetic (int8_splitk_kernel in w8a16.hip): 16-byte loads of B rows, a
// 16x16 byte transpose in registers, v_mfma_i32_16x16x64_i8, exact int32
// split-K partials summed in split order by the last workgroup of each
// column tile, one launch.  The entry point has no workspace argument, so the
// library keeps one per (device, stream).
//
// Larger M: v_mfma_i32_32x32x32_i8 on 128x128 tiles, 4 waves of 64x64, K in
// slices of 64 staged through double-buffered LDS (next slice in registers
// during the current one's MFMAs).  A fragments are ds_read_b128 of a row;
// B fragments come from two ds_read_b64_tr_b8 each (a 16-lane group reads an
// 8-row x 16-column byte block and lane i receives column i).  Row strides
// are padded so both reads are free of bank conflicts.
//
// Full tiles (M, N multiples of 256, K of 64) take the bf16 GEMM's LDS-DMA
// design instead (int8_dma_kernel below).  Shapes whose rows are not 16-byte
// aligned (K or N not a multiple of 16, or misaligned pointers) take a plain
// LDS-tiled SIMT kernel.
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
    // 32x32 tile, column fr; per-column and per-row factors loaded once
    float cs[2], bv[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = min(n0 + wn * 64 + 32 * j + fr, N - 1);
        cs[j] = col_scale ? col_scale[n] : scale_b;
        bv[j] = bias ? bias[n] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        float rs[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int m = min(m0 + wm * 64 + 32 * i + 8 * (e >> 2) + 4 * kh + (e & 3), M - 1);
            rs[e] = row_scale ? row_scale[m] : scale_a;
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + wn * 64 + 32 * j + fr;
            if (n >= N) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + wm * 64 + 32 * i + 8 * (e >> 2) + 4 * kh + (e & 3);
                if (m < M) {
                    float c = (float)acc[i][j][e] * (rs[e] * cs[j]);
                    if (bias) c = c + bv[j];
                    C[(int64_t)m * N + n] = c;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Full tiles (M, N multiples of 256, K of 64): the bf16 GEMM's LDS-DMA design
// (gemm_bf16.hip) on v_mfma_i32_32x32x32_i8.  256x256 blocks, 4 waves of
// 128x128 (4x4 MFMA tiles, 256 accumulators), K in slices of 64 through a
// ring of 4 LDS stages filled by global_load_lds_dwordx4 (each lane's 16
// bytes land at base + 16 * lane) three slices ahead, so the copies have two
// to three slices of MFMA time to land.
//   A stage: [256 rows][64 k] (64-byte rows), 16-byte chunk c of row r at
//      c ^ ((r >> 2) & 3): a fragment read (16 rows, one chunk) touches 16
//      distinct 16-byte bank groups.
//   B stage: [64 k][256 n] (256-byte rows), 16-byte unit u of row r at
//      u ^ 2 (r & 7).  A B fragment is two ds_read_b64_tr_b8 (rows +0..7 and
//      +8..15 of the lane's 16 k); the two 16-lane groups served together
//      read units u and u+1 (u even) of the same 8 rows, which the swizzle
//      spreads over all 16 units of the 256-byte bank window.
// Each lane's DMA source address is chosen so the data lands swizzled.  Per
// 32-deep k-step a wave issues 4 ds_read_b128 and 8 ds_read_b64_tr_b8 for
// 16 MFMAs, one read and (every fourth MFMA) one copy after each MFMA.
// ---------------------------------------------------------------------------
constexpr int QBK = 64;                // k per stage
constexpr int QNSTAGE = 4;
constexpr int QBM = 256, QBN = 256;
constexpr int QTILE = 256 * QBK;       // one operand stage: 16 KiB
constexpr int QSTAGE = 2 * QTILE;      // A then B

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ int qswz_a(int row, int chunk) {
    return row * QBK + ((chunk ^ ((row >> 2) & 3)) << 4);
}
__device__ __forceinline__ int qswz_b(int row, int unit) {
    return QTILE + row * QBN + ((unit ^ (2 * (row & 7))) << 4);
}

// LDS reads as inline asm (untracked by the compiler's wait-count pass,
// which would otherwise drain every copy in flight before a transposed
// read); lgkm_wait below orders their uses.
__device__ __forceinline__ u32x2_t q_read_tr8(const uint8_t* p) {
    u32x2_t v;
    asm volatile("ds_read_b64_tr_b8 %0, %1" : "=v"(v) : "v"((uint32_t)(uintptr_t)p) : "memory");
    return v;
}
__device__ __forceinline__ u32x4_t q_read_b128(const uint8_t* p) {
    u32x4_t v;
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"((uint32_t)(uintptr_t)p) : "memory");
    return v;
}

struct QFrags {
    u32x4_t a[4];
    u32x4_t b[4];
};
// at most N LDS reads outstanding; the operands pass through the asm so no
// MFMA that uses them is scheduled before it
template <int N>
__device__ __forceinline__ void q_lgkm_wait(QFrags& f) {
    asm volatile("s_waitcnt lgkmcnt(%8)"
                 : "+v"(f.a[0]), "+v"(f.a[1]), "+v"(f.a[2]), "+v"(f.a[3]), "+v"(f.b[0]),
                   "+v"(f.b[1]), "+v"(f.b[2]), "+v"(f.b[3])
                 : "n"(N)
                 : "memory");
}

__global__ __launch_bounds__(256, 1) void int8_dma_kernel(
    const int8_t* __restrict__ A, const int8_t* __restrict__ B, float* __restrict__ C, int M, int N,
    int K, float scale_a, float scale_b, const float* __restrict__ row_scale,
    const float* __restrict__ col_scale, const float* __restrict__ bias) {
    __shared__ __attribute__((aligned(1024))) uint8_t sm[QNSTAGE * QSTAGE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // XCD-aware order: each XCD gets a contiguous run of tiles, walked in
    // groups of 4 row bands
    const int tiles_m = M / QBM, tiles_n = N / QBN;
    const int nblk = tiles_m * tiles_n;
    int t = blockIdx.x;
    if ((nblk & 7) == 0) t = (t & 7) * (nblk >> 3) + (t >> 3);
    constexpr int GM = 4;
    const int group = t / (GM * tiles_n);
    const int first_m = group * GM;
    const int gsize = min(GM, tiles_m - first_m);
    const int tile_m = first_m + (t % (GM * tiles_n)) % gsize;
    const int tile_n = (t % (GM * tiles_n)) / gsize;
    const int m0 = tile_m * QBM, n0 = tile_n * QBN;
    const int wave_s = __builtin_amdgcn_readfirstlane(wave);

    // copy pieces: 16 A segments (16 rows x 64 B) and 16 B segments (4 rows x
    // 256 B) of 1 KiB per slice; wave w moves segments w, w+4, w+8, w+12
    const int8_t* a_src[4];
    const int8_t* b_src[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int seg = i * 4 + wave_s;
        const int row = seg * 16 + (lane >> 2);
        const int lc = (lane & 3) ^ ((row >> 2) & 3);
        a_src[i] = A + (int64_t)(m0 + row) * K + 16 * lc;
        const int r = seg * 4 + (lane >> 4);
        const int lu = (lane & 15) ^ (2 * (r & 7));
        b_src[i] = B + (int64_t)r * N + n0 + 16 * lu;
    }
    auto dma_piece = [&](int stage, int kt, int q) {
        uint8_t* st = sm + stage * QSTAGE;
        const int i = q & 3;
        const int seg = i * 4 + wave_s;
        if (q < 4)
            __builtin_amdgcn_global_load_lds(a_src[i] + kt * QBK, (lds_void*)(st + seg * 1024), 16, 0, 0);
        else
            __builtin_amdgcn_global_load_lds(b_src[i] + (int64_t)kt * QBK * N,
                                             (lds_void*)(st + QTILE + seg * 1024), 16, 0, 0);
    };

    i32x16_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = i32x16_t{};

    const int wm = wave >> 1, wn = wave & 1;
    const int frag_row = lane & 31, frag_half = lane >> 5;
    const int ts = lane & 15, tdh = (lane >> 4) & 1;
    // LDS offsets of the 12 reads of k-step ks: p < 4 the A fragment of
    // m-tile p; p = 4 + 2 nt + h half h (rows +8h) of the B fragment of n-tile nt
    auto piece_addr = [&](int ks, int p) -> int {
        if (p < 4) return qswz_a(wm * 128 + p * 32 + frag_row, ks * 2 + frag_half);
        const int nt = (p - 4) >> 1, h = (p - 4) & 1;
        const int unit = (wn * 128 + nt * 32 + 16 * tdh) / 16;
        const int r0 = 32 * ks + 16 * frag_half + 8 * h + (ts >> 1);
        return qswz_b(r0, unit) + 8 * (ts & 1);
    };
    int off[2][12];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int p = 0; p < 12; ++p) off[ks][p] = piece_addr(ks, p);

    auto read_piece = [&](QFrags& f, const uint8_t* stage_base, int ks, int p) {
        const uint8_t* ptr = stage_base + off[ks][p];
        if (p < 4) {
            f.a[p] = q_read_b128(ptr);
        } else {
            const int nt = (p - 4) >> 1;
            const u32x2_t v = q_read_tr8(ptr);
            if ((p & 1) == 0) {
                f.b[nt][0] = v[0];
                f.b[nt][1] = v[1];
            } else {
                f.b[nt][2] = v[0];
                f.b[nt][3] = v[1];
            }
        }
    };
    auto mfma1 = [&](const QFrags& f, int i) {
        const int mt = i >> 2, nt = i & 3;
        acc[mt][nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4_t, f.a[mt]),
                                                           __builtin_bit_cast(i32x4_t, f.b[nt]),
                                                           acc[mt][nt], 0, 0, 0);
    };

    // The software pipeline of the bf16 kernel: k-step 0 of slice kt runs
    // its MFMAs with the reads of k-step 1 and copies 0-3 of slice kt+3;
    // k-step 1 waits for slice kt+1 (vmcnt + bare barrier), runs its MFMAs
    // with copies 4-7 of slice kt+3 and the reads of slice kt+1's k-step 0.
    // Stage (kt+3)%4 = (kt-1)%4 was last read in k-step 0 of slice kt-1, and
    // every wave passed the barrier of slice kt-1 after those reads completed.
    const int KT = K / QBK;
    auto wait_slice = [&](int outstanding) {
        if (outstanding >= 16) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
        else if (outstanding >= 12) asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
        else if (outstanding >= 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        else if (outstanding >= 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
    };
    QFrags fr[2];
    auto slice = [&](int kt, auto with_dma, auto with_next) {
        constexpr bool DMA = decltype(with_dma)::value;
        constexpr bool NEXT = decltype(with_next)::value;
        const uint8_t* cur = sm + (kt % QNSTAGE) * QSTAGE;
        const int dst = (kt + QNSTAGE - 1) % QNSTAGE;
        QFrags& f0 = fr[0];
        QFrags& f1 = fr[1];
        q_lgkm_wait<0>(f0);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            mfma1(f0, i);
            if (i < 12) read_piece(f1, cur, 1, i);
            if constexpr (DMA)
                if ((i & 3) == 1) dma_piece(dst, kt + QNSTAGE - 1, i >> 2);
            __builtin_amdgcn_sched_barrier(0);
        }
        q_lgkm_wait<0>(f1);
        mfma1(f1, 0);
        __builtin_amdgcn_sched_barrier(0);
        // issued after slice kt+1: slice kt+2 if it exists (8), and the first
        // half of slice kt+3 (4)
        if constexpr (NEXT) wait_slice((kt + 2 < KT ? 8 : 0) + (DMA ? 4 : 0));
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t* nxt = sm + ((kt + 1) % QNSTAGE) * QSTAGE;
#pragma unroll
        for (int i = 1; i < 16; ++i) {
            mfma1(f1, i);
            if constexpr (NEXT)
                if (i <= 12) read_piece(f0, nxt, 0, i - 1);
            if constexpr (DMA)
                if ((i & 3) == 3) dma_piece(dst, kt + QNSTAGE - 1, 4 + (i >> 2));
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // prologue: slices 0..2 into stages 0..2 (stage 3 is filled during slice 0)
#pragma unroll
    for (int p = 0; p < QNSTAGE - 1; ++p)
        if (p < KT)
#pragma unroll
            for (int q = 0; q < 8; ++q) dma_piece(p, p, q);
    wait_slice(8 * min(KT - 1, QNSTAGE - 2));
#pragma unroll
    for (int p = 0; p < 12; ++p) read_piece(fr[0], sm, 0, p);
    using yes = std::integral_constant<bool, true>;
    using no = std::integral_constant<bool, false>;
    int kt = 0;
    for (; kt + QNSTAGE - 1 < KT; ++kt) slice(kt, yes{}, yes{});
    for (; kt + 1 < KT; ++kt) slice(kt, no{}, yes{});
    slice(kt, no{}, no{});

    // epilogue: element e of acc[mt][nt] is row 8(e/4) + 4 frag_half + e%4 of
    // the 32x32 tile, column frag_row.  The per-column and per-row factors
    // are loaded once (the pointers are uniform), then per element the
    // scalar path's arithmetic: fp32 scale product, one multiply, one add.
    float cs[4], bv[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
        const int n = n0 + wn * 128 + nt * 32 + frag_row;
        cs[nt] = col_scale ? col_scale[n] : scale_b;
        bv[nt] = bias ? bias[n] : 0.0f;
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        float rs[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int m = m0 + wm * 128 + mt * 32 + 8 * (e >> 2) + 4 * frag_half + (e & 3);
            rs[e] = row_scale ? row_scale[m] : scale_a;
        }
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
            const int n = n0 + wn * 128 + nt * 32 + frag_row;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + wm * 128 + mt * 32 + 8 * (e >> 2) + 4 * frag_half + (e & 3);
                float c = (float)acc[mt][nt][e] * (rs[e] * cs[nt]);
                if (bias) c = c + bv[nt];
                C[(int64_t)m * N + n] = c;
            }
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
        void* ws = nullptr;
        const hipError_t e = stream_workspace(int8_decode_workspace_size(M, N, K), s, &ws);
        if (e != hipSuccess) return e;
        return launch_int8_decode(A, B, C, M, N, K, scale_a, scale_b, row_scale, col_scale, bias, ws, s);
    }
    if (vec && M % QBM == 0 && N % QBN == 0 && K % QBK == 0) {
        const int nt = (M / QBM) * (N / QBN);
        hipLaunchKernelGGL(int8_dma_kernel, dim3(nt), dim3(256), 0, s, A, B, C, M, N, K, scale_a,
                           scale_b, row_scale, col_scale, bias);
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
