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
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"
#include "tiles.hpp"

namespace jh {
namespace {

constexpr int BM = 256, BN = 256, BK = 64;
static_assert(BM == kBf16Tile && BN == kBf16Tile && BK == kBf16RegK, "tile table (tiles.hpp)");
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

// ---------------------------------------------------------------------------
// Full-tile kernel (M % 256 == 0, N % 256 == 0, K % 32 == 0).
//
// Both operand tiles are copied HBM -> LDS by the LDS DMA path
// (global_load_lds_dwordx4: each lane's 16 bytes land at base + 16 * lane),
// with no register staging, through a ring of 4 stages of 32 k each
// (4 x 32 KiB): the copy of slice k+3 is spread over the computation of
// slice k, so a copy has two to three slices of MFMA time to land.
// The LDS has 64 banks of 4 bytes (256 bytes per clock); a ds_read_b128
// serves 16 lanes per clock, a ds_read_b64_tr_b16 32 lanes.
//   A stage: [256 rows][32 k] (64-byte rows), 16-byte chunk c of row r at
//      c ^ ((r >> 2) & 3): the fragment read (16 consecutive rows, one chunk)
//      touches 16 distinct 16-byte bank groups.  Each lane's DMA source
//      address is chosen so the data lands swizzled.
//   B stage: row-major [32 k][256 n] (512-byte rows), 32-byte block b of
//      row r at b ^ (2 * (r & 3)).  The MFMA B operand (8 consecutive k of
//      one n per lane) comes from two ds_read_b64_tr_b16: in each 16-lane
//      group lane s addresses row rb + s/4, 8-byte chunk cb + s%4, and lane i
//      receives B[rb + k][4 cb + i] for k = 0..3.  The two 16-lane groups
//      served together read blocks b and b+1 (b even) of the same 4 rows; the
//      swizzle spreads those 8 reads over all 8 blocks of a 256-byte window.
// A partial K slice cannot be zero-filled by the DMA copy; other shapes use
// the register-staged kernel above.
// ---------------------------------------------------------------------------
constexpr int DBK = 32;                   // k per stage
static_assert(DBK == kBf16DmaK, "tile table (tiles.hpp)");
constexpr int NSTAGE = 4;
constexpr int DTILE = 256 * DBK * 2;      // one operand stage: 16 KiB
constexpr int DSTAGE = 2 * DTILE;         // A then B

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ int swz_a32(int row, int chunk) {
    return row * (DBK * 2) + ((chunk ^ ((row >> 2) & 3)) << 4);
}

// LDS reads issued as inline asm.  Through the builtins, the compiler's
// wait-count pass assumes a transposed read may alias any LDS DMA still in
// flight and inserts a full vmcnt(0) wait before it, serialising the copies
// with the compute.  As asm the reads are not tracked: the code below waits
// on lgkmcnt itself before using a result (lgkm_wait), and reads only stages
// whose copies have completed (vmcnt wait + barrier at the top of a slice).
__device__ __forceinline__ u32x2_t ds_read_tr16_b64(const uint8_t* lds_ptr) {
    u32x2_t v;
    const uint32_t a = (uint32_t)(uintptr_t)lds_ptr;
    asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(v) : "v"(a) : "memory");
    return v;
}
__device__ __forceinline__ u32x4_t ds_read_b128_asm(const uint8_t* lds_ptr) {
    u32x4_t v;
    const uint32_t a = (uint32_t)(uintptr_t)lds_ptr;
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(a) : "memory");
    return v;
}

// One k-step's MFMA operands: 4 A fragments (one ds_read_b128 each) and 4 B
// fragments (two ds_read_b64_tr_b16 each) = 12 LDS reads.
struct Frags {
    u32x4_t a[4];
    u32x4_t b[4];
};

// Waits until at most N LDS reads are outstanding.  LDS reads complete in
// issue order, so with the 12 reads of the next k-step issued after this
// one's, lgkmcnt(12) means this k-step's operands have arrived.  The operands
// pass through the asm so no MFMA that uses them is scheduled before it.
template <int N>
__device__ __forceinline__ void lgkm_wait(Frags& f) {
    asm volatile("s_waitcnt lgkmcnt(%8)"
                 : "+v"(f.a[0]), "+v"(f.a[1]), "+v"(f.a[2]), "+v"(f.a[3]), "+v"(f.b[0]),
                   "+v"(f.b[1]), "+v"(f.b[2]), "+v"(f.b[3])
                 : "n"(N)
                 : "memory");
}

template <int ACT>
__global__ __launch_bounds__(THREADS, 1) void gemm_bf16_dma_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
    const float* __restrict__ bias, uint16_t* __restrict__ C, int M, int N, int K) {
    __shared__ __attribute__((aligned(1024))) uint8_t sm[NSTAGE * DSTAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    // ---- XCD-aware tile order (see gemm_bf16_kernel) ----
    const int tiles_m = M / BM, tiles_n = N / BN;
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

    // wave index as a scalar: the LDS destinations of the copies (M0) and
    // their segment offsets are then computed on the scalar unit
    const int wave_s = __builtin_amdgcn_readfirstlane(wave);

    // ---- copy of one slice: 16 A segments (16 rows x 64 B) and 16 B segments
    // (2 rows x 512 B) of 1 KiB; wave w moves segments w, w+4, w+8, w+12.
    // Piece q (0..7) is one global_load_lds instruction: q < 4 an A segment,
    // else a B segment. ----
    const uint16_t* a_src[4];
    const uint16_t* b_src[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int seg = i * 4 + wave_s;
        const int row = seg * 16 + (lane >> 2);
        const int lc = (lane & 3) ^ ((row >> 2) & 3);
        a_src[i] = A + (int64_t)(m0 + row) * K + 8 * lc;
        const int r = seg * 2 + (lane >> 5);
        const int lu = (lane & 31) ^ (4 * (r & 3));  // 16-byte units: block ^ 2 (r & 3)
        b_src[i] = B + (int64_t)r * N + n0 + 8 * lu;
    }
    auto dma_piece = [&](int stage, int kt, int q) {
        uint8_t* As = sm + stage * DSTAGE;
        const int i = q & 3;
        const int seg = i * 4 + wave_s;
        if (q < 4)
            __builtin_amdgcn_global_load_lds(a_src[i] + kt * DBK, (lds_void*)(As + seg * 1024), 16,
                                             0, 0);
        else
            __builtin_amdgcn_global_load_lds(b_src[i] + (int64_t)kt * DBK * N,
                                             (lds_void*)(As + DTILE + seg * 1024), 16, 0, 0);
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
    const int ts = lane & 15, tdh = (lane >> 4) & 1;

    // LDS byte offsets (within a stage) of the 12 reads of one k-step; the
    // k-step adds 32 bytes to the A offsets (two 16-byte chunks, applied
    // before the swizzle) and 16 rows to the B offsets.
    // Piece p (0..11): p < 4 the A fragment of m-tile p (one ds_read_b128);
    // p = 4 + 2 nt + h the half h of the B fragment of n-tile nt.
    auto piece_addr = [&](int ks, int p) -> int {
        if (p < 4) return swz_a32(wm * 128 + p * 32 + frag_row, ks * 2 + frag_half);
        const int nt = (p - 4) >> 1, h = (p - 4) & 1;
        const int c8 = (wn * 128 + nt * 32 + 16 * tdh) / 4 + (ts & 3);
        const int r0 = 16 * ks + 8 * frag_half + (ts >> 2) + 4 * h;
        return DTILE + r0 * 512 + ((c8 ^ (8 * (r0 & 3))) << 3);
    };
    int off[2][12];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int p = 0; p < 12; ++p) off[ks][p] = piece_addr(ks, p);

    auto read_piece = [&](Frags& f, const uint8_t* stage_base, int ks, int p) {
        const uint8_t* ptr = stage_base + off[ks][p];
        if (p < 4) {
            f.a[p] = ds_read_b128_asm(ptr);
        } else {
            const int nt = (p - 4) >> 1;
            const u32x2_t v = ds_read_tr16_b64(ptr);
            if ((p & 1) == 0) {
                f.b[nt][0] = v[0];
                f.b[nt][1] = v[1];
            } else {
                f.b[nt][2] = v[0];
                f.b[nt][3] = v[1];
            }
        }
    };
    auto mfma1 = [&](const Frags& f, int i) {
        const int mt = i >> 2, nt = i & 3;
        acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(bf16x8_t, f.a[mt]), __builtin_bit_cast(bf16x8_t, f.b[nt]),
            acc[mt][nt], 0, 0, 0);
    };

    // Software pipeline over k-steps of 16.  Each MFMA (32 cycles) is followed
    // by at most one LDS read of the next k-step's operands and, every fourth
    // MFMA, one copy instruction of a later slice, so they issue while the
    // matrix core is busy instead of between groups of MFMAs.  Spreading the
    // copies matters: the four waves' 32 copies of a slice move 32 KiB through
    // the vector memory path (64 bytes per clock), and a burst of them stalls
    // the issuing waves, MFMAs included.  sched_barrier(0) pins this order
    // (the scheduler would otherwise cluster the reads and copies).
    //   k-step 0 of slice kt: MFMAs on f0, reads of k-step 1 into f1, copies
    //     0-3 of slice kt+3 into stage (kt+3)%4.
    //   k-step 1 of slice kt: wait for slice kt+1 (vmcnt + barrier), MFMAs on
    //     f1, copies 4-7 of slice kt+3 and the reads of slice kt+1's k-step 0
    //     into f0.
    // Stage (kt+3)%4 = (kt-1)%4 was last read in k-step 0 of slice kt-1, and
    // every wave passed the barrier of slice kt-1 after those reads completed.
    const int KT = K / DBK;
    auto wait_slice = [&](int kt, int outstanding) {
        // this wave's copies of slice kt have landed once at most the
        // `outstanding` copy instructions issued after them remain
        if (outstanding >= 16) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
        else if (outstanding >= 12) asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
        else if (outstanding >= 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        // A bare s_barrier: __syncthreads() adds a workgroup fence whose wait
        // drains all of this wave's copies (vmcnt(0)).  The waits and the
        // LDS-read asm carry "memory" clobbers, so the compiler keeps copies
        // and reads on their side of the barrier.
        __builtin_amdgcn_s_barrier();
    };
    Frags fr[2];
    auto slice = [&](int kt, auto with_dma, auto with_next) {
        constexpr bool DMA = decltype(with_dma)::value;
        constexpr bool NEXT = decltype(with_next)::value;
        const uint8_t* cur = sm + (kt % NSTAGE) * DSTAGE;
        const int dst = (kt + NSTAGE - 1) % NSTAGE;
        Frags& f0 = fr[0];
        Frags& f1 = fr[1];
        lgkm_wait<0>(f0);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            mfma1(f0, i);
            if (i < 12) read_piece(f1, cur, 1, i);
            if constexpr (DMA)
                if ((i & 3) == 1) dma_piece(dst, kt + NSTAGE - 1, i >> 2);
            __builtin_amdgcn_sched_barrier(0);
        }
        lgkm_wait<0>(f1);
        mfma1(f1, 0);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (NEXT) {
            // issued after slice kt+1: slice kt+2 if it exists (8), and the
            // first half of slice kt+3 (4)
            wait_slice(kt + 1, (kt + 2 < KT ? 8 : 0) + (DMA ? 4 : 0));
        }
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t* nxt = sm + ((kt + 1) % NSTAGE) * DSTAGE;
#pragma unroll
        for (int i = 1; i < 16; ++i) {
            mfma1(f1, i);
            if constexpr (NEXT)
                if (i <= 12) read_piece(f0, nxt, 0, i - 1);
            if constexpr (DMA)
                if ((i & 3) == 3) dma_piece(dst, kt + NSTAGE - 1, 4 + (i >> 2));
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // prologue: slices 0..2 into stages 0..2 (stage 3 is filled during slice 0)
#pragma unroll
    for (int p = 0; p < NSTAGE - 1; ++p)
        if (p < KT)
#pragma unroll
            for (int q = 0; q < 8; ++q) dma_piece(p, p, q);
    wait_slice(0, 8 * (min(KT - 1, NSTAGE - 2)));
#pragma unroll
    for (int p = 0; p < 12; ++p) read_piece(fr[0], sm, 0, p);
    using yes = std::integral_constant<bool, true>;
    using no = std::integral_constant<bool, false>;
    int kt = 0;
    for (; kt + NSTAGE - 1 < KT; ++kt) slice(kt, yes{}, yes{});
    for (; kt + 1 < KT; ++kt) slice(kt, no{}, yes{});
    slice(kt, no{}, no{});

#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
        const int col = n0 + wn * 128 + nt * 32 + frag_row;
        const float bv = bias ? bias[col] : 0.0f;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm * 128 + mt * 32 + 8 * (e >> 2) + 4 * frag_half + (e & 3);
                const float v = act_bf16<ACT>(acc[mt][nt][e] + bv);
                C[(int64_t)row * N + col] = __builtin_bit_cast(uint16_t, (__bf16)v);
            }
        }
    }
}

}  // namespace

hipError_t launch_gemm_bf16(int act, const uint16_t* A, const uint16_t* B, const float* bias,
                            uint16_t* C, int M, int N, int K, hipStream_t s) {
    const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    const bool full = bf16_gemm_tile(M, N, K).variant == GV_BF16_DMA;
    hipError_t e = hipSuccess;
    JH_DISPATCH_ACT(act, ACT, {
        if (full)
            hipLaunchKernelGGL(gemm_bf16_dma_kernel<ACT>, dim3(tiles), dim3(THREADS), 0, s, A, B,
                               bias, C, M, N, K);
        else
            hipLaunchKernelGGL(gemm_bf16_kernel<ACT>, dim3(tiles), dim3(THREADS), 0, s, A, B, bias,
                               C, M, N, K);
        e = hipGetLastError();
    });
    return e;
}

}  // namespace jh
