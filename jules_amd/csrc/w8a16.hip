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
// partials are summed in LDS in wave order and the workgroup stores its fp32
// partial tile to the workspace.  The last of the KS workgroups of a
// column tile to finish (found through per-call flags in the workspace) sums
// the KS partials of the tile in split order and applies scale, bias and the
// activation, so one launch does the whole operation.  The summation order is
// fixed, so results are deterministic run to run.
#include <atomic>
#include <random>

#include "common.hpp"
#include "launch.hpp"

namespace jh {
namespace {

constexpr int COLS = 256;       // columns per workgroup: 16 lanes x 16 columns
constexpr int WAVES = 8;
constexpr int THREADS = WAVES * 64;
constexpr int KSTEP = 32;       // rows per MFMA k-step
constexpr int DEPTH = 4;        // k-steps per wave in flight
constexpr int MAX_KS = 8;       // most K splits (partials) per output
// s_waitcnt immediate for vmcnt(0) with expcnt/lgkmcnt unconstrained (gfx9 encoding)
constexpr unsigned kWaitVm0 = 0x0F70;

struct Plan {
    int ks;         // number of K splits (partials)
    int steps;      // k-steps per wave
};

inline Plan plan(int K) {
    const int total_steps = (K + KSTEP - 1) / KSTEP;
    // aim for DEPTH k-steps per wave, all in flight from the start (fewer
    // splits starve the chip, more cost partial traffic); at most MAX_KS
    // splits (larger K gives each wave more k-steps)
    int ks = (total_steps + WAVES * DEPTH - 1) / (WAVES * DEPTH);
    if (ks > MAX_KS) ks = MAX_KS;
    if (ks < 1) ks = 1;
    const int per_split = (total_steps + ks - 1) / ks;
    const int steps = (per_split + WAVES - 1) / WAVES;
    return {ks, steps};
}

// cache policy bits of buffer instructions: nt (streaming), sc1 (coherent at
// agent scope)
constexpr int kNT = 2;
constexpr int kSc1 = 16;
// a buffer offset past every range used here (buffers hold < 2^31 bytes):
// loads there return 0, stores are dropped
constexpr uint32_t kOOB = 0x80000000u;
constexpr int PART_FLOATS = 16 * 64 * 4;  // one (split, tile) partial: [j][lane] x 4 rows

// Workgroup barrier that orders LDS accesses only: global loads and stores
// stay in flight across it (__syncthreads() waits for them to complete).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// buffer resource over the partial tile of (split, tile); an empty range
// (loads return 0, stores are dropped) when !valid
__device__ __forceinline__ __amdgpu_buffer_rsrc_t part_rsrc(float* partials, int split, int tiles,
                                                           int tile, bool valid) {
    return __builtin_amdgcn_make_buffer_rsrc(partials + ((int64_t)split * tiles + tile) * PART_FLOATS,
                                             0, valid ? PART_FLOATS * 4 : 0, 0x00020000);
}

// COUNTER selects how the last workgroup of a column tile is found: per-call
// flags (flags, call_id; the workspace needs no initialisation) or one
// arrival counter per tile (counters; zero before the call and reset to zero
// by the tile's last workgroup, so the launch arguments never change from
// call to call and a captured graph can replay the launch).
template <int ACT, bool COUNTER>
__global__ __launch_bounds__(THREADS, 1) void w8a16_splitk_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ W, int M, int N, int K, int KS,
    int steps, float* __restrict__ partials, const float* __restrict__ scale,
    const float* __restrict__ bias, uint16_t* __restrict__ y, uint64_t* __restrict__ flags,
    uint64_t call_id, uint32_t* __restrict__ counters) {
    __shared__ f32x4_t red[WAVES * 16 * 64];  // 128 KiB: [wave][j][lane]

    // wave index through readfirstlane: the compiler then knows it (and the
    // per-step buffer resources built from it) to be wave-uniform
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tile = blockIdx.x, split = blockIdx.y;
    const int n0 = tile * COLS;
    const int lc = lane & 15, lg = lane >> 4;     // column chunk, k group
    const int col0 = n0 + 16 * lc;                // this lane's 16 columns
    const bool col_ok = col0 < N;

    f32x4_t acc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // scale and bias of the two columns this lane finishes if its workgroup
    // reduces the tile (see the reducer below), loaded now so that their
    // latency is off the tail
    float sc[2], bi[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int c = min(n0 + 16 * lc + 2 * wave + h, N - 1);
        sc[h] = scale[c];
        bi[h] = bias ? bias[c] : 0.0f;
    }

    // k-steps of this split: [s0, s1); wave w takes s0 + w + WAVES * t
    const int total_steps = (K + KSTEP - 1) / KSTEP;
    const int per_split = (total_steps + KS - 1) / KS;
    const int s0 = split * per_split;
    const int s1 = min(total_steps, s0 + per_split);

    // Weight stream: DEPTH k-steps of every wave in flight (for the decode
    // shape, all of them from the start), each converted as soon as its
    // loads land while the later ones stream.  The loads are buffer loads,
    // whose range check stands in for every bounds test: a k-step gets a
    // buffer over its own rows (no bytes for a step past the split: all its
    // loads return 0), a lane past N gets an out-of-range offset, and the x
    // loads get one where the row is past M or the k-range past K.  So no
    // loaded value passes through a select, and each is waited for only
    // where it is converted.  A lane's offset within a step is fixed: row
    // 8*lg + r, its 16 columns.
    uint32_t wofs[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) wofs[r] = col_ok ? (uint32_t)(8 * lg + r) * (uint32_t)N + col0 : kOOB;
    const __amdgpu_buffer_rsrc_t xsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(x), 0, (uint32_t)M * (uint32_t)K * 2u, 0x00020000);

    u32x4_t wr[DEPTH][8];
    u32x4_t xr[DEPTH];
    auto issue = [&](int t, int slot) {
        const int st = s0 + wave + WAVES * t;
        const bool live = t < steps && st < s1;
        const int rows = live ? min(K - st * KSTEP, KSTEP) : 0;
        const __amdgpu_buffer_rsrc_t wsrc = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<int8_t*>(W) + (live ? (int64_t)st * KSTEP * N : 0), 0, (uint32_t)rows * (uint32_t)N,
            0x00020000);
#pragma unroll
        for (int r = 0; r < 8; ++r) wr[slot][r] = __builtin_amdgcn_raw_buffer_load_b128(wsrc, wofs[r], 0, kNT);
        // A operand: x[m = lane & 15][kb .. kb+7]
        const int kb = st * KSTEP + 8 * lg;
        const uint32_t xo = (live && lc < M && kb < K) ? (uint32_t)(lc * K + kb) * 2u : kOOB;
        xr[slot] = __builtin_amdgcn_raw_buffer_load_b128(xsrc, xo, 0, 0);
    };
    auto convert_mfma = [&](int slot) {
        const bf16x8_t xa = __builtin_bit_cast(bf16x8_t, xr[slot]);
        // column j of the 16: bytes j of the 8 rows -> 8 bf16 (k = kb..kb+7)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int dw = j >> 2, sh = 8 * (j & 3);
            float f[8];
#pragma unroll
            for (int r = 0; r < 8; ++r) f[r] = (float)(int8_t)(wr[slot][r][dw] >> sh);
            u32x4_t b;
            b[0] = pack_bf16x2(f[0], f[1]);
            b[1] = pack_bf16x2(f[2], f[3]);
            b[2] = pack_bf16x2(f[4], f[5]);
            b[3] = pack_bf16x2(f[6], f[7]);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, __builtin_bit_cast(bf16x8_t, b), acc[j], 0, 0, 0);
        }
    };

#pragma unroll
    for (int d = 0; d < DEPTH; ++d) issue(d, d);
    for (int t0 = 0; t0 < steps; t0 += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            if (t0 + d < steps) convert_mfma(d);
            // the step DEPTH ahead into the slot just used; past the last
            // step these loads are out of range (no memory traffic)
            issue(t0 + d + DEPTH, d);
        }
    }

    // ---- reduction of the 8 wave partials in LDS ----
    // Every wave writes its 16 accumulators ([wave][j][lane]: 1 KiB
    // contiguous per instruction); then wave w sums accumulators j = 2w and
    // 2w+1 over the 8 waves in wave order and owns that part of the
    // workgroup's partial tile from here on.  Only lanes holding rows < M
    // (lane < 16 * ceil(M / 4)) take part: the rest hold the zero padding.
    const int lanes_live = 16 * ((M + 3) / 4);
    const bool live = lane < lanes_live;
    if (live) {
#pragma unroll
        for (int j = 0; j < 16; ++j) red[(wave * 16 + j) * 64 + lane] = acc[j];
    }
    lds_barrier();
    f32x4_t r[2] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
    if (live) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int j = 2 * wave + h;
            r[h] = red[j * 64 + lane];
#pragma unroll
            for (int w = 1; w < WAVES; ++w) r[h] += red[(w * 16 + j) * 64 + lane];
        }
    }

    // ---- partial tile out, then the last workgroup of the column tile ----
    // Partials and flags are shared between workgroups on different XCDs,
    // whose L2s are not coherent with each other.  Every access to them
    // carries sc1 (coherent at agent scope: the cache policy of the
    // compiler's agent-scope atomics), so no L2 write-back or invalidate is
    // needed, and the order between them comes from waiting for the waves'
    // own memory operations to complete (vmcnt(0)): the waits of the
    // compiler's agent-scope seq_cst sequences, minus their L2 write-back and
    // invalidate, which exist only for plain (non-coherent) data.  An
    // earlier version released the partials with __threadfence(); its L2
    // write-back (buffer_wbl2) cost more than a separate reduction kernel.
    //
    // A partial tile is stored in the MFMA accumulator layout, [j][lane] x 16
    // bytes (16 KiB per (split, tile)), so each store instruction writes
    // whole cache lines: write-through stores of scattered 8-byte pieces cost
    // a line transfer each.
    //
    // Protocol per workgroup: every wave waits for its partial stores to
    // complete; then wave 0 stores flags[tile][split] = call_id, waits, and
    // loads the tile's KS flags.  The workgroup whose flag store completes
    // last sees every flag equal to call_id (each load is issued after its
    // own flag store completed), so some workgroup reduces; if several do,
    // they write the same bits (same partials, summed in split order).
    // call_id is new for every call, so flags from earlier calls or
    // uninitialised workspace never match.
    // Counter protocol (COUNTER): after its partial stores complete, wave 0
    // increments counters[tile] with a wrapping atomic (global_atomic_inc
    // with limit KS-1: old == KS-1 stores 0, otherwise old+1, one agent-scope
    // read-modify-write); the workgroup that receives KS-1 is the tile's last
    // arrival and reduces, and its own increment has already put the counter
    // back to 0 for the next call.  Exactly one workgroup reduces.  Because
    // the reset is part of the atomic, an increment of an overlapping call
    // is never lost: once every call that ran has finished, each counter has
    // taken a multiple of KS increments and is 0 again.
    const int tiles = gridDim.x;
    {
        const __amdgpu_buffer_rsrc_t pr = part_rsrc(partials, split, tiles, tile, true);
        if (live) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, r[h]), pr,
                                                       ((2 * wave + h) * 64 + lane) * 16, 0, kSc1);
        }
    }
    __builtin_amdgcn_s_waitcnt(kWaitVm0);  // this wave's partial stores are done
    __shared__ int last;
    lds_barrier();                        // ... and every wave's
    if constexpr (COUNTER) {
        if (wave == 0 && lane == 0) {
            const uint32_t old = __builtin_amdgcn_atomic_inc32(counters + tile, (uint32_t)(KS - 1),
                                                               __ATOMIC_RELAXED, "agent");
            last = old == (uint32_t)(KS - 1);
        }
    } else if (wave == 0) {
        uint64_t* tf = flags + (int64_t)tile * KS;
        if (lane == 0) __hip_atomic_store(tf + split, call_id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(kWaitVm0);
        const uint64_t f =
            lane < KS ? __hip_atomic_load(tf + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : call_id;
        const bool all = __builtin_amdgcn_ballot_w64(f != call_id) == 0;
        if (lane == 0) last = all;
    }
    lds_barrier();
    if (!last) return;

    // ---- reducer: y = act(scale * sum_p partials[p] + bias) for the tile ----
    // Wave w finishes accumulators j = 2w, 2w+1: lane (lc, lg) holds rows
    // 4*lg.. of column n0 + 16*lc + j.  The other splits' partials are
    // loaded (contiguous across lanes), its own is r[]; the sum is taken in
    // split order.  The loads are branch-free: a split that is absent or
    // this workgroup's own gets an empty buffer range, and a lane past the
    // rows < M an out-of-range offset (the load returns 0 without touching
    // memory); the absent and own splits are replaced by a select.
    f32x4_t pv[2][MAX_KS];
#pragma unroll
    for (int p = 0; p < MAX_KS; ++p) {
        const __amdgpu_buffer_rsrc_t pr = part_rsrc(partials, p, tiles, tile, p < KS && p != split);
#pragma unroll
        for (int h = 0; h < 2; ++h)
            pv[h][p] = __builtin_bit_cast(
                f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                             pr, live ? ((2 * wave + h) * 64 + lane) * 16 : kOOB, 0, kSc1));
    }
    // keep every load here, in flight together (the compiler would otherwise
    // sink some into the conditional sums below and wait for each in turn)
#pragma unroll
    for (int p = 0; p < MAX_KS; ++p)
#pragma unroll
        for (int h = 0; h < 2; ++h) asm volatile("" : "+v"(pv[h][p]));
    // The tile's outputs go through LDS ([m][256 columns] bf16, 8 KiB at
    // most, in the reduction buffer: every wave has finished reading it) so
    // that y is written with 8-byte stores of 4 consecutive columns.
    uint16_t* stage = reinterpret_cast<uint16_t*>(red);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        f32x4_t sum = split == 0 ? r[h] : pv[h][0];
#pragma unroll
        for (int p = 1; p < MAX_KS; ++p) {
            const f32x4_t v = p == split ? r[h] : pv[h][p];
            if (p < KS) sum += v;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 4 * lg + i;
            if (m < M) {
                float t = sum[i] * sc[h];
                if (bias) t = t + bi[h];
                stage[m * COLS + 16 * lc + 2 * wave + h] = __builtin_bit_cast(uint16_t, (__bf16)activate<ACT>(t));
            }
        }
    }
    lds_barrier();
    for (int e = tid; e < M * (COLS / 4); e += THREADS) {
        const int m = e / (COLS / 4), q = e % (COLS / 4);
        if (n0 + 4 * q < N)  // N % 16 == 0: a group of 4 columns is all in or all out
            *reinterpret_cast<uint2*>(y + (int64_t)m * N + n0 + 4 * q) =
                *reinterpret_cast<const uint2*>(stage + m * COLS + 4 * q);
    }
}

// ---------------------------------------------------------------------------
// int8 x int8 at decode shapes (matmulInt8 / W8A8 with M <= 16): the same
// streaming design and split-K reduction with exact integer arithmetic.
// A lane loads 16 consecutive columns of 16 consecutive B rows, transposes
// the 16x16 bytes in registers (v_perm_b32, 4x4 blocks) and feeds column j
// as the B operand of v_mfma_i32_16x16x64_i8 with A (M padded to 16) as the
// A operand.  Partials are int32 (exact for K <= 131071), summed in split
// order by the last workgroup of the column tile, which applies the epilogue
// C = float(sum) * (sA * sB) + bias of matmulInt8's scalar path.
// ---------------------------------------------------------------------------
constexpr int I8_KSTEP = 64;  // rows per int8 MFMA k-step

typedef int i32x4_t __attribute__((ext_vector_type(4)));

inline Plan plan_int8(int K) {
    const int total_steps = (K + I8_KSTEP - 1) / I8_KSTEP;
    // two k-steps per wave, at most MAX_KS splits (larger K: more k-steps per wave)
    int ks = (total_steps + 2 * WAVES - 1) / (2 * WAVES);
    if (ks > MAX_KS) ks = MAX_KS;
    if (ks < 1) ks = 1;
    const int per_split = (total_steps + ks - 1) / ks;
    return {ks, (per_split + WAVES - 1) / WAVES};
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

__global__ __launch_bounds__(THREADS, 1) void int8_splitk_kernel(
    const int8_t* __restrict__ A, const int8_t* __restrict__ B, int M, int N, int K, int KS,
    int steps, float* __restrict__ partials, float scale_a, float scale_b,
    const float* __restrict__ row_scale, const float* __restrict__ col_scale,
    const float* __restrict__ bias, float* __restrict__ C, uint64_t* __restrict__ flags,
    uint64_t call_id) {
    __shared__ i32x4_t red[WAVES * 16 * 64];  // 128 KiB: [wave][j][lane]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tile = blockIdx.x, split = blockIdx.y;
    const int n0 = tile * COLS;
    const int lc = lane & 15, lg = lane >> 4;  // column chunk, k group
    const int col0 = n0 + 16 * lc;             // this lane's 16 columns
    const bool col_ok = col0 < N;

    i32x4_t acc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = i32x4_t{0, 0, 0, 0};

    // epilogue operands of the two columns this lane finishes if its
    // workgroup reduces the tile, loaded now (off the tail)
    float csc[2], bi[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int c = min(n0 + 16 * lc + 2 * wave + h, N - 1);
        csc[h] = col_scale ? col_scale[c] : scale_b;
        bi[h] = bias ? bias[c] : 0.0f;
    }

    const int total_steps = (K + I8_KSTEP - 1) / I8_KSTEP;
    const int per_split = (total_steps + KS - 1) / KS;
    const int s0 = split * per_split;
    const int s1 = min(total_steps, s0 + per_split);

    for (int t = 0; t < steps; ++t) {
        const int st = s0 + wave + WAVES * t;
        const bool live = st < s1;
        const int kb = st * I8_KSTEP + 16 * lg;  // this lane's 16 rows
        // branch-free loads: an out-of-range row reads element 0 and is
        // replaced by zeros (K % 16 == 0: a lane's rows are all in or all out)
        u32x4_t wr[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const bool ok = live && col_ok && kb + r < K;
            const int64_t off = ok ? (int64_t)(kb + r) * N + col0 : 0;
            const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(B + off));
            const u32x4_t z = {0u, 0u, 0u, 0u};
            wr[r] = ok ? v : z;
        }
        // A operand: A[m = lane & 15][kb .. kb+15]
        const bool aok = live && lc < M && kb < K;
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

    // ---- the 8 wave partials summed in LDS (wave w then owns j = 2w, 2w+1) ----
#pragma unroll
    for (int j = 0; j < 16; ++j) red[(wave * 16 + j) * 64 + lane] = acc[j];
    lds_barrier();
    i32x4_t r[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int j = 2 * wave + h;
        r[h] = red[j * 64 + lane];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) r[h] += red[(w * 16 + j) * 64 + lane];
    }

    // ---- partial tile out, flags, the last workgroup reduces (the protocol
    // of w8a16_splitk_kernel above) ----
    const int tiles = gridDim.x;
    const int lanes_live = 16 * ((M + 3) / 4);
    const bool live = lane < lanes_live;
    {
        const __amdgpu_buffer_rsrc_t pr = part_rsrc(partials, split, tiles, tile, true);
        if (live) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, r[h]), pr,
                                                       ((2 * wave + h) * 64 + lane) * 16, 0, kSc1);
        }
    }
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __shared__ int last;
    lds_barrier();
    if (wave == 0) {
        uint64_t* tf = flags + (int64_t)tile * KS;
        if (lane == 0) __hip_atomic_store(tf + split, call_id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(kWaitVm0);
        const uint64_t f =
            lane < KS ? __hip_atomic_load(tf + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : call_id;
        const bool all = __builtin_amdgcn_ballot_w64(f != call_id) == 0;
        if (lane == 0) last = all;
    }
    lds_barrier();
    if (!last || !live) return;

    i32x4_t pv[2][MAX_KS];
#pragma unroll
    for (int p = 0; p < MAX_KS; ++p) {
        const __amdgpu_buffer_rsrc_t pr = part_rsrc(partials, p, tiles, tile, p < KS && p != split);
#pragma unroll
        for (int h = 0; h < 2; ++h)
            pv[h][p] = __builtin_bit_cast(
                i32x4_t, __builtin_amdgcn_raw_buffer_load_b128(pr, ((2 * wave + h) * 64 + lane) * 16, 0, kSc1));
    }
#pragma unroll
    for (int p = 0; p < MAX_KS; ++p)
#pragma unroll
        for (int h = 0; h < 2; ++h) asm volatile("" : "+v"(pv[h][p]));
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int c = n0 + 16 * lc + 2 * wave + h;
        i32x4_t sum = split == 0 ? r[h] : pv[h][0];
#pragma unroll
        for (int p = 1; p < MAX_KS; ++p) {
            const i32x4_t v = p == split ? r[h] : pv[h][p];
            if (p < KS) sum += v;
        }
        if (c >= N) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 4 * lg + i;
            if (m < M) {
                // the scale product rounded to fp32, one multiply, one add
                const float sc = (row_scale ? row_scale[m] : scale_a) * csc[h];
                float v = (float)sum[i] * sc;
                if (bias) v = v + bi[h];
                C[(int64_t)m * N + c] = v;
            }
        }
    }
}

}  // namespace

// workspace: KS x tiles partial tiles of PART_FLOATS fp32 each, then one
// 64-bit flag per (column tile, split)
size_t w8a16_workspace_size(int M, int N, int K) {
    (void)M;
    const Plan p = plan(K);
    const size_t tiles = (size_t)(N + COLS - 1) / COLS;
    return tiles * p.ks * (PART_FLOATS * sizeof(float) + sizeof(uint64_t));
}

namespace {
// A value no earlier call of this process used: a per-process random start
// plus a call counter (flags left in a workspace by other processes or by
// earlier calls differ from it).
uint64_t next_call_id() {
    static const uint64_t start = [] {
        std::random_device rd;
        return ((uint64_t)rd() << 32) ^ (uint64_t)rd() ^ (uint64_t)(uintptr_t)&rd;
    }();
    static std::atomic<uint64_t> counter{0};
    return start + counter.fetch_add(1, std::memory_order_relaxed) + 1;
}
}  // namespace

// int8 decode workspace: the same layout with the int8 split plan
size_t int8_decode_workspace_size(int M, int N, int K) {
    (void)M;
    const Plan p = plan_int8(K);
    const size_t tiles = (size_t)(N + COLS - 1) / COLS;
    return tiles * p.ks * (PART_FLOATS * sizeof(float) + sizeof(uint64_t));
}

hipError_t launch_int8_decode(const int8_t* A, const int8_t* B, float* C, int M, int N, int K,
                              float scale_a, float scale_b, const float* row_scale,
                              const float* col_scale, const float* bias, void* ws, hipStream_t s) {
    const Plan p = plan_int8(K);
    const int tiles = (N + COLS - 1) / COLS;
    float* partials = static_cast<float*>(ws);
    uint64_t* flags = reinterpret_cast<uint64_t*>(partials + (size_t)tiles * p.ks * PART_FLOATS);
    hipLaunchKernelGGL(int8_splitk_kernel, dim3(tiles, p.ks), dim3(THREADS), 0, s, A, B, M, N, K, p.ks,
                       p.steps, partials, scale_a, scale_b, row_scale, col_scale, bias, C, flags,
                       next_call_id());
    return hipGetLastError();
}

hipError_t launch_w8a16(int act, const uint16_t* x, const int8_t* W, const float* scale,
                        const float* bias, uint16_t* y, int M, int N, int K, void* ws,
                        hipStream_t s) {
    const Plan p = plan(K);
    const int tiles = (N + COLS - 1) / COLS;
    float* partials = static_cast<float*>(ws);
    uint64_t* flags = reinterpret_cast<uint64_t*>(partials + (size_t)tiles * p.ks * PART_FLOATS);
    const uint64_t id = next_call_id();
    hipError_t e = hipSuccess;
    JH_DISPATCH_ACT(act, ACT, {
        hipLaunchKernelGGL((w8a16_splitk_kernel<ACT, false>), dim3(tiles, p.ks), dim3(THREADS), 0, s,
                           x, W, M, N, K, p.ks, p.steps, partials, scale, bias, y, flags, id,
                           nullptr);
        e = hipGetLastError();
    });
    return e;
}

size_t w8a16_partials_size(int M, int N, int K) {
    (void)M;
    const Plan p = plan(K);
    return (size_t)((N + COLS - 1) / COLS) * p.ks * PART_FLOATS * sizeof(float);
}

hipError_t launch_w8a16_counters(int act, const uint16_t* x, const int8_t* W, const float* scale,
                                 const float* bias, uint16_t* y, int M, int N, int K,
                                 float* partials, uint32_t* counters, hipStream_t s) {
    const Plan p = plan(K);
    const int tiles = (N + COLS - 1) / COLS;
    hipError_t e = hipSuccess;
    JH_DISPATCH_ACT(act, ACT, {
        hipLaunchKernelGGL((w8a16_splitk_kernel<ACT, true>), dim3(tiles, p.ks), dim3(THREADS), 0, s,
                           x, W, M, N, K, p.ks, p.steps, partials, scale, bias, y, nullptr,
                           uint64_t(0), counters);
        e = hipGetLastError();
    });
    return e;
}

}  // namespace jh
