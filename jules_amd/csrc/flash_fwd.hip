// flash_fwd.hip - flash-attention forward on gfx950 MFMA.
//
// O = softmax(scale * Q K^T [causal mask]) V per (batch, head); Q, K, V, O are
// [B,H,S,D] row-major, D in {64, 128}.  The reference is flashAttention
// (include/jules/Kernel/FlashAttention.h:130-309): per query tile, per key
// tile, scores -> running row max -> rescale of the accumulator and the
// running sum by exp(m_old - m_new) -> p = exp(s - m_new) -> acc += p V ->
// O = acc / sum.  This kernel keeps that online-softmax recurrence and adds
// the causal mask and an explicit scale.
//
// Orientation.  Scores are computed transposed, S^T = K Q^T: the MFMA's A
// operand is a 32-key slice of K (k-dimension = head dim, contiguous in HBM),
// its B operand 32 queries of Q.  In the 32x32 MFMA output layout every lane
// then owns ONE query column (lane & 31) and 16 of the 32 keys, the other half
// of the keys sitting in lane ^ 32.  Consequences:
//   - the running max/sum are per-lane scalars; the row max needs a single
//     exchange with lane ^ 32, the row sum none until the very end;
//   - the accumulator rescale by exp(m_old - m_new) is a per-lane multiply;
//   - the score registers are, after conversion, directly the B operand of
//     O^T = V^T P^T: for key step kk the 8 keys a lane holds are
//     {16kk + 4g + 0..3, 16kk + 8 + 4g + 0..3} (g = lane / 32), which are
//     accumulator elements 8*(kk%2) .. 8*(kk%2)+7 of score tile kk/2.
// V^T must supply the same 8 keys per lane; the bf16 kernel reads it with
// transposing LDS reads (ds_read_b64_tr_b16), the fp32 kernel needs no
// transpose (see the per-kernel notes below).
//
// Blocks: bf16 = 8 waves x 32 queries (256 rows) sharing K/V tiles of 64
// keys; fp32 = 32 queries whose key range is split across 4 waves.  Causal
// blocks stop at the diagonal, the heaviest query tiles of a head are
// dispatched first, and each XCD works through whole heads so K and V are
// re-read from its L2.
//
// bf16: v_mfma_f32_32x32x16_bf16, fp32 softmax statistics, exp2 with
// scale*log2(e) folded into one fma.  fp32: v_mfma_f32_32x32x2_f32 (full fp32
// products), same recurrence.
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"

namespace jh {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32, 64); }

// Workgroup -> (head, query tile).  Workgroups are dealt to the 8 XCDs round
// robin; the mapping gives each XCD whole heads (head = 8*j + xcd), taken four
// at a time: the query tiles of heads j = 4g .. 4g+3 are interleaved, heaviest
// (causal: most keys) first.  The workgroups an XCD runs at once then span a
// few heads whose K and V tiles are read by neighbouring query tiles close
// together in time, so they come from that XCD's L2 rather than HBM, and the
// CUs that finish early take the next heavy tiles.
// Why four: inside an XCD workgroups start in order and are dealt to its 4
// shader engines in a fixed rotation (timestamps with HW_ID show it); a
// workgroup waits for a free CU on its own engine even when others are idle.
// With four heads interleaved the four engines receive identical sequences of
// tile sizes.  Two heads interleaved gave two engines all the even query
// tiles and two all the odd ones, one key tile per workgroup apart: the
// lighter engines idled behind the in-order dispatch (30.3 of 32 CUs busy on
// average at C4's shape, causal; 1.103 -> 1.082 ms with four).
__device__ __forceinline__ void block_coords(int BH, int nq, int bq, int* bh, int* q0) {
    const int b = blockIdx.x;
    int head, qi;
    if ((BH & 7) == 0) {
        const int xcd = b & 7, i = b >> 3;
        const int J = BH >> 3;                   // heads of this XCD
        const int g = i / (4 * nq), r = i - g * 4 * nq;
        const int gs = min(4, J - 4 * g);        // heads in this group (fewer in a last one)
        head = 8 * (4 * g + r % gs) + xcd;
        qi = r / gs;
    } else {
        head = b / nq;
        qi = b % nq;
    }
    *bh = head;
    *q0 = (nq - 1 - qi) * bq;
}

// ---------------------------------------------------------------------------
// bf16
//
// Workgroup: 8 waves x 32 queries = 256 query rows, two waves per SIMD (up to
// 256 registers each).  The waves form two groups, A = waves 0-3 and B =
// waves 4-7, one wave of each per SIMD, run half a tile out of phase.  Phase
// p ends with a barrier of all 8 waves; in each phase one group issues MFMAs
// while the other runs the softmax on the vector ALU, so the SIMD's matrix
// core and vector ALU work at the same time (they co-issue across waves):
//   MFMA(j):    S_j = K_j Q^T (this wave's 32 queries x 64 keys) and
//               O^T += V_{j-1}^T P_{j-1}^T;
//   SOFTMAX(j): row max of S_j, running-max update (acc *= alpha when it
//               moved), P_j = exp2(S_j c - m) packed to bf16, row sums.
//   group A: MFMA(j) in phase 2j,     SOFTMAX(j) in phase 2j+1;
//   group B: MFMA(j) in phase 2j+1,   SOFTMAX(j) in phase 2j+2.
// At D = 128 only the barriers after odd phases are kept (one per key tile):
// each group runs its two halves of a tile back to back and the groups meet
// once per tile, still half a tile apart.
//
// K and V tiles of 64 keys go HBM -> LDS by the LDS DMA path
// (global_load_lds_dwordx4: each lane's 16 bytes land at base + 16 * lane)
// through a ring of 4 stages; tile t lives in stage t % 4.  K_t is read in
// phases 2t and 2t+1, V_t in phases 2t+2 and 2t+3, so the K half of tile
// t+4 is copied in phase 2t+4 and its V half in phase 2t+5 (all 8 waves
// share the copies; splitting them spreads their LDS writes over both
// phases), and the tile has until phase 2t+8 to land.
// Each lane's source address is permuted so the data lands in the swizzled
// layouts below (LDS: 64 banks of 4 bytes; a ds_read_b128 serves 16 lanes per
// clock, a ds_read_b64_tr_b16 32 lanes).  Both tiles are row-major [key][d],
// D*2 bytes per row:
//   K: 16-byte unit u of row r at u ^ kswz(r).  The S^T A operand (one key
//      row, 8 consecutive d per lane) is one ds_read_b128; the 16 rows a
//      read serves per clock land in 16 distinct 16-byte bank groups.
//   V: 8-byte chunk c of row r at c ^ vswz(r).  The V^T A operand (8 keys of
//      one d per lane) comes from two ds_read_b64_tr_b16: in each 16-lane
//      group lane s addresses row rb + s/4, chunk cb + s%4, and lane i
//      receives V[rb + k][4 cb + i] for k = 0..3; the two groups served
//      together read chunks cb..cb+7 of the same 4 rows, which the swizzle
//      spreads over all 8 32-byte blocks of a 256-byte bank window.
// The MFMA phase's LDS reads form one stream with a fixed look-ahead, so each
// MFMA waits on a constant lgkmcnt.  The reads are inline asm: through the
// builtins the compiler's wait-count pass assumes they may alias any LDS DMA
// in flight and drains all copies (vmcnt(0)) first.
//
// Lazy rescale: the running max only moves when a tile's max exceeds it by
// more than 8 (log2 units); p = exp2(s*c - m) then stays <= 256, exact in the
// recurrence because the sum l uses the same m.
// ---------------------------------------------------------------------------
constexpr int BQ2 = 256;  // query rows per bf16 workgroup
constexpr int NW2 = 8;    // waves per bf16 workgroup

template <int D>
struct Bf16Cfg {
    static constexpr int BKV = 64;
    static constexpr int ROW = D * 2;              // bytes per K / V row in LDS
    static constexpr int TILE = BKV * ROW;         // one operand tile
    static constexpr int STAGE = 2 * TILE;         // K then V
    static constexpr int NSTAGE = 4;
    static constexpr int UNITS = ROW / 16;         // 16-byte units per row
    static constexpr int NSEG = TILE / 1024;       // 1 KiB DMA segments per operand tile
    static constexpr int SEGW = NSEG / NW2;        // copy instructions per wave per operand tile
    static constexpr int RPS = 1024 / ROW;         // rows per segment
    static constexpr int KS = D / 16;              // k-steps of S^T = K Q^T
    static constexpr int DT = D / 32;              // 32-row d tiles of O^T
    static constexpr int NS = 2 * KS;              // MFMAs of one S tile (two 32-key halves)
    static constexpr int NPV = 4 * DT;             // MFMAs of one PV product (four 16-key steps)
};

// Order of the MFMAs of one MFMA phase: S and PV products alternate when
// both are present.  MFMA m needs one LDS read (S: a K fragment) or two (PV:
// the two halves of a V^T fragment), read in MFMA order.
template <bool DO_S, bool DO_PV, int NS, int NPV>
struct MfmaSeq {
    static constexpr int NM = (DO_S ? NS : 0) + (DO_PV ? NPV : 0);
    static constexpr bool is_s(int m) { return DO_S && (!DO_PV || (m % 2 == 0)); }
    static constexpr int idx(int m) { return (DO_S && DO_PV) ? m / 2 : m; }
    // reads of MFMAs 0..m
    static constexpr int reads_upto(int m) {
        int r = 0;
        for (int k = 0; k <= m && k < NM; ++k) r += is_s(k) ? 1 : 2;
        return r;
    }
    // the MFMA read r belongs to
    static constexpr int owner(int r) {
        int k = 0;
        while (reads_upto(k) <= r) ++k;
        return k;
    }
};

template <int D>
__host__ __device__ constexpr int kswz(int r) { return D == 128 ? (r & 15) : ((r >> 1) & 7); }
template <int D>
__host__ __device__ constexpr int vswz(int r) { return D == 128 ? 8 * (r & 3) : 8 * ((r >> 1) & 1); }

typedef __attribute__((address_space(3))) void lds_void;

template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

template <int OFF>
__device__ __forceinline__ u32x4_t lds_b128(uint32_t addr) {
    u32x4_t v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF) : "memory");
    return v;
}
template <int OFF>
__device__ __forceinline__ u32x2_t lds_tr16(uint32_t addr) {
    u32x2_t v;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF) : "memory");
    return v;
}
// Waits until at most N LDS reads are outstanding; the operand passes through
// the asm so its consumer is not scheduled above the wait.
template <int N, typename T>
__device__ __forceinline__ void lgkm_wait(T& v) {
    static_assert(N >= 0 && N <= 15, "lgkmcnt is a 4-bit count");
    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(v) : "n"(N) : "memory");
}
template <int N, typename T>
__device__ __forceinline__ void lgkm_wait2(T& a, T& b) {
    static_assert(N >= 0 && N <= 15, "lgkmcnt is a 4-bit count");
    asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "n"(N) : "memory");
}
__device__ __forceinline__ void vm_wait(int n) {
    // n is one of the counts the copy schedule produces
    if (n >= 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else if (n >= 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else if (n >= 2) asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}
// A 16-byte global load the compiler's wait-count pass does not track; the
// caller waits for it with an explicit vmcnt.
__device__ __forceinline__ u32x4_t global_b128_untracked(const void* p) {
    u32x4_t v;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p) : "memory");
    return v;
}
// The value is redefined here: its uses stay after this point.
__device__ __forceinline__ void reg_fence(u32x4_t& v) { asm volatile("" : "+v"(v)); }
// Barrier of the workgroup without the fence __syncthreads() adds (whose wait
// would drain every copy in flight).  The empty asm keeps the compiler from
// moving copies or LDS reads across it, the sched_barriers keep the
// scheduler from moving any other instruction across it: a phase's vector
// work must stay in its phase.
__device__ __forceinline__ void bare_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// Lanes l and l ^ 32 exchange v: v_permlane32_swap swaps the upper 32 lanes
// of its first operand with the lower 32 lanes of its second, so with both
// holding v, a = {v[0..31], v[0..31]} and b = {v[32..63], v[32..63]}.  As asm
// because the builtin's second result came back as a copy of the first.
// s_nop 1: the VALU writes of the operands must be two wait states old.
__device__ __forceinline__ void pair_swap(float v, float& a, float& b) {
    a = v;
    b = v;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ float pair_max(float v) {
    float a, b;
    pair_swap(v, a, b);
    return fmaxf(a, b);
}
__device__ __forceinline__ float pair_sum(float v) {
    float a, b;
    pair_swap(v, a, b);
    return a + b;
}

template <int D, bool CAUSAL>
__device__ __forceinline__ void flash_bf16_body(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
    const uint16_t* __restrict__ V, uint16_t* __restrict__ O, float* __restrict__ lse, int BH, int S,
    float c_log2) {
    using C = Bf16Cfg<D>;
    constexpr int BKV = C::BKV;
    constexpr float kLazy = 8.0f;
    constexpr int LA = 5;                       // MFMAs whose LDS reads are in flight (at most 15 reads)
    constexpr int KR = LA + 2, VR = LA + 2;     // K / V fragment ring sizes
    constexpr int PIECES = 2 * C::SEGW;         // copy instructions per wave per tile
    __shared__ __attribute__((aligned(1024))) uint8_t sm[C::NSTAGE * C::STAGE];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave >> 2;  // 0: group A, 1: group B
    const int g = lane >> 5, col = lane & 31;
    const int nq = (S + BQ2 - 1) / BQ2;
    int bh, q0;
    block_coords(BH, nq, BQ2, &bh, &q0);
    const int64_t hoff = (int64_t)bh * S * D;
    const uint16_t* Qh = Q + hoff;
    const uint16_t* Kh = K + hoff;
    const uint16_t* Vh = V + hoff;

    // this lane's query row and its Q fragments (B operand of S^T = K Q^T).
    // Loaded by asm so the compiler does not track them: it cannot count the
    // copies issued after them (it loses track across the asm waits) and would
    // drain every copy (vmcnt(0)) before the first use.  They are issued
    // before the first copy, so the wait for tile 0 covers them.
    const int qw0 = q0 + wave * 32;
    const int qrow = qw0 + col;
    u32x4_t qv[C::KS];
    bf16x8_t qf[C::KS];  // set once Q has landed
    {
        const int qr = min(qrow, S - 1);  // rows past S compute on a valid row, never stored
#pragma unroll
        for (int ks = 0; ks < C::KS; ++ks)
            qv[ks] = global_b128_untracked(Qh + (int64_t)qr * D + ks * 16 + 8 * g);
    }

    const int kv_end = CAUSAL ? min(S, q0 + BQ2) : S;
    const int n_kv = (kv_end + BKV - 1) / BKV;  // >= 1

    // ---- copy piece p of tile t: p < SEGW a K segment, else a V segment;
    // wave w moves segments w, w+8, ... of each operand tile ----
    const uint32_t sm0 = (uint32_t)(uintptr_t)sm;
    auto dma_part = [&](int t, int p0, int p1) {
#pragma unroll
        for (int p = 0; p < PIECES; ++p) {
            if (p < p0 || p >= p1) continue;
            const int i = p % C::SEGW;
            const int seg = i * NW2 + wave;
            const int r = seg * C::RPS + lane / C::UNITS;  // row within the tile
            const int up = lane % C::UNITS;                // physical 16-byte unit
            const int64_t key = min(t * BKV + r, S - 1);   // rows past S read a valid row
            uint8_t* dst = sm + (t % C::NSTAGE) * C::STAGE + seg * 1024;
            if (p < C::SEGW)
                __builtin_amdgcn_global_load_lds(Kh + key * D + 8 * (up ^ kswz<D>(r)),
                                                 (lds_void*)dst, 16, 0, 0);
            else
                __builtin_amdgcn_global_load_lds(Vh + key * D + 8 * (up ^ (vswz<D>(r) >> 1)),
                                                 (lds_void*)(dst + C::TILE), 16, 0, 0);
        }
    };
    auto dma_tile = [&](int t) { dma_part(t, 0, PIECES); };

    // ---- per-lane LDS offsets within a stage (recomputed per phase, which
    // costs a few VALU ops in the MFMA phase but no registers across phases) ----
    // K read for S MFMA i = (ks, half): key row half*32 + col, 16-byte unit 2 ks + g
    auto k_off = [&](int ks) -> uint32_t {
        return col * C::ROW + (((2 * ks + g) ^ kswz<D>(col)) << 4);
    };
    // V reads for PV MFMA (kk, dt): rows 16 kk + 4 g + s/4 (+8), chunk 8 dt + 4 vdh + s%4;
    // the swizzle only depends on s/4, so (kk, half) is a constant row offset
    auto v_off = [&](int dt) -> uint32_t {
        const int vs = lane & 15, vdh = (lane >> 4) & 1;
        const int r0 = 4 * g + (vs >> 2);
        return C::TILE + r0 * C::ROW + (((8 * dt + 4 * vdh + (vs & 3)) ^ vswz<D>(r0)) << 3);
    };

    f32x16_t acc_o[C::DT];
#pragma unroll
    for (int i = 0; i < C::DT; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc_o[i][e] = 0.0f;
    f32x16_t sc[2];         // S_j: keys [32 h + 8 (e/4) + 4 g + e%4] of this lane's query
    bf16x8_t pf[4];         // P_{j}: B operand of the PV product, 16-key step kk
    float m_run = kNegInf;  // running max of scaled scores, log2 domain
    float l_run = 0.0f;     // this lane's partial running sum (its 32 keys per tile)

    // ---- MFMA(j): S_j (j < n_kv) and PV_{j-1} (j >= 1) ----
    // The MFMA sequence alternates S and PV products when both are present:
    // six independent accumulators in rotation, so no MFMA waits on the
    // result of the one before it.  The LDS reads follow the same order (one
    // K read per S MFMA, two V reads per PV MFMA) and are issued LA MFMAs
    // ahead of their consumer.
    auto mfma_phase = [&](int j, auto do_s_tag, auto do_pv_tag) {
        constexpr bool DO_S = decltype(do_s_tag)::value;
        constexpr bool DO_PV = decltype(do_pv_tag)::value;
        // the MFMA wave's issue goes first when both waves of a SIMD are ready
        __builtin_amdgcn_s_setprio(1);
        using Q_ = MfmaSeq<DO_S, DO_PV, C::NS, C::NPV>;
        constexpr int NM = Q_::NM;
        constexpr int TOT = Q_::reads_upto(NM - 1);
        const uint32_t kbase = sm0 + (j % C::NSTAGE) * C::STAGE;
        const uint32_t vbase = sm0 + ((j + C::NSTAGE - 1) % C::NSTAGE) * C::STAGE;
        uint32_t ka[C::KS], va[C::DT];
#pragma unroll
        for (int ks = 0; ks < C::KS; ++ks) ka[ks] = kbase + k_off(ks);
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) va[dt] = vbase + v_off(dt);
        u32x4_t kf[KR];
        u32x2_t vlo[VR], vhi[VR];
        // read r of the stream, r in MFMA order
        auto issue_read = [&](auto rc) {
            constexpr int r = decltype(rc)::value;
            if constexpr (r < TOT) {
                // the MFMA m this read belongs to, and which of its reads it is
                constexpr int m = Q_::owner(r);
                constexpr int first = m == 0 ? 0 : Q_::reads_upto(m - 1);
                constexpr int i = Q_::idx(m);
                if constexpr (Q_::is_s(m)) {
                    constexpr int ks = i / 2, half = i % 2;
                    kf[i % KR] = lds_b128<half * 32 * C::ROW>(ka[ks]);
                } else {
                    constexpr int kk = i / C::DT, dt = i % C::DT;
                    if constexpr (r == first) vlo[i % VR] = lds_tr16<16 * kk * C::ROW>(va[dt]);
                    else vhi[i % VR] = lds_tr16<(16 * kk + 8) * C::ROW>(va[dt]);
                }
            }
        };
        constexpr int R0 = Q_::reads_upto(LA - 1 < NM - 1 ? LA - 1 : NM - 1);
        static_for<0, R0>(issue_read);
        static_for<0, NM>([&](auto mc) {
            constexpr int m = decltype(mc)::value;
            constexpr int i = Q_::idx(m);
            constexpr int issued = Q_::reads_upto(m + LA - 1 < NM - 1 ? m + LA - 1 : NM - 1);
            constexpr int need = Q_::reads_upto(m);
            if constexpr (Q_::is_s(m)) {
                lgkm_wait<issued - need>(kf[i % KR]);
                // the first k-step starts from zero (an inline constant operand)
                const f32x16_t zero = {};
                sc[i % 2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    __builtin_bit_cast(bf16x8_t, kf[i % KR]), qf[i / 2], i < 2 ? zero : sc[i % 2],
                    0, 0, 0);
            } else {
                constexpr int kk = i / C::DT, dt = i % C::DT;
                lgkm_wait2<issued - need>(vlo[i % VR], vhi[i % VR]);
                const u32x2_t lo = vlo[i % VR], hi = vhi[i % VR];
                const u32x4_t v4 = {lo[0], lo[1], hi[0], hi[1]};
                acc_o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    __builtin_bit_cast(bf16x8_t, v4), pf[kk], acc_o[dt], 0, 0, 0);
            }
            // keep LA MFMAs' reads in flight
            constexpr int nxt = Q_::reads_upto(m + LA < NM - 1 ? m + LA : NM - 1);
            static_for<issued, nxt>(issue_read);
        });
        __builtin_amdgcn_s_setprio(0);
    };

    // ---- SOFTMAX(j) ----
    auto softmax_phase = [&](int j) {
        const int k0 = j * BKV;
        if (k0 + BKV > S || (CAUSAL && k0 + BKV - 1 > qw0)) {
            // keys past S and (causal) keys after this lane's query -> -inf.
            // Element (h, e) holds key k0 + 4g + off with off = 32h + 8(e/4) +
            // e%4 a constant, so one compare against a per-lane limit masks it.
            int lim = S - 1 - k0 - 4 * g;
            if (CAUSAL) lim = min(lim, qrow - k0 - 4 * g);
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    if (h * 32 + 8 * (e >> 2) + (e & 3) > lim) sc[h][e] = kNegInf;
        }
        float mx = kNegInf;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < 16; ++e) mx = fmaxf(mx, sc[h][e]);
        mx = pair_max(mx) * c_log2;
        const bool grow = mx > m_run + kLazy;
        if (__builtin_amdgcn_ballot_w64(grow)) {
            const float alpha = grow ? __builtin_amdgcn_exp2f(m_run - mx) : 1.0f;  // 0 on the first tile
            m_run = grow ? mx : m_run;
            l_run *= alpha;
#pragma unroll
            for (int i = 0; i < C::DT; ++i) acc_o[i] *= alpha;
        }
        const float m_use = (m_run == kNegInf) ? 0.0f : m_run;  // row with no visible key yet
        float ls[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[h][e], c_log2, -m_use));
                sc[h][e] = p;
                ls[e & 3] += p;
            }
        l_run += (ls[0] + ls[1]) + (ls[2] + ls[3]);
        asm volatile("" : "+v"(l_run));  // computed in this phase, not sunk into the next
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            u32x4_t u;
#pragma unroll
            for (int w = 0; w < 4; ++w)
                u[w] = pack_bf16x2(sc[kk >> 1][8 * (kk & 1) + 2 * w], sc[kk >> 1][8 * (kk & 1) + 2 * w + 1]);
            reg_fence(u);
            pf[kk] = __builtin_bit_cast(bf16x8_t, u);
        }
    };

    // ---- prologue: Q, tiles 0 and 1 in flight; wait for Q and tile 0 ----
    dma_tile(0);
    // tile 1 is copied even when there is no tile 1 (its rows clamp to S-1 and
    // land in a stage nothing reads), so the wait count is one constant on
    // every path: the static ISA check cannot correlate two branches on n_kv
    dma_tile(1);
    vm_wait(PIECES);
    bare_barrier();
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) {
        reg_fence(qv[ks]);  // after the wait above
        qf[ks] = __builtin_bit_cast(bf16x8_t, qv[ks]);
    }

    using yes = std::integral_constant<bool, true>;
    using no = std::integral_constant<bool, false>;
    // Phases 0 .. 2 n_kv + 1, each closed by a barrier of all 8 waves.
    // Tile u+2 is copied into the stage tile u-2 left (last read in phase
    // 2u-1): its K half in phase 2u, its V half in phase 2u+1, which spreads
    // the copies' LDS writes over both phases.  Before phase 2u, tile u must
    // have landed: the copies issued after it are those of tile u+1.
    auto copy_k = [&](int u) {
        if (u + 2 < n_kv) dma_part(u + 2, 0, C::SEGW);
    };
    auto copy_v = [&](int u) {
        if (u + 2 < n_kv) dma_part(u + 2, C::SEGW, PIECES);
    };
    auto land = [&](int u) {
        if (u < n_kv) vm_wait(u + 1 < n_kv ? PIECES : 0);
    };
    // Causal: key tile t is needed by this wave only if its first key is at
    // or before the wave's last query.  A wave skips the softmax and the S
    // products of tiles it does not need (every wave still copies and meets
    // every barrier).  MFMA(j) also carries PV_{j-1}, so it runs while tile
    // j-1 is needed; for the first unneeded tile j its S_j is computed and
    // left unused, which keeps a single MFMA-phase shape in the loop.
    auto need = [&](int t) { return !CAUSAL || t * BKV <= qw0 + 31; };
    // D = 128: the barrier between phases 2j and 2j+1 is left out, so each
    // group runs its MFMA and softmax phases of a key tile back to back and
    // the groups meet once per tile.  They stay in opposite phases (A starts
    // a tile with its MFMAs, B with its softmax), and a group whose phase ends
    // early goes straight on instead of idling until the other's ends.  The
    // stage and landing rules above still hold: a stage is refilled only after
    // the barrier that closes the step in which it was last read, and tile
    // j+1 lands before the barrier that closes step j.  Measured at
    // [8,32,4096,128]: causal 1.068 -> 1.052 ms, non-causal 1.892 -> 1.882
    // ms.  At D = 64 the softmax phase is the longer one, and without the
    // middle barrier the two groups' softmax phases overlap on a SIMD (1.42
    // -> 1.44 ms at [8,64,4096,64] causal), so D = 64 keeps it.
    constexpr bool MID = D == 64;
    if (grp == 0) {
        copy_k(0);
        mfma_phase(0, yes{}, no{});
        bare_barrier();  // phase 0
        copy_v(0);
        softmax_phase(0);
        land(1);
        bare_barrier();  // phase 1
        for (int j = 1; j < n_kv; ++j) {
            copy_k(j);
            if (need(j - 1)) mfma_phase(j, yes{}, yes{});
            if constexpr (MID) bare_barrier();  // phase 2j
            copy_v(j);
            if (need(j)) softmax_phase(j);
            land(j + 1);
            bare_barrier();  // phase 2j+1
        }
        if (need(n_kv - 1)) mfma_phase(n_kv, no{}, yes{});
        bare_barrier();  // phase 2 n_kv
        bare_barrier();  // phase 2 n_kv + 1
    } else {
        copy_k(0);
        bare_barrier();  // phase 0
        copy_v(0);
        mfma_phase(0, yes{}, no{});
        land(1);
        bare_barrier();  // phase 1
        for (int j = 1; j < n_kv; ++j) {
            copy_k(j);
            if (need(j - 1)) softmax_phase(j - 1);
            if constexpr (MID) bare_barrier();  // phase 2j
            copy_v(j);
            if (need(j - 1)) mfma_phase(j, yes{}, yes{});
            land(j + 1);
            bare_barrier();  // phase 2j+1
        }
        if (need(n_kv - 1)) softmax_phase(n_kv - 1);
        bare_barrier();  // phase 2 n_kv
        if (need(n_kv - 1)) mfma_phase(n_kv, no{}, yes{});
        bare_barrier();  // phase 2 n_kv + 1
    }

    // ---- epilogue: O = acc / l, bf16; lse = (m + log2 l) * ln 2 ----
    const float l_tot = pair_sum(l_run);
    const float inv = (l_tot > 0.0f) ? 1.0f / l_tot : 0.0f;
    // The rows go out through LDS, which every wave has finished with at the
    // last barrier: each wave writes its 32 rows of O to its own 32 x D
    // region (16-byte unit u of row r at u ^ (r % U), so the 32 rows a write
    // serves spread over the banks), then reads them back a row-contiguous
    // 16 bytes per lane, so one store instruction writes 64 / U whole rows
    // instead of 16 bytes of each of 32 rows.
    constexpr int U = D / 8;                    // 16-byte units per row
    constexpr int RPI = 64 / U;                 // rows per store instruction
    uint8_t* stg = sm + wave * 32 * D * 2;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            u32x2_t w;
            w[0] = pack_bf16x2(acc_o[dt][4 * jb + 0] * inv, acc_o[dt][4 * jb + 1] * inv);
            w[1] = pack_bf16x2(acc_o[dt][4 * jb + 2] * inv, acc_o[dt][4 * jb + 3] * inv);
            const int u = 4 * dt + jb;          // columns 8u .. 8u+7 of the row; lane g holds half g
            *reinterpret_cast<u32x2_t*>(stg + col * (D * 2) + ((u ^ (col & (U - 1))) << 4) + 8 * g) = w;
        }
    if (lse && g == 0 && qrow < S)
        lse[(int64_t)bh * S + qrow] = (m_run + __builtin_amdgcn_logf(l_tot)) * 0.6931471805599453f;
#pragma unroll
    for (int s = 0; s < U / 2; ++s) {
        const int r = s * RPI + lane / U, u = lane % U;
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(stg + r * (D * 2) + ((u ^ (r & (U - 1))) << 4));
        if (qw0 + r < S) *reinterpret_cast<u32x4_t*>(O + hoff + (int64_t)(qw0 + r) * D + 8 * u) = v;
    }
}

// The body lives in a device function: with it inline in the kernel template,
// clang's host pass silently skipped the kernel's launch stub.
template <int D, bool CAUSAL>
__global__ __launch_bounds__(512, 1) void flash_fwd_bf16(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
    const uint16_t* __restrict__ V, uint16_t* __restrict__ O, float* __restrict__ lse, int BH, int S,
    float c_log2) {
    flash_bf16_body<D, CAUSAL>(Q, K, V, O, lse, BH, S, c_log2);
}

// ---------------------------------------------------------------------------
// fp32: same recurrence on v_mfma_f32_32x32x2_f32.  The 32x32x2 A/B operands
// are one fp32 per lane (row/col = lane & 31, k = lane >> 5), so K and V are
// read from LDS as [key][d] rows without any transpose: for the PV product
// k-step (j, i) pairs keys 8j+i (lanes 0-31) and 8j+4+i (lanes 32-63), which
// are exactly the score accumulator element 4j+i each lane already holds.
//
// Work split: a workgroup owns 32 queries, and its 4 waves split the key
// range (wave w takes key tiles w, w+4, ...), each with its own running
// max, sum and accumulator; at the end the four partial states are merged
// in LDS in a fixed order.  With causal masking the query groups near the
// diagonal carry the longest key ranges; splitting the range bounds the
// longest chain a single wave runs to a quarter of it.  Each wave stages its
// own K/V tiles through a private LDS region (register prefetch of the next
// tile while the current one is computed), so the main loop needs no
// workgroup barrier.
// ---------------------------------------------------------------------------
constexpr int BQF = 32;  // query rows per fp32 workgroup
constexpr int NWF = 4;   // waves per fp32 workgroup (key-range split)

template <int D>
struct F32Cfg {
    static constexpr int BKV = 32;
    static constexpr int ROWF = D + 4;                 // padded row (floats): rows shift by 16 B
    static constexpr int K_FLOATS = BKV * ROWF;
    static constexpr int WAVE_FLOATS = 2 * K_FLOATS;   // one wave's K then V tile
    static constexpr int PT = BKV * D / 4 / 64;        // 16-byte chunks per lane per operand
};

template <int D, bool CAUSAL>
__device__ __forceinline__ void flash_f32_body(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    float* __restrict__ O, float* __restrict__ lse, int BH, int S, float c_log2) {
    using C = F32Cfg<D>;
    constexpr int BKV = C::BKV;
    // K/V stages during the loop; the merge reuses the same memory
    constexpr int MERGE_FLOATS = NWF * (BQF * D + 2 * BQF);
    constexpr int SMEM_FLOATS = NWF * C::WAVE_FLOATS > MERGE_FLOATS ? NWF * C::WAVE_FLOATS
                                                                       : MERGE_FLOATS;
    __shared__ __attribute__((aligned(16))) float smem[SMEM_FLOATS];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 5, col = lane & 31;
    const int nq = (S + BQF - 1) / BQF;
    int bh, q0;
    block_coords(BH, nq, BQF, &bh, &q0);
    const int64_t hoff = (int64_t)bh * S * D;
    const float* Qh = Q + hoff;
    const float* Kh = K + hoff;
    const float* Vh = V + hoff;
    const int qrow = q0 + col;

    float qf[D / 2];  // Q[qrow][2 ks + g]
#pragma unroll
    for (int ks = 0; ks < D / 2; ++ks) qf[ks] = (qrow < S) ? Qh[(int64_t)qrow * D + 2 * ks + g] : 0.0f;

    const int kv_end = CAUSAL ? min(S, q0 + BQF) : S;
    const int n_kv = (kv_end + BKV - 1) / BKV;

    float* Ks = smem + wave * C::WAVE_FLOATS;  // this wave's tile
    float* Vs = Ks + C::K_FLOATS;
    f32x4_t rk[C::PT], rv[C::PT];
    // rows past S read row S-1 (branch-free loads): their scores are masked
    // to -inf, so their p is 0 and the values never reach the output
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < C::PT; ++i) {
            const int c = lane + 64 * i;
            const int key = c / (D / 4), ch = c % (D / 4);
            const int64_t row = min(k0 + key, S - 1);
            rk[i] = *reinterpret_cast<const f32x4_t*>(Kh + row * D + 4 * ch);
            rv[i] = *reinterpret_cast<const f32x4_t*>(Vh + row * D + 4 * ch);
        }
    };
    // the wave's LDS reads of the previous tile are issued before these
    // writes and LDS operations of one wave execute in order
    auto lstore = [&]() {
#pragma unroll
        for (int i = 0; i < C::PT; ++i) {
            const int c = lane + 64 * i;
            const int key = c / (D / 4), ch = c % (D / 4);
            *reinterpret_cast<f32x4_t*>(Ks + key * C::ROWF + 4 * ch) = rk[i];
            *reinterpret_cast<f32x4_t*>(Vs + key * C::ROWF + 4 * ch) = rv[i];
        }
    };

    f32x16_t acc_o[D / 32];
#pragma unroll
    for (int i = 0; i < D / 32; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc_o[i][e] = 0.0f;
    float m_run = kNegInf, l_run = 0.0f;

    auto compute = [&](int k0) {
        // two independent accumulation chains (even / odd k-steps), summed
        f32x16_t s, s1;
#pragma unroll
        for (int e = 0; e < 16; ++e) s[e] = s1[e] = 0.0f;
#pragma unroll
        for (int ks = 0; ks < D / 2; ks += 2) {
            s = __builtin_amdgcn_mfma_f32_32x32x2f32(Ks[col * C::ROWF + 2 * ks + g], qf[ks], s, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_32x32x2f32(Ks[col * C::ROWF + 2 * ks + 2 + g], qf[ks + 1],
                                                      s1, 0, 0, 0);
        }
        s += s1;
        const bool need_mask = (k0 + BKV > S) || (CAUSAL && k0 + BKV - 1 > q0);
        if (need_mask) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int key = k0 + 8 * (e >> 2) + 4 * g + (e & 3);
                if (key >= S || (CAUSAL && key > qrow)) s[e] = kNegInf;
            }
        }
        float mx = kNegInf;
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[e]);
        mx = fmaxf(mx, xor32(mx));
        const float m_new = fmaxf(m_run, mx * c_log2);
        const float m_use = (m_new == kNegInf) ? 0.0f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
        m_run = m_new;
        float ls = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[e], c_log2, -m_use));
            s[e] = p;
            ls += p;
        }
        l_run = __builtin_fmaf(l_run, alpha, ls);
#pragma unroll
        for (int i = 0; i < D / 32; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc_o[i][e] *= alpha;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = 8 * j + 4 * g + i;
#pragma unroll
                for (int dt = 0; dt < D / 32; ++dt)
                    acc_o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(Vs[key * C::ROWF + dt * 32 + col],
                                                                     s[4 * j + i], acc_o[dt], 0, 0, 0);
            }
    };

    // this wave's key tiles: wave, wave + 4, ...
    if (wave < n_kv) {
        gload(wave * BKV);
        lstore();
        for (int j = wave; j < n_kv; j += NWF) {
            const bool more = j + NWF < n_kv;
            if (more) gload((j + NWF) * BKV);
            compute(j * BKV);
            if (more) lstore();
        }
    }

    // ---- merge the four partial states: M = max m_w, O = sum acc_w 2^(m_w - M),
    // L = sum l_w 2^(m_w - M), in wave order ----
    __syncthreads();  // every wave is done with its K/V tile
    float* macc = smem + wave * (BQF * D + 2 * BQF);  // [q][d] accumulator, then m[q], l[q]
    const float l_pair = l_run + xor32(l_run);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int d = dt * 32 + 8 * (e >> 2) + 4 * g + (e & 3);
            macc[col * D + d] = acc_o[dt][e];
        }
    if (g == 0) {
        macc[BQF * D + col] = m_run;
        macc[BQF * D + BQF + col] = l_pair;
    }
    __syncthreads();
    // every wave merges D/4 of the d columns of all 32 queries: lane -> (q, 8 d)
    const int q = lane >> 1;
    const int dbase = wave * (D / 4) + (lane & 1) * (D / 8);
    float mw[NWF], mm = kNegInf;
#pragma unroll
    for (int w = 0; w < NWF; ++w) {
        mw[w] = smem[w * (BQF * D + 2 * BQF) + BQF * D + q];
        mm = fmaxf(mm, mw[w]);
    }
    const float m_ref = (mm == kNegInf) ? 0.0f : mm;
    float sc[NWF], L = 0.0f;
#pragma unroll
    for (int w = 0; w < NWF; ++w) {
        sc[w] = (mw[w] == kNegInf) ? 0.0f : __builtin_amdgcn_exp2f(mw[w] - m_ref);
        L += smem[w * (BQF * D + 2 * BQF) + BQF * D + BQF + q] * sc[w];
    }
    const float inv = (L > 0.0f) ? 1.0f / L : 0.0f;
    const int orow = q0 + q;
    if (orow < S) {
        float* Orow = O + hoff + (int64_t)orow * D;
#pragma unroll
        for (int c4 = 0; c4 < D / 32; ++c4) {
            f32x4_t v;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = dbase + 4 * c4 + i;
                float o = 0.0f;
#pragma unroll
                for (int w = 0; w < NWF; ++w) o += smem[w * (BQF * D + 2 * BQF) + q * D + d] * sc[w];
                v[i] = o * inv;
            }
            *reinterpret_cast<f32x4_t*>(Orow + dbase + 4 * c4) = v;
        }
        if (lse && wave == 0 && (lane & 1) == 0)
            lse[(int64_t)bh * S + orow] = (mm + __builtin_amdgcn_logf(L)) * 0.6931471805599453f;
    }
}

template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, D == 64 ? 2 : 1) void flash_fwd_f32(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    float* __restrict__ O, float* __restrict__ lse, int BH, int S, float c_log2) {
    flash_f32_body<D, CAUSAL>(Q, K, V, O, lse, BH, S, c_log2);
}

template <typename KFN, typename T>
hipError_t go(KFN kfn, const void* Q, const void* K, const void* V, void* O, float* lse, int BH,
              int S, float c_log2, hipStream_t s) {
    // bf16: 256-row blocks of 8 waves; fp32: 32-row blocks of 4 waves
    constexpr bool BF = sizeof(T) == 2;
    const int bq = BF ? BQ2 : BQF;
    const int nq = (S + bq - 1) / bq;
    hipLaunchKernelGGL(kfn, dim3(BH * nq), dim3((BF ? NW2 : NWF) * 64), 0, s, static_cast<const T*>(Q),
                       static_cast<const T*>(K), static_cast<const T*>(V), static_cast<T*>(O), lse,
                       BH, S, c_log2);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_flash_fwd(int dtype, int causal, float scale, const void* Q, const void* K,
                            const void* V, void* O, float* lse, int B, int H, int S, int D,
                            hipStream_t s) {
    const int BH = B * H;
    if ((int64_t)BH * ((S + BQF - 1) / BQF) > 2147483647) return hipErrorInvalidValue;
    const float c = scale * kLog2e;
    if (dtype == JH_BF16) {
        if (D == 128)
            return causal ? go<decltype(&flash_fwd_bf16<128, true>), uint16_t>(&flash_fwd_bf16<128, true>, Q, K, V, O, lse, BH, S, c, s)
                          : go<decltype(&flash_fwd_bf16<128, false>), uint16_t>(&flash_fwd_bf16<128, false>, Q, K, V, O, lse, BH, S, c, s);
        return causal ? go<decltype(&flash_fwd_bf16<64, true>), uint16_t>(&flash_fwd_bf16<64, true>, Q, K, V, O, lse, BH, S, c, s)
                      : go<decltype(&flash_fwd_bf16<64, false>), uint16_t>(&flash_fwd_bf16<64, false>, Q, K, V, O, lse, BH, S, c, s);
    }
    if (D == 128)
        return causal ? go<decltype(&flash_fwd_f32<128, true>), float>(&flash_fwd_f32<128, true>, Q, K, V, O, lse, BH, S, c, s)
                      : go<decltype(&flash_fwd_f32<128, false>), float>(&flash_fwd_f32<128, false>, Q, K, V, O, lse, BH, S, c, s);
    return causal ? go<decltype(&flash_fwd_f32<64, true>), float>(&flash_fwd_f32<64, true>, Q, K, V, O, lse, BH, S, c, s)
                  : go<decltype(&flash_fwd_f32<64, false>), float>(&flash_fwd_f32<64, false>, Q, K, V, O, lse, BH, S, c, s);
}

}  // namespace jh
