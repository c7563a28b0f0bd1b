// flash_bwd_dq.hip - the dQ pass of the flash-attention backward as an
// 8-wave ping-pong (gfx950 MFMA, bf16), the forward kernel's schedule.
//
//   dQ = scale * dS K,  dS = P * (dP - dvec),  P = exp(scale * Q K^T - lse),
//   dP = dO V^T   (masked entries 0), per (batch, head); Q, K, V, dO, dQ
//   [B,H,S,D] bf16 row-major, D in {64, 128}; lse, dvec [B,H,S] fp32.
//
// Workgroup: 8 waves x 32 queries = 256 query rows.  Per wave the scores are
// computed transposed, as in the forward: S^T = K Q^T and dP^T = V dO^T for a
// unit of 32 keys (lane = query, 16 keys per lane), then dQ^T += K^T dS^T
// with dS^T packed from the accumulator registers as the B operand and K^T
// read from LDS with ds_read_b64_tr_b16.  The waves form two groups, A = waves
// 0-3 and B = waves 4-7, one of each per SIMD, half a unit out of phase: one
// group issues the MFMAs of a unit (S^T_u, dP^T_u and the dQ^T product of
// unit u-1: 24 MFMAs at D = 128) while the other turns its S^T, dP^T into
// dS^T on the vector ALU.  Step u is closed by one barrier of all 8 waves:
//   group A: MFMA(u), then VALU(u);
//   group B: VALU(u-1), then MFMA(u).
// The groups meet only at the barrier, so a group whose first half ends
// early goes on with its second instead of waiting for the other group (a
// barrier between the halves measured 2-3% slower over the whole backward).
// A lane's lse and dvec are per-query scalars, so there is no running
// statistic to carry between units.
//
// K and V tiles of 64 keys (two units) go HBM -> LDS by LDS DMA through a ring
// of 4 stages; tile t in stage t % 4.  The K half of tile t+2 is copied at
// the start of step 2t, its V half at the start of step 2t+1, and tile t+1
// has landed (each wave waits for its own copies, then the barrier) at the
// end of step 2t+1, before its first use in step 2t+2.  Tile t-2, which
// stage (t+2) % 4 held, was last read in step 2t-2 (MFMA(2t-2) reads K^T of
// unit 2t-3 for its dQ^T product).
// Both tiles are row-major [key][d], 16-byte unit u of row r at u ^ sw(r).
// V is read by rows (ds_read_b128: 8 d of one key per lane, 16 rows per
// clock); K by rows too and, for dQ, transposed (ds_read_b64_tr_b16: a
// 16-lane group reads 4 rows x 16 d, two groups 4 rows x 64 bytes per clock).
// sw serves both without bank conflicts:
//   D = 128 (16 units per row): sw(r) = (r & 15) ^ ((r & 3) << 2): a bijection
//     on 16 consecutive rows, and rows 4a .. 4a+3 get distinct bits 2-3, so
//     their 64-byte windows differ;
//   D = 64 (8 units, two rows per 256-byte bank window): m = (r >> 1) & 7,
//     sw(r) = m ^ ((m & 1) << 2): a bijection on m, and rows 4a, 4a+2 (and
//     4a+1, 4a+3, which share a half-window) differ in bit 2.
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"

namespace jh {
namespace {

typedef __attribute__((address_space(3))) void lds_void_dq;

constexpr int DQ_W = 8;         // waves per workgroup
constexpr int DQ_BQ = DQ_W * 32;  // queries per workgroup
constexpr int DQ_BKV = 64;      // keys per LDS tile (two 32-key units)
constexpr float kLog2eDq = 1.4426950408889634f;

template <int D>
struct DqCfg {
    static constexpr int ROW = D * 2;           // bytes per K / V row
    static constexpr int TILE = DQ_BKV * ROW;   // one operand tile
    static constexpr int STAGE = 2 * TILE;      // K then V
    static constexpr int NSTAGE = 4;
    static constexpr int UNITS = ROW / 16;      // 16-byte units per row
    static constexpr int NSEG = TILE / 1024;    // 1 KiB DMA segments per operand tile
    static constexpr int SEGW = NSEG / DQ_W;    // copy instructions per wave per operand tile
    static constexpr int RPS = 1024 / ROW;      // rows per segment
    static constexpr int KS = D / 16;           // k-steps of S^T (and dP^T)
    static constexpr int DT = D / 32;           // 32-row d blocks of dQ^T
    static constexpr int NQ = 2 * DT;           // dQ MFMAs per unit (= KS)
};

template <int D>
__host__ __device__ constexpr int dq_sw(int r) {
    if constexpr (D == 128) {
        return (r & 15) ^ ((r & 3) << 2);
    } else {
        const int m = (r >> 1) & 7;
        return m ^ ((m & 1) << 2);
    }
}

template <int I, int N, typename F>
__device__ __forceinline__ void sfor(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        sfor<I + 1, N>(f);
    }
}

template <int OFF>
__device__ __forceinline__ u32x4_t dq_b128(uint32_t addr) {
    u32x4_t v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF) : "memory");
    return v;
}
template <int OFF>
__device__ __forceinline__ u32x2_t dq_tr16(uint32_t addr) {
    u32x2_t v;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF) : "memory");
    return v;
}
template <int N>
__device__ __forceinline__ void dq_lgkm(u32x4_t& v) {
    static_assert(N >= 0 && N <= 15, "lgkmcnt is a 4-bit count");
    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(v) : "n"(N) : "memory");
}
__device__ __forceinline__ void dq_vm(int n) {
    // n is one of the counts the copy schedule produces
    if (n >= 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else if (n >= 2) asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}
__device__ __forceinline__ u32x4_t dq_load_untracked(const void* p) {
    u32x4_t v;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p) : "memory");
    return v;
}
__device__ __forceinline__ float dq_load_f32_untracked(const float* p) {
    float v;
    asm volatile("global_load_dword %0, %1, off" : "=v"(v) : "v"(p) : "memory");
    return v;
}
__device__ __forceinline__ void dq_fence(u32x4_t& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void dq_fence(float& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void dq_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}
__device__ __forceinline__ bf16x8_t dq_pack8(const float* f) {
    u32x4_t u;
    u[0] = pack_bf16x2(f[0], f[1]);
    u[1] = pack_bf16x2(f[2], f[3]);
    u[2] = pack_bf16x2(f[4], f[5]);
    u[3] = pack_bf16x2(f[6], f[7]);
    return __builtin_bit_cast(bf16x8_t, u);
}

// MFMA order of one MFMA phase: for i = 0 .. KS-1, S_i and dP_i (if SP) then
// Q_i, the dQ product (dt = i / 2, 16-key step kk = i % 2; if Q).  S and dP
// take one row read each, Q two transposing reads.
template <bool SP, bool Q, int KS>
struct DqSeq {
    static constexpr int PER = (SP ? 2 : 0) + (Q ? 1 : 0);
    static constexpr int NM = PER * KS;
    // kind of MFMA m: 0 S, 1 dP, 2 Q
    static constexpr int kind(int m) { return SP ? (m % PER < 2 ? m % PER : 2) : 2; }
    static constexpr int idx(int m) { return m / PER; }
    static constexpr int nreads(int m) { return kind(m) == 2 ? 2 : 1; }
    static constexpr int reads_upto(int m) {  // reads of MFMAs 0 .. m
        int r = 0;
        for (int k = 0; k <= m && k < NM; ++k) r += nreads(k);
        return r;
    }
};

template <int D, bool CAUSAL>
__global__ __launch_bounds__(512, 1) void flash_bwd_dq_pp_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    const uint16_t* __restrict__ dO, const float* __restrict__ lse, const float* __restrict__ dvec,
    uint16_t* __restrict__ dQ, int BH, int S, float scale) {
    using C = DqCfg<D>;
    constexpr int LA = 4;           // MFMAs whose LDS reads are in flight
    constexpr int R = LA + 2;       // fragment ring
    constexpr int PIECES = 2 * C::SEGW;
    __shared__ __attribute__((aligned(1024))) uint8_t sm[C::NSTAGE * C::STAGE];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave >> 2;
    const int g = lane >> 5, col = lane & 31;

    // workgroup -> (head, query block): the forward's order (whole heads per
    // XCD, four interleaved, longest causal range first)
    const int nq = (S + DQ_BQ - 1) / DQ_BQ;
    int bh, qi;
    {
        const int b = blockIdx.x;
        if ((BH & 7) == 0) {
            const int xcd = b & 7, i = b >> 3;
            const int J = BH >> 3;
            const int gi = i / (4 * nq), r = i - gi * 4 * nq;
            const int gs = min(4, J - 4 * gi);
            bh = 8 * (4 * gi + r % gs) + xcd;
            qi = r / gs;
        } else {
            bh = b / nq;
            qi = b % nq;
        }
    }
    const int q0 = (nq - 1 - qi) * DQ_BQ;
    const int64_t hoff = (int64_t)bh * S * D;
    const uint16_t* Kh = K + hoff;
    const uint16_t* Vh = V + hoff;
    const float c = scale * kLog2eDq;

    // this lane's query and its Q, dO fragments (B operands), lse and dvec,
    // loaded untracked before the first copy (the wait for tile 0 covers them)
    const int qw0 = q0 + wave * 32;
    const int qrow = qw0 + col;
    const int qr = min(qrow, S - 1);
    u32x4_t qv[C::KS], ov[C::KS];
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) {
        qv[ks] = dq_load_untracked(Q + hoff + (int64_t)qr * D + 16 * ks + 8 * g);
        ov[ks] = dq_load_untracked(dO + hoff + (int64_t)qr * D + 16 * ks + 8 * g);
    }
    float lse_v = dq_load_f32_untracked(lse + (int64_t)bh * S + qr);
    float dv_v = dq_load_f32_untracked(dvec + (int64_t)bh * S + qr);

    const int kv_end = CAUSAL ? min(S, q0 + DQ_BQ) : S;
    const int n_t = (kv_end + DQ_BKV - 1) / DQ_BKV;  // >= 1
    const int U = 2 * n_t;                           // 32-key units

    // ---- copy piece p of tile t: p < SEGW a K segment, else a V segment;
    // wave w moves segments w, w+8, ... of each operand tile.  Buffer loads
    // over the tile's rows that exist: rows past S read 0 (their keys are
    // masked), and every offset stays small whatever S is ----
    const uint32_t sm0 = (uint32_t)(uintptr_t)sm;
    auto dma_part = [&](int t, int p0, int p1) {
        const int64_t tr0 = (int64_t)min(t * DQ_BKV, S);  // a tile past the end: an empty range at S
        const uint32_t bytes = (uint32_t)max(0, min(DQ_BKV, S - t * DQ_BKV)) * (uint32_t)C::ROW;
        const __amdgpu_buffer_rsrc_t ksrc = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(Kh + tr0 * D), 0, bytes, 0x00020000);
        const __amdgpu_buffer_rsrc_t vsrc = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(Vh + tr0 * D), 0, bytes, 0x00020000);
#pragma unroll
        for (int p = 0; p < PIECES; ++p) {
            if (p < p0 || p >= p1) continue;
            const int i = p % C::SEGW;
            const int seg = i * DQ_W + wave;
            const int r = seg * C::RPS + lane / C::UNITS;  // row within the tile
            const int up = lane % C::UNITS;                // physical 16-byte unit
            const uint32_t vo = (uint32_t)(r * C::ROW + ((up ^ dq_sw<D>(r)) << 4));
            uint8_t* dst = sm + (t % C::NSTAGE) * C::STAGE + seg * 1024;
            if (p < C::SEGW)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ksrc, (lds_void_dq*)dst, 16, vo, 0, 0, 0);
            else
                __builtin_amdgcn_raw_ptr_buffer_load_lds(vsrc, (lds_void_dq*)(dst + C::TILE), 16, vo, 0, 0, 0);
        }
    };

    // per-lane parts of the LDS read addresses (within a stage, unit half 0)
    // row reads of key row col, unit 2 i + g: col * ROW + 16 ((2 i + g) ^ sw)
    const int swr = dq_sw<D>(col);
    auto row_off = [&](int i, int z) -> uint32_t {
        return (uint32_t)((col + z) * C::ROW + (((2 * i + g) ^ (swr + z)) << 4));
    };
    // transposing reads of d block dt, rows 4 g + s / 4 (+ 8 for hi), 8-byte
    // chunk 8 dt + 4 vdh + s % 4 (s = lane % 16, vdh = lane / 16 % 2)
    const int vs = lane & 15, vdh = (lane >> 4) & 1;
    const int trow = 4 * g + (vs >> 2);
    auto tr_off = [&](int dt, int hi, int z) -> uint32_t {
        const int r = trow + z + 8 * hi;
        const int chunk = 8 * dt + 4 * vdh + (vs & 3);
        const int u = (chunk >> 1) ^ dq_sw<D>(r);
        return (uint32_t)(r * C::ROW + (u << 4) + 8 * (chunk & 1));
    };

    f32x16_t acc[C::DT];
#pragma unroll
    for (int i = 0; i < C::DT; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][e] = 0.0f;
    f32x16_t s, dp;    // S^T, dP^T of the current unit
    bf16x8_t sb[2];    // dS^T of the previous unit: B operands of its two 16-key steps
    bf16x8_t qf[C::KS], of[C::KS];

    // ---- MFMA(u): S^T_u, dP^T_u (SP) and dQ^T += K^T_{u-1} dS^T_{u-1} (QQ) ----
    auto mfma_phase = [&](int u, auto sp_tag, auto q_tag) {
        constexpr bool SP = decltype(sp_tag)::value;
        constexpr bool QQ = decltype(q_tag)::value;
        __builtin_amdgcn_s_setprio(1);
        using Sq = DqSeq<SP, QQ, C::KS>;
        constexpr int NM = Sq::NM;
        // an opaque zero keeps the per-lane address parts from being hoisted
        // out of the loop into registers held across phases
        int z = 0;
        asm volatile("" : "+v"(z));
        const uint32_t kb = sm0 + ((u >> 1) % C::NSTAGE) * C::STAGE + (u & 1) * 32 * C::ROW + z;
        const uint32_t tb = sm0 + (((u - 1) >> 1) % C::NSTAGE) * C::STAGE + ((u - 1) & 1) * 32 * C::ROW + z;
        u32x4_t ring[R];
        auto issue = [&](auto mc) {
            constexpr int m = decltype(mc)::value;
            if constexpr (m < NM) {
                constexpr int kd = Sq::kind(m), i = Sq::idx(m);
                if constexpr (kd == 0) {
                    ring[m % R] = dq_b128<0>(kb + row_off(i, z));
                } else if constexpr (kd == 1) {
                    ring[m % R] = dq_b128<C::TILE>(kb + row_off(i, z));
                } else {
                    constexpr int dt = i >> 1, kk = i & 1;
                    const u32x2_t lo = dq_tr16<16 * kk * C::ROW>(tb + tr_off(dt, 0, z));
                    const u32x2_t hi = dq_tr16<16 * kk * C::ROW>(tb + tr_off(dt, 1, z));
                    ring[m % R] = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
                }
            }
        };
        sfor<0, (LA < NM ? LA : NM)>(issue);
        sfor<0, NM>([&](auto mc) {
            constexpr int m = decltype(mc)::value;
            constexpr int kd = Sq::kind(m), i = Sq::idx(m);
            // reads issued after this MFMA's: those of MFMAs m+1 .. min(m+LA-1, NM-1)
            constexpr int last = (m + LA - 1 < NM - 1) ? m + LA - 1 : NM - 1;
            constexpr int after = Sq::reads_upto(last) - Sq::reads_upto(m);
            dq_lgkm<after>(ring[m % R]);
            const bf16x8_t a = __builtin_bit_cast(bf16x8_t, ring[m % R]);
            if constexpr (kd == 0) {
                const f32x16_t zero = {};
                s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[i], i == 0 ? zero : s, 0, 0, 0);
            } else if constexpr (kd == 1) {
                const f32x16_t zero = {};
                dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, of[i], i == 0 ? zero : dp, 0, 0, 0);
            } else {
                constexpr int dt = i >> 1, kk = i & 1;
                acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, sb[kk], acc[dt], 0, 0, 0);
            }
            issue(std::integral_constant<int, m + LA>{});
        });
        __builtin_amdgcn_s_setprio(0);
    };

    // ---- VALU(u): dS^T of unit u from its S^T, dP^T; element r of a lane is
    // key 32 u + 8 (r / 4) + 4 g + r % 4 of query qrow ----
    auto valu_phase = [&](int u) {
        float ds[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], c, -lse_v));
            ds[r] = pv * (dp[r] - dv_v);
        }
        const int k0 = 32 * u;
        if (k0 + 31 >= S || (CAUSAL && k0 + 31 > qw0)) {
            // keys past S and (causal) keys after the lane's query
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int k = k0 + 8 * (r >> 2) + 4 * g + (r & 3);
                if (!(k < S && (!CAUSAL || k <= qrow))) ds[r] = 0.0f * (dp[r] - dv_v);
            }
        }
        sb[0] = dq_pack8(ds);
        sb[1] = dq_pack8(ds + 8);
    };

    auto copy_k = [&](int t) {
        if (t < n_t) dma_part(t, 0, C::SEGW);
    };
    auto copy_v = [&](int t) {
        if (t < n_t) dma_part(t, C::SEGW, PIECES);
    };
    // start of step u: unit u = 2t copies tile t+2's K half, u = 2t+1 its V half
    auto copies = [&](int u) {
        if (u & 1) copy_v((u >> 1) + 2);
        else copy_k((u >> 1) + 2);
    };
    // end of step u for odd u = 2t+1: tile t+1 has landed
    auto land = [&](int u) {
        if ((u & 1) && (u >> 1) + 1 < n_t) dq_vm((u >> 1) + 2 < n_t ? PIECES : 0);
    };
    // a unit is needed by this wave if it has a key before S and (causal) at
    // or before the wave's last query.  Needed units come first, so MFMA(u)
    // runs while unit u-1 is needed: for the first unneeded unit u its S^T and
    // dP^T are computed and left unused, which keeps one MFMA-phase shape in
    // the loop (with several, the accumulators moved between registers).
    auto need = [&](int u) { return 32 * u < S && (!CAUSAL || 32 * u <= qw0 + 31); };

    // ---- prologue: Q, dO, lse, dvec and tiles 0, 1 in flight; wait for all but tile 1 ----
    // tile 1 is copied even when there is no tile 1 (an empty buffer range:
    // no traffic, into a stage nothing reads), so the wait count is one
    // constant on every path: the static ISA check cannot correlate two
    // branches on n_t
    dma_part(0, 0, PIECES);
    dma_part(1, 0, PIECES);
    dq_vm(PIECES);
    dq_barrier();
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) {
        dq_fence(qv[ks]);
        dq_fence(ov[ks]);
        qf[ks] = __builtin_bit_cast(bf16x8_t, qv[ks]);
        of[ks] = __builtin_bit_cast(bf16x8_t, ov[ks]);
    }
    dq_fence(lse_v);
    dq_fence(dv_v);
    lse_v *= kLog2eDq;

    using yes = std::integral_constant<bool, true>;
    using no = std::integral_constant<bool, false>;
    // Step 0 is split in two (group B has no VALU work yet, and starting it
    // half a unit late puts the groups out of phase); the last step is split
    // the same way for the tail of group B.
    if (grp == 0) {
        copies(0);
        if (need(0)) mfma_phase(0, yes{}, no{});
        dq_barrier();
        if (need(0)) valu_phase(0);
        land(0);
        dq_barrier();  // step 0
        for (int u = 1; u < U; ++u) {
            copies(u);
            if (need(u - 1)) mfma_phase(u, yes{}, yes{});
            if (need(u)) valu_phase(u);
            land(u);
            dq_barrier();  // step u
        }
        if (need(U - 1)) mfma_phase(U, no{}, yes{});
        dq_barrier();
        dq_barrier();  // step U
    } else {
        copies(0);
        dq_barrier();
        if (need(0)) mfma_phase(0, yes{}, no{});
        land(0);
        dq_barrier();  // step 0
        for (int u = 1; u < U; ++u) {
            copies(u);
            if (need(u - 1)) valu_phase(u - 1);
            if (need(u - 1)) mfma_phase(u, yes{}, yes{});
            land(u);
            dq_barrier();  // step u
        }
        if (need(U - 1)) valu_phase(U - 1);
        dq_barrier();
        if (need(U - 1)) mfma_phase(U, no{}, yes{});
        dq_barrier();  // step U
    }

    // ---- epilogue: dQ = scale * acc, bf16, through LDS (free after the last
    // barrier): each wave's 32 rows to its own region (16-byte unit u of row r
    // at u ^ (r % UNITS)), read back row-contiguous, 64 / UNITS rows per store ----
    constexpr int UN = D / 8;
    constexpr int RPI = 64 / UN;
    uint8_t* stg = sm + wave * 32 * D * 2;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            u32x2_t w;
            w[0] = pack_bf16x2(acc[dt][4 * jb + 0] * scale, acc[dt][4 * jb + 1] * scale);
            w[1] = pack_bf16x2(acc[dt][4 * jb + 2] * scale, acc[dt][4 * jb + 3] * scale);
            const int un = 4 * dt + jb;
            *reinterpret_cast<u32x2_t*>(stg + col * (D * 2) + ((un ^ (col & (UN - 1))) << 4) + 8 * g) = w;
        }
#pragma unroll
    for (int st = 0; st < UN / 2; ++st) {
        const int r = st * RPI + lane / UN, un = lane % UN;
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(stg + r * (D * 2) + ((un ^ (r & (UN - 1))) << 4));
        if (qw0 + r < S) *reinterpret_cast<u32x4_t*>(dQ + hoff + (int64_t)(qw0 + r) * D + 8 * un) = v;
    }
}

}  // namespace

hipError_t launch_flash_bwd_dq(int D, bool causal, const uint16_t* Q, const uint16_t* K,
                                  const uint16_t* V, const uint16_t* dO, const float* lse,
                                  const float* dvec, uint16_t* dQ, int BH, int S, float scale,
                                  hipStream_t s) {
    const int nq = (S + DQ_BQ - 1) / DQ_BQ;
    const dim3 grid(BH * nq), block(DQ_W * 64);
    if (D == 128) {
        if (causal)
            hipLaunchKernelGGL((flash_bwd_dq_pp_kernel<128, true>), grid, block, 0, s, Q, K, V, dO, lse, dvec,
                               dQ, BH, S, scale);
        else
            hipLaunchKernelGGL((flash_bwd_dq_pp_kernel<128, false>), grid, block, 0, s, Q, K, V, dO, lse, dvec,
                               dQ, BH, S, scale);
    } else {
        if (causal)
            hipLaunchKernelGGL((flash_bwd_dq_pp_kernel<64, true>), grid, block, 0, s, Q, K, V, dO, lse, dvec,
                               dQ, BH, S, scale);
        else
            hipLaunchKernelGGL((flash_bwd_dq_pp_kernel<64, false>), grid, block, 0, s, Q, K, V, dO, lse, dvec,
                               dQ, BH, S, scale);
    }
    return hipGetLastError();
}

}  // namespace jh
