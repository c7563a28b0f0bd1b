// flash_bwd.hip - flash-attention backward on gfx950 MFMA (bf16).
//
// Gradients of O = softmax(scale * Q K^T [causal mask]) V per (batch, head),
// Q, K, V, O, dO [B,H,S,D] bf16 row-major, D in {64, 128}, given the
// forward's natural-log row log-sum-exp lse [B,H,S] (jules_hip_flash_attn_fwd):
//   P   = exp(scale * Q K^T - lse)           (masked entries 0)
//   dV  = P^T dO
//   dP  = dO V^T
//   dS  = P * (dP - rowsum(dO * O))
//   dQ  = scale * dS K,   dK = scale * dS^T Q
// The reference has no backward pass (its flashAttention, FlashAttention.h:
// 130-309, is forward only); this is the training counterpart of the forward
// kernel in flash_fwd.hip, with the same operand layouts.
//
// Three launches, none with atomics, so results are deterministic:
//   1. dvec = rowsum(dO * O) in fp32 (HBM-bound);
//   2. dK, dV: a workgroup owns 128 keys (4 waves x 32) and walks the query
//      blocks of 64 (from the diagonal on, if causal);
//   3. dQ (flash_bwd_dq.hip): a workgroup owns 256 queries (8 waves x 32)
//      and walks the key units of 32 (up to the diagonal, if causal) in the
//      forward kernel's ping-pong.
// The dQ pass recomputes P and dP instead of accumulating dQ across key
// blocks with atomics.
//
// MFMA v_mfma_f32_32x32x16_bf16: lane l supplies A[l%32][8(l/32)..+7] and
// B[8(l/32)..+7][l%32]; the result's register r of lane l is row
// 8(r/4) + 4(l/32) + r%4, column l%32.  A product over a 16-long k can take
// any k order, as long as A and B use the same one: results of one product,
// whose lane holds the 8 rows {4g + 0..3, 8 + 4g + 0..3} of a 16-row step
// (g = l/32), are fed straight back as the A (dK/dV pass) or B (dQ pass)
// operand of the next, and the other operand is read in that order with
// transposing LDS reads (ds_read_b64_tr_b16: a 16-lane group reads 4 rows x
// 16 columns, lane i receiving column i of the 4 rows).
//
//   dK/dV pass (lane = key column):  S = Q K^T, dP = dO V^T;  then
//     dV += P^T dO and dK += dS^T Q with P, dS as A and dO, Q read transposed.
//   dQ pass (lane = query column):   S^T = K Q^T, dP^T = V dO^T;  then
//     dQ^T += K^T dS^T with dS^T as B and K read transposed.
// Tiles are staged through LDS with 16 bytes of padding per row (row reads
// then hit 16 distinct bank groups).
#include "common.hpp"
#include "launch.hpp"

namespace jh {
namespace {


constexpr float kLog2e = 1.4426950408889634f;
constexpr int BW = 4;            // waves per workgroup
constexpr int BT = BW * 64;      // threads per workgroup
constexpr int BOWN = BW * 32;    // keys (dK/dV pass) or queries (dQ pass) a workgroup owns

// Workgroup -> (head, block rank), rank 0 the block with the longest causal
// range.  Workgroups are dealt to the 8 XCDs round robin; each XCD takes whole
// heads (head = 8*j + xcd) two at a time with their blocks interleaved,
// longest first, so the heads' operands stay in that XCD's L2 and the CUs
// that finish early take the next long blocks.  (The forward interleaves four
// heads, which gives the XCD's four shader engines equal work there; with two
// workgroups per CU here, four heads measured the same as two.)
__device__ __forceinline__ void bwd_block(int nblk, int* bh, int* rank) {
    const int b = blockIdx.x, BH = gridDim.x / nblk;
    if ((BH & 7) == 0) {
        const int xcd = b & 7, i = b >> 3;
        const int J = BH >> 3;
        const int g = i / (2 * nblk), r = i - g * 2 * nblk;
        const int gs = min(2, J - 2 * g);
        *bh = 8 * (2 * g + r % gs) + xcd;
        *rank = r / gs;
    } else {
        *bh = b / nblk;
        *rank = b % nblk;
    }
}

template <int D>
struct BwdCfg {
    static constexpr int PITCH = D * 2 + 16;   // bytes per LDS row
    static constexpr int KS = D / 16;          // 16-wide k steps over the head dim
    static constexpr int DT = D / 32;          // 32-wide d blocks
};

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

// 8 fp32 -> bf16x8 (round to nearest even)
__device__ __forceinline__ bf16x8_t pack8(const float* f) {
    u32x4_t u;
    u[0] = pack_bf16x2(f[0], f[1]);
    u[1] = pack_bf16x2(f[2], f[3]);
    u[2] = pack_bf16x2(f[4], f[5]);
    u[3] = pack_bf16x2(f[6], f[7]);
    return __builtin_bit_cast(bf16x8_t, u);
}

// Copy rows [r0, r0 + nrows) of a [S][D] bf16 matrix into an LDS tile with
// the padded pitch; rows past S are copies of row S-1 (their results are
// masked or never stored).
template <int D>
__device__ __forceinline__ void load_tile(uint8_t* tile, const uint16_t* __restrict__ src, int r0,
                                          int nrows, int S, int tid) {
    constexpr int UNITS = D / 8;  // 16-byte units per row
    for (int e = tid; e < nrows * UNITS; e += BT) {
        const int r = e / UNITS, u = e % UNITS;
        const int gr = min(r0 + r, S - 1);
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(src + (int64_t)gr * D + 8 * u);
        *reinterpret_cast<u32x4_t*>(tile + r * BwdCfg<D>::PITCH + 16 * u) = v;
    }
}

template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

// The same transposed fragment by inline asm with an explicit wait
// (tr_issue / tr_wait): the compiler then keeps the issue order, so reads run
// ahead of the MFMAs that consume them.  LDS reads complete in order, so a
// wait for at most N outstanding reads covers every read issued N or more
// reads earlier.
template <int D>
__device__ __forceinline__ uint32_t tr_addr(const uint8_t* tile, int rb, int dt, int lane) {
    const int g = lane >> 5, vs = lane & 15, vdh = (lane >> 4) & 1;
    const int r = rb + 4 * g + (vs >> 2);
    const int chunk = 8 * dt + 4 * vdh + (vs & 3);
    return (uint32_t)(uintptr_t)(tile + r * BwdCfg<D>::PITCH + chunk * 8);
}
struct TrFrag {
    u32x2_t lo, hi;
};
// OFF: a compile-time byte offset added by the instruction itself (one base
// register per pipeline instead of one address computation per read)
template <int D, int OFF>
__device__ __forceinline__ TrFrag tr_issue(uint32_t addr) {
    static_assert(OFF >= 0 && OFF + 8 * BwdCfg<D>::PITCH < 65536, "16-bit LDS offset");
    TrFrag f;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(f.lo) : "v"(addr), "n"(OFF) : "memory");
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2"
                 : "=v"(f.hi)
                 : "v"(addr), "n"(OFF + 8 * BwdCfg<D>::PITCH)
                 : "memory");
    return f;
}
template <int N>
__device__ __forceinline__ bf16x8_t tr_wait(TrFrag& f) {
    asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(f.lo), "+v"(f.hi) : "n"(N) : "memory");
    const u32x4_t v = {f.lo[0], f.lo[1], f.hi[0], f.hi[1]};
    return as_bf16x8(v);
}

// Runs NM MFMAs whose fragments come from transposing reads: the reads of
// MFMAs m+1 .. m+L are in flight while m runs, in a ring of L+2 fragments
// (a fragment is refilled only after the MFMA two before has taken it).
// MFMA m reads at base + off(m), off returning std::integral_constant (a
// compile-time offset); use(m, frag) issues MFMA m.
template <int M>
using ic = std::integral_constant<int, M>;
template <int D, int NM, int L, typename O, typename U>
__device__ __forceinline__ void tr_pipeline(uint32_t base, O&& off, U&& use) {
    constexpr int R = L + 2;
    TrFrag ring[R];
    static_for<0, L>([&](auto mi) {
        constexpr int m = decltype(mi)::value;
        ring[m] = tr_issue<D, decltype(off(ic<m>{}))::value>(base);
    });
    static_for<0, NM>([&](auto mi) {
        constexpr int m = decltype(mi)::value;
        if constexpr (m + L < NM) ring[(m + L) % R] = tr_issue<D, decltype(off(ic<m + L>{}))::value>(base);
        constexpr int later = (m + L < NM ? L : NM - 1 - m);  // MFMAs whose reads follow m's
        use(mi, tr_wait<2 * later>(ring[m % R]));
    });
}

// A/B fragment of the S and dP products: 8 consecutive head-dim elements of
// one row (16 bytes), read by inline asm at a compile-time byte offset and
// waited for with row_wait (the compiler's own schedule waited on every read
// right before its MFMA)
template <int OFF>
__device__ __forceinline__ u32x4_t row_issue(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "16-bit LDS offset");
    u32x4_t v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF) : "memory");
    return v;
}
template <int N>
__device__ __forceinline__ void row_wait1(u32x4_t& a) {
    static_assert(N >= 0 && N <= 15, "lgkmcnt is a 4-bit count");
    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(a) : "n"(N) : "memory");
}
template <int N>
__device__ __forceinline__ void row_wait2(u32x4_t& a, u32x4_t& b) {
    static_assert(N >= 0 && N <= 15, "lgkmcnt is a 4-bit count");
    asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "n"(N) : "memory");
}

__device__ __forceinline__ f32x16_t mfma(bf16x8_t a, bf16x8_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16_t zero16() {
    f32x16_t z;
#pragma unroll
    for (int i = 0; i < 16; ++i) z[i] = 0.0f;
    return z;
}

// ---- 1. dvec = rowsum(dO * O): 16 lanes per row, 16 bytes each -------------
template <int D>
__global__ __launch_bounds__(256) void flash_bwd_dvec_kernel(const uint16_t* __restrict__ O,
                                                             const uint16_t* __restrict__ dO,
                                                             float* __restrict__ dvec, int64_t rows) {
    constexpr int LPR = D / 8;  // lanes per row
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t row = t / LPR;
    const int u = (int)(t % LPR);
    float s = 0.0f;
    if (row < rows) {
        const u32x4_t o = *reinterpret_cast<const u32x4_t*>(O + row * D + 8 * u);
        const u32x4_t d = *reinterpret_cast<const u32x4_t*>(dO + row * D + 8 * u);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s = fmaf(bf16_lo(o[i]), bf16_lo(d[i]), s);
            s = fmaf(bf16_hi(o[i]), bf16_hi(d[i]), s);
        }
    }
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if (row < rows && u == 0) dvec[row] = s;
}

// ---- 2. dK, dV ----------------------------------------------------------------
// 4 waves x 32 keys.  Each wave holds its keys' K rows (the B operand of S)
// in registers next to the dK/dV accumulators; the V rows (B of dP) are read
// from an LDS copy of the workgroup's 128 V rows.  With 32-query steps this
// fits in 256 registers, so two workgroups share a CU (two waves per SIMD).  Q/dO tiles of 32 queries
// are double buffered in LDS: the global loads of block i+1 are issued into
// registers before block i is multiplied and stored to the other buffer
// after, one barrier per block.
constexpr int KVSTEP = 32;  // queries per dK/dV loop step
template <int D, bool CAUSAL>
__global__ __launch_bounds__(BT, 2) void flash_bwd_dkdv_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    const uint16_t* __restrict__ dO, const float* __restrict__ lse, const float* __restrict__ dvec,
    uint16_t* __restrict__ dK, uint16_t* __restrict__ dV, int S, float scale) {
    using C = BwdCfg<D>;
    constexpr int UNITS = D / 8;
    constexpr int PF = 2 * KVSTEP * UNITS / BT;  // prefetched units per thread (Q then dO)
    __shared__ __attribute__((aligned(16))) uint8_t qo_t[2][2][KVSTEP * C::PITCH];  // [buf][Q, dO]
    __shared__ __attribute__((aligned(16))) float ld_t[2][2][KVSTEP];               // [buf][lse, dvec]
    __shared__ __attribute__((aligned(16))) uint8_t v_t[BOWN * C::PITCH];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 5, col = lane & 31;
    const int nkb = (S + BOWN - 1) / BOWN;
    int bh, rank;
    bwd_block(nkb, &bh, &rank);
    const int k0 = rank * BOWN;  // longest causal range (first keys) first
    const int64_t hoff = (int64_t)bh * S * D;
    const uint16_t* Qh = Q + hoff;
    const uint16_t* Oh = dO + hoff;
    const float c = scale * kLog2e;

    // this lane's key (S / dP column) and its K row (B operand of S)
    const int key = k0 + wave * 32 + col;
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    const int kr = min(key, S - 1);
    bf16x8_t kf[C::KS];
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks)
        kf[ks] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(K + hoff + (int64_t)kr * D + 16 * ks + 8 * g));
    load_tile<D>(v_t, V + hoff, k0, BOWN, S, tid);  // made visible by the first barrier
    const int vrow = wave * 32 + col;

    u32x4_t pf[PF];
    float pl = 0.0f;
    auto gload = [&](int q0) {
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            const int e = tid + BT * p;
            const int r = (e / UNITS) % KVSTEP, u = e % UNITS;
            const int64_t gr = min(q0 + r, S - 1);
            pf[p] = *reinterpret_cast<const u32x4_t*>((e / UNITS < KVSTEP ? Qh : Oh) + gr * D + 8 * u);
        }
        if (tid < 2 * KVSTEP) {
            const int64_t q = (int64_t)bh * S + min(q0 + (tid % KVSTEP), S - 1);
            pl = tid < KVSTEP ? lse[q] * kLog2e : dvec[q];
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            const int e = tid + BT * p;
            const int r = (e / UNITS) % KVSTEP, u = e % UNITS;
            *reinterpret_cast<u32x4_t*>(&qo_t[buf][e / UNITS / KVSTEP][r * C::PITCH + 16 * u]) = pf[p];
        }
        if (tid < 2 * KVSTEP) ld_t[buf][tid / KVSTEP][tid % KVSTEP] = pl;
    };

    f32x16_t dk[C::DT], dv[C::DT];
#pragma unroll
    for (int i = 0; i < C::DT; ++i) {
        dk[i] = zero16();
        dv[i] = zero16();
    }

    const int qb_begin = CAUSAL ? (k0 / KVSTEP) : 0;
    const int qb_end = (S + KVSTEP - 1) / KVSTEP;
    gload(qb_begin * KVSTEP);
    sstore(0);
    __syncthreads();
    for (int qb = qb_begin; qb < qb_end; ++qb) {
        const int buf = (qb - qb_begin) & 1, q0 = qb * KVSTEP;
        if (qb + 1 < qb_end) gload(q0 + KVSTEP);
        const uint8_t* q_t = qo_t[buf][0];
        const uint8_t* do_t = qo_t[buf][1];
        const float* lse_t = ld_t[buf][0];
        const float* dv_t = ld_t[buf][1];

        // every query of the step is < S and (causal) after every key of the wave
        const bool unmasked = q0 + KVSTEP <= S && (!CAUSAL || k0 + wave_u * 32 + 31 <= q0);
        // S = Q K^T and dP = dO V^T for the 32 queries x this wave's 32 keys
        bf16x8_t pa[1][2], sa[1][2];  // P and dS as A operands: [16-query step]
#pragma unroll
        for (int h = 0; h < 1; ++h) {
            f32x16_t s = zero16(), dp = zero16();
            // each MFMA's fragments are read one MFMA ahead (inline asm with
            // explicit waits; one register set per operand)
            const uint32_t qa = (uint32_t)(uintptr_t)(q_t + (h * 32 + col) * C::PITCH + 16 * g);
            const uint32_t da = (uint32_t)(uintptr_t)(do_t + (h * 32 + col) * C::PITCH + 16 * g);
            const uint32_t va = (uint32_t)(uintptr_t)(v_t + vrow * C::PITCH + 16 * g);
            u32x4_t rq = row_issue<0>(qa), rd = row_issue<0>(da), rv = row_issue<0>(va);
            static_for<0, C::KS>([&](auto ksc) {
                constexpr int ks = decltype(ksc)::value;
                constexpr bool more = ks + 1 < C::KS;
                row_wait1<2>(rq);  // dO(ks), V(ks) may still be in flight
                s = mfma(as_bf16x8(rq), kf[ks], s);
                if constexpr (more) rq = row_issue<32 * (ks + 1)>(qa);
                row_wait2<more ? 1 : 0>(rd, rv);  // Q(ks+1) may still be in flight
                dp = mfma(as_bf16x8(rd), as_bf16x8(rv), dp);
                if constexpr (more) {
                    rd = row_issue<32 * (ks + 1)>(da);
                    rv = row_issue<32 * (ks + 1)>(va);
                }
            });
            // register r: query 8(r/4) + 4g + r%4 of this block.  Every step
            // computes P and dS unmasked; only the last block and the
            // diagonal then zero the masked elements (queries past S, causal
            // keys after the query).  The
            // per-element compares and selects on every step were ~a quarter
            // of the step's vector work.
            float p[16], ds[16];
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int ql = h * 32 + 8 * r4 + 4 * g;
                const f32x4_t l4 = *reinterpret_cast<const f32x4_t*>(&lse_t[ql]);
                const f32x4_t d4 = *reinterpret_cast<const f32x4_t*>(&dv_t[ql]);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = 4 * r4 + i;
                    const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], c, -l4[i]));
                    p[r] = pv;
                    ds[r] = pv * (dp[r] - d4[i]);
                }
            }
            if (!unmasked) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int q = q0 + h * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                    if (!(q < S && (!CAUSAL || key <= q))) {
                        p[r] = 0.0f;
                        ds[r] = 0.0f;
                    }
                }
            }
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                pa[h][t] = pack8(p + 8 * t);
                sa[h][t] = pack8(ds + 8 * t);
            }
        }
        // dV += P^T dO, dK += dS^T Q: A = P / dS (this lane's key), B read
        // transposed in the matching query order
        // MFMA m = (dt, t, which): which 0 = dV (dO read), 1 = dK (Q read);
        // the reads of MFMAs m+1 and m+2 are in flight while m runs
        // MFMA m reads rows 16 ((m >> 1) & 1) + .. of Q (odd m) or dO, d block
        // m >> 2: do_t = q_t + KVSTEP rows, so one base and constant offsets
        tr_pipeline<D, 4 * C::DT, 2>(
            tr_addr<D>(q_t, 0, 0, lane),
            [](auto mi) {
                constexpr int m = decltype(mi)::value;
                return ic<((m & 1) ? 0 : KVSTEP * C::PITCH) + 16 * ((m >> 1) & 1) * C::PITCH + 64 * (m >> 2)>{};
            },
            [&](auto mi, bf16x8_t b) {
                constexpr int m = decltype(mi)::value, dt = m >> 2, t = (m >> 1) & 1;
                if constexpr (m & 1) dk[dt] = mfma(sa[0][t], b, dk[dt]);
                else dv[dt] = mfma(pa[0][t], b, dv[dt]);
            });
        // keep the transposing reads two MFMAs ahead of their use
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
        for (int i = 0; i < 4 * C::DT - 2; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        if (qb + 1 < qb_end) sstore(buf ^ 1);
        __syncthreads();
    }

    // dK = scale * dS^T Q, dV = P^T dO; register r of block dt: key row
    // 8(r/4) + 4g + r%4 of this wave's 32, head dim 32 dt + col
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int kk = k0 + wave * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
            if (kk >= S) continue;
            const int64_t o = hoff + (int64_t)kk * D + 32 * dt + col;
            dK[o] = __builtin_bit_cast(uint16_t, (__bf16)(dk[dt][r] * scale));
            dV[o] = __builtin_bit_cast(uint16_t, (__bf16)dv[dt][r]);
        }
}

// ---- 3. dQ: flash_bwd_dq.hip (an 8-wave ping-pong like the forward kernel) ----

template <int D, bool CAUSAL>
hipError_t launch_bwd(const uint16_t* Q, const uint16_t* K, const uint16_t* V, const uint16_t* O,
                      const uint16_t* dO, const float* lse, uint16_t* dQ, uint16_t* dK,
                      uint16_t* dV, int BH, int S, float scale, float* dvec, hipStream_t s) {
    const int64_t rows = (int64_t)BH * S;
    const int64_t threads = rows * (D / 8);
    hipLaunchKernelGGL(flash_bwd_dvec_kernel<D>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       s, O, dO, dvec, rows);
    const int nb = (S + BOWN - 1) / BOWN;
    hipLaunchKernelGGL((flash_bwd_dkdv_kernel<D, CAUSAL>), dim3(BH * nb), dim3(BT), 0, s, Q, K, V, dO,
                       lse, dvec, dK, dV, S, scale);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_flash_bwd_dq(D, CAUSAL, Q, K, V, dO, lse, dvec, dQ, BH, S, scale, s);
}

}  // namespace

size_t flash_bwd_workspace_size(int B, int H, int S) { return (size_t)B * H * S * sizeof(float); }

hipError_t launch_flash_bwd(int dtype, int causal, float scale, const void* Q, const void* K,
                            const void* V, const void* O, const void* dO, const float* lse,
                            void* dQ, void* dK, void* dV, int B, int H, int S, int D, void* ws,
                            hipStream_t s) {
    if (dtype != JH_BF16) return hipErrorInvalidValue;
    const auto* q = static_cast<const uint16_t*>(Q);
    const auto* k = static_cast<const uint16_t*>(K);
    const auto* v = static_cast<const uint16_t*>(V);
    const auto* o = static_cast<const uint16_t*>(O);
    const auto* dout = static_cast<const uint16_t*>(dO);
    auto* dq = static_cast<uint16_t*>(dQ);
    auto* dk = static_cast<uint16_t*>(dK);
    auto* dv = static_cast<uint16_t*>(dV);
    float* dvec = static_cast<float*>(ws);
    const int BH = B * H;
    if (D == 128) {
        return causal ? launch_bwd<128, true>(q, k, v, o, dout, lse, dq, dk, dv, BH, S, scale, dvec, s)
                      : launch_bwd<128, false>(q, k, v, o, dout, lse, dq, dk, dv, BH, S, scale, dvec, s);
    }
    return causal ? launch_bwd<64, true>(q, k, v, o, dout, lse, dq, dk, dv, BH, S, scale, dvec, s)
                  : launch_bwd<64, false>(q, k, v, o, dout, lse, dq, dk, dv, BH, S, scale, dvec, s);
}

}  // namespace jh
