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
// V^T must supply the same 8 keys per lane: V tiles are transposed into LDS
// (d-major, keys contiguous) with the key order inside each 16-key group
// stored as [0-3, 8-11, 4-7, 12-15], so each operand is one 16-byte read.
//
// Block: 4 waves x 32 queries = 128 query rows; key tiles of 64 (bf16) or 32
// (fp32) rows, double-buffered in LDS, loaded by the whole block.  Causal
// blocks stop at the diagonal, waves skip key tiles that are wholly above
// their own diagonal, and the heaviest query tiles of a head are dispatched
// first; each XCD works through whole heads so K and V are re-read from L2.
//
// bf16: v_mfma_f32_32x32x16_bf16, fp32 softmax statistics, exp2 with
// scale*log2(e) folded into one fma.  fp32: v_mfma_f32_32x32x2_f32 (full fp32
// products), same recurrence.
#include "common.hpp"
#include "launch.hpp"

namespace jh {
namespace {

constexpr int BQ = 128;
constexpr int NW = 4;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32, 64); }

// Workgroup -> (head, query tile).  Workgroups are dealt to the 8 XCDs round
// robin; the mapping gives each XCD whole heads (head = 8*j + xcd), all query
// tiles of a head in a row, heaviest (causal) first.  The ~64 workgroups an
// XCD runs at once then span about two heads, whose K and V (2 MiB each at
// S=4096, D=128) stay in that XCD's 4 MiB L2 instead of being re-read from
// HBM by every query tile.
__device__ __forceinline__ void block_coords(int BH, int nq, int* bh, int* q0) {
    const int b = blockIdx.x;
    int head, qi;
    if ((BH & 7) == 0) {
        const int xcd = b & 7, i = b >> 3;
        head = 8 * (i / nq) + xcd;
        qi = i % nq;
    } else {
        head = b / nq;
        qi = b % nq;
    }
    *bh = head;
    *q0 = (nq - 1 - qi) * BQ;
}

__device__ __forceinline__ bf16x8_t pack8(const float* p) {
    u32x4_t u;
    u[0] = pack_bf16x2(p[0], p[1]);
    u[1] = pack_bf16x2(p[2], p[3]);
    u[2] = pack_bf16x2(p[4], p[5]);
    u[3] = pack_bf16x2(p[6], p[7]);
    return __builtin_bit_cast(bf16x8_t, u);
}

// ---------------------------------------------------------------------------
// bf16
//
// K and V tiles are copied HBM -> LDS by the LDS DMA path
// (global_load_lds_dwordx4: each lane's 16 bytes land at base + 16 * lane),
// with no register staging; the source address of every lane is permuted so
// the data lands in the swizzled layout below.  Both tiles are row-major
// [key][d] (D*2 bytes per row):
//   K: 16-byte unit u of row r at unit u ^ (r & 7).  The S^T A operand (one
//      key row, 8 consecutive d per lane) is one ds_read_b128; 8 consecutive
//      rows hit distinct bank groups.
//   V: 8-byte chunk c of row r at chunk c ^ (4 * (r & 3)).  The V^T A operand
//      (8 keys of one d per lane) comes from two ds_read_b64_tr_b16: in each
//      16-lane group, lane s addresses row rb + s/4, chunk cb + s%4, and lane
//      i receives V[rb + k][4 cb + i] for k = 0..3.  The swizzle makes the 16
//      addresses of a group fall in 16 distinct chunks.
// Lazy rescale: the running max only moves when a tile's max exceeds it by
// more than 8 (log2 units); p = exp2(s*c - m) then stays <= 256, exact in the
// recurrence because the sum l uses the same m.
// ---------------------------------------------------------------------------
template <int D>
struct Bf16Cfg {
    static constexpr int BKV = 64;
    static constexpr int ROW = D * 2;                   // bytes per K / V row in LDS
    static constexpr int TILE = BKV * ROW;              // one operand tile
    static constexpr int STAGE = 2 * TILE;              // K then V
    static constexpr int UNITS = ROW / 16;              // 16-byte units per row
    static constexpr int NSEG = TILE / 1024;            // 1 KiB DMA segments per tile
};

__device__ __forceinline__ int k_off(int row, int unit, int rowbytes) {
    return row * rowbytes + ((unit ^ (row & 7)) << 4);
}
__device__ __forceinline__ int v_off(int row, int chunk8, int rowbytes) {
    return row * rowbytes + ((chunk8 ^ (4 * (row & 3))) << 3);
}

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4;
typedef __attribute__((address_space(3))) void lds_void;

template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void flash_fwd_bf16(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
    const uint16_t* __restrict__ V, uint16_t* __restrict__ O, float* __restrict__ lse, int BH, int S,
    float c_log2) {
    using C = Bf16Cfg<D>;
    constexpr int BKV = C::BKV;
    constexpr float kLazy = 8.0f;
    // One array per stage and operand, and the tile loop unrolled by two, so
    // every LDS access names its array statically: the compiler can then see
    // that reads of one stage never alias the DMA in flight into the other
    // and does not wait for that DMA before reading.
    __shared__ __attribute__((aligned(1024))) uint8_t k_s0[C::TILE];
    __shared__ __attribute__((aligned(1024))) uint8_t v_s0[C::TILE];
    __shared__ __attribute__((aligned(1024))) uint8_t k_s1[C::TILE];
    __shared__ __attribute__((aligned(1024))) uint8_t v_s1[C::TILE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 5, col = lane & 31;
    const int nq = (S + BQ - 1) / BQ;
    int bh, q0;
    block_coords(BH, nq, &bh, &q0);
    const int64_t hoff = (int64_t)bh * S * D;
    const uint16_t* Qh = Q + hoff;
    const uint16_t* Kh = K + hoff;
    const uint16_t* Vh = V + hoff;

    // this lane's query row and its Q fragments (B operand of S^T = K Q^T)
    const int qw0 = q0 + wave * 32;
    const int qrow = qw0 + col;
    bf16x8_t qf[D / 16];
    {
        const int qr = min(qrow, S - 1);  // rows past S compute on a valid row, never stored
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks)
            qf[ks] = __builtin_bit_cast(
                bf16x8_t, *reinterpret_cast<const u32x4_t*>(Qh + (int64_t)qr * D + ks * 16 + 8 * g));
    }

    const int kv_end = CAUSAL ? min(S, q0 + BQ) : S;
    const int n_kv = (kv_end + BKV - 1) / BKV;

    // ---- LDS DMA of one K + V tile: wave w moves segments w, w+4, ... ----
    constexpr int RPS = 1024 / C::ROW;  // rows per 1 KiB segment
    auto dma = [&](uint8_t* Ks, uint8_t* Vs, int k0) {
#pragma unroll
        for (int i = 0; i < C::NSEG / NW; ++i) {
            const int seg = i * NW + wave;
            const int r = seg * RPS + lane / C::UNITS;  // row within the tile
            const int up = lane % C::UNITS;             // physical 16-byte unit
            const int64_t key = min(k0 + r, S - 1);     // rows past S read a valid row
            const int ku = up ^ (r & 7);
            const int vu = up ^ (2 * (r & 3));
            __builtin_amdgcn_global_load_lds(Kh + key * D + 8 * ku, (lds_void*)(Ks + seg * 1024), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(Vh + key * D + 8 * vu, (lds_void*)(Vs + seg * 1024), 16, 0, 0);
        }
    };

    f32x16_t acc_o[D / 32];
#pragma unroll
    for (int i = 0; i < D / 32; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc_o[i][e] = 0.0f;
    float m_run = kNegInf;  // running max of scaled scores, log2 domain
    float l_run = 0.0f;     // this lane's partial running sum (its 16 keys per tile)

    auto compute = [&](const uint8_t* Ks, const uint8_t* Vs, int k0) {
        if (CAUSAL && k0 > qw0 + 31) return;  // whole tile above this wave's diagonal
        f32x16_t s[BKV / 32];
#pragma unroll
        for (int mt = 0; mt < BKV / 32; ++mt)
#pragma unroll
            for (int e = 0; e < 16; ++e) s[mt][e] = 0.0f;
        // all K fragments of the tile first, so LDS latency hides under MFMAs
        bf16x8_t kf[D / 16][BKV / 32];
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks)
#pragma unroll
            for (int mt = 0; mt < BKV / 32; ++mt)
                kf[ks][mt] = *reinterpret_cast<const bf16x8_t*>(
                    Ks + k_off(mt * 32 + col, 2 * ks + g, C::ROW));
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks)
#pragma unroll
            for (int mt = 0; mt < BKV / 32; ++mt)
                s[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks][mt], qf[ks], s[mt], 0, 0, 0);
        // masks: keys past S, and (causal) keys after this lane's query
        const bool need_mask = (k0 + BKV > S) || (CAUSAL && k0 + BKV - 1 > qw0);
        if (need_mask) {
#pragma unroll
            for (int mt = 0; mt < BKV / 32; ++mt)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int key = k0 + mt * 32 + 8 * (e >> 2) + 4 * g + (e & 3);
                    if (key >= S || (CAUSAL && key > qrow)) s[mt][e] = kNegInf;
                }
        }
        float mx = kNegInf;
#pragma unroll
        for (int mt = 0; mt < BKV / 32; ++mt)
#pragma unroll
            for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[mt][e]);
        mx = fmaxf(mx, xor32(mx)) * c_log2;
        // lazy rescale: move the running max only when it grows by > kLazy
        const bool grow = mx > m_run + kLazy;
        if (__ballot(grow)) {
            const float m_new = grow ? mx : m_run;
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first tile
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (int i = 0; i < D / 32; ++i)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc_o[i][e] *= alpha;
        }
        const float m_use = (m_run == kNegInf) ? 0.0f : m_run;  // row with no visible key yet
        float ls = 0.0f;
#pragma unroll
        for (int mt = 0; mt < BKV / 32; ++mt)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[mt][e], c_log2, -m_use));
                s[mt][e] = p;
                ls += p;
            }
        l_run += ls;
        // O^T += V^T P^T
        const int vs = lane & 15, vdh = (lane >> 4) & 1;
#pragma unroll
        for (int kk = 0; kk < BKV / 16; ++kk) {
            float pv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) pv[e] = s[kk >> 1][8 * (kk & 1) + e];
            const bf16x8_t pf = pack8(pv);
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) {
                const int c8 = 8 * dt + 4 * vdh + (vs & 3);
                const int r0 = 16 * kk + 4 * g + (vs >> 2);
                const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_s16x4*)(Vs + v_off(r0, c8, C::ROW)));
                const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_s16x4*)(Vs + v_off(r0 + 8, c8, C::ROW)));
                const s16x4_t v8[2] = {lo, hi};
                const bf16x8_t vf = __builtin_bit_cast(bf16x8_t, v8);
                acc_o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, acc_o[dt], 0, 0, 0);
            }
        }
    };

    if (n_kv > 0) {
        dma(k_s0, v_s0, 0);
        __builtin_amdgcn_s_waitcnt(0);  // this wave's DMA writes have landed
        __syncthreads();
        for (int j = 0; j < n_kv; j += 2) {
            if (j + 1 < n_kv) dma(k_s1, v_s1, (j + 1) * BKV);
            compute(k_s0, v_s0, j * BKV);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (j + 1 >= n_kv) break;
            if (j + 2 < n_kv) dma(k_s0, v_s0, (j + 2) * BKV);
            compute(k_s1, v_s1, (j + 1) * BKV);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
        }
    }

    // ---- epilogue: O = acc / l, bf16; lse = (m + log2 l) * ln 2 ----
    const float l_tot = l_run + xor32(l_run);
    const float inv = (l_tot > 0.0f) ? 1.0f / l_tot : 0.0f;
    if (qrow < S) {
        uint16_t* Orow = O + hoff + (int64_t)qrow * D;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int jb = 0; jb < 4; ++jb) {
                u32x2_t w;
                w[0] = pack_bf16x2(acc_o[dt][4 * jb + 0] * inv, acc_o[dt][4 * jb + 1] * inv);
                w[1] = pack_bf16x2(acc_o[dt][4 * jb + 2] * inv, acc_o[dt][4 * jb + 3] * inv);
                *reinterpret_cast<u32x2_t*>(Orow + dt * 32 + 8 * jb + 4 * g) = w;
            }
        if (lse && g == 0)
            lse[(int64_t)bh * S + qrow] = (m_run + __builtin_amdgcn_logf(l_tot)) * 0.6931471805599453f;
    }
}

// ---------------------------------------------------------------------------
// fp32: same recurrence on v_mfma_f32_32x32x2_f32.  The 32x32x2 A/B operands
// are one fp32 per lane (row/col = lane & 31, k = lane >> 5), so K and V are
// read from LDS as [key][d] rows without any transpose: for the PV product
// k-step (j, i) pairs keys 8j+i (lanes 0-31) and 8j+4+i (lanes 32-63), which
// are exactly the score accumulator element 4j+i each lane already holds.
// ---------------------------------------------------------------------------
template <int D>
struct F32Cfg {
    static constexpr int BKV = 32;
    static constexpr int ROWF = D + 4;  // padded row (floats): rows shift by 16 B
    static constexpr int K_FLOATS = BKV * ROWF;
    static constexpr int STAGE_FLOATS = 2 * K_FLOATS;  // K then V
    static constexpr int CHUNKS = BKV * D / 4;         // 16-byte chunks per tile
};

template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void flash_fwd_f32(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    float* __restrict__ O, float* __restrict__ lse, int BH, int S, float c_log2) {
    using C = F32Cfg<D>;
    constexpr int BKV = C::BKV;
    __shared__ __attribute__((aligned(16))) float smem[2 * C::STAGE_FLOATS];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 5, col = lane & 31;
    const int nq = (S + BQ - 1) / BQ;
    int bh, q0;
    block_coords(BH, nq, &bh, &q0);
    const int64_t hoff = (int64_t)bh * S * D;
    const float* Qh = Q + hoff;
    const float* Kh = K + hoff;
    const float* Vh = V + hoff;
    const int qw0 = q0 + wave * 32;
    const int qrow = qw0 + col;

    float qf[D / 2];  // Q[qrow][2 ks + g]
#pragma unroll
    for (int ks = 0; ks < D / 2; ++ks) qf[ks] = (qrow < S) ? Qh[(int64_t)qrow * D + 2 * ks + g] : 0.0f;

    const int kv_end = CAUSAL ? min(S, q0 + BQ) : S;
    const int n_kv = (kv_end + BKV - 1) / BKV;
    constexpr int PT = (C::CHUNKS + 255) / 256;
    f32x4_t rk[PT], rv[PT];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const int c = tid + 256 * i;
            const int key = c / (D / 4), ch = c % (D / 4);
            f32x4_t a = {0.f, 0.f, 0.f, 0.f}, b = {0.f, 0.f, 0.f, 0.f};
            if (c < C::CHUNKS && k0 + key < S) {
                a = *reinterpret_cast<const f32x4_t*>(Kh + (int64_t)(k0 + key) * D + 4 * ch);
                b = *reinterpret_cast<const f32x4_t*>(Vh + (int64_t)(k0 + key) * D + 4 * ch);
            }
            rk[i] = a;
            rv[i] = b;
        }
    };
    auto lstore = [&](int stage) {
        float* Ks = smem + stage * C::STAGE_FLOATS;
        float* Vs = Ks + C::K_FLOATS;
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const int c = tid + 256 * i;
            if (c < C::CHUNKS) {
                const int key = c / (D / 4), ch = c % (D / 4);
                *reinterpret_cast<f32x4_t*>(Ks + key * C::ROWF + 4 * ch) = rk[i];
                *reinterpret_cast<f32x4_t*>(Vs + key * C::ROWF + 4 * ch) = rv[i];
            }
        }
    };

    f32x16_t acc_o[D / 32];
#pragma unroll
    for (int i = 0; i < D / 32; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc_o[i][e] = 0.0f;
    float m_run = kNegInf, l_run = 0.0f;

    auto compute = [&](int stage, int k0) {
        if (CAUSAL && k0 > qw0 + 31) return;
        const float* Ks = smem + stage * C::STAGE_FLOATS;
        const float* Vs = Ks + C::K_FLOATS;
        f32x16_t s;
#pragma unroll
        for (int e = 0; e < 16; ++e) s[e] = 0.0f;
#pragma unroll
        for (int ks = 0; ks < D / 2; ++ks)
            s = __builtin_amdgcn_mfma_f32_32x32x2f32(Ks[col * C::ROWF + 2 * ks + g], qf[ks], s, 0, 0, 0);
        const bool need_mask = (k0 + BKV > S) || (CAUSAL && k0 + BKV - 1 > qw0);
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

    if (n_kv > 0) {
        gload(0);
        lstore(0);
        __syncthreads();
        for (int j = 0; j < n_kv; ++j) {
            const bool more = j + 1 < n_kv;
            if (more) gload((j + 1) * BKV);
            compute(j & 1, j * BKV);
            if (more) lstore((j + 1) & 1);
            __syncthreads();
        }
    }

    const float l_tot = l_run + xor32(l_run);
    const float inv = (l_tot > 0.0f) ? 1.0f / l_tot : 0.0f;
    if (qrow < S) {
        float* Orow = O + hoff + (int64_t)qrow * D;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int jb = 0; jb < 4; ++jb) {
                f32x4_t w;
#pragma unroll
                for (int i = 0; i < 4; ++i) w[i] = acc_o[dt][4 * jb + i] * inv;
                *reinterpret_cast<f32x4_t*>(Orow + dt * 32 + 8 * jb + 4 * g) = w;
            }
        if (lse && g == 0)
            lse[(int64_t)bh * S + qrow] = (m_run + __builtin_amdgcn_logf(l_tot)) * 0.6931471805599453f;
    }
}

template <typename KFN, typename T>
hipError_t go(KFN kfn, const void* Q, const void* K, const void* V, void* O, float* lse, int BH,
              int S, float c_log2, hipStream_t s) {
    const int nq = (S + BQ - 1) / BQ;
    hipLaunchKernelGGL(kfn, dim3(BH * nq), dim3(NW * 64), 0, s, static_cast<const T*>(Q),
                       static_cast<const T*>(K), static_cast<const T*>(V), static_cast<T*>(O), lse,
                       BH, S, c_log2);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_flash_fwd(int dtype, int causal, float scale, const void* Q, const void* K,
                            const void* V, void* O, float* lse, int B, int H, int S, int D,
                            hipStream_t s) {
    const int BH = B * H;
    if ((int64_t)BH * ((S + BQ - 1) / BQ) > 2147483647) return hipErrorInvalidValue;
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
