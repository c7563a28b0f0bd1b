// rowops.hip - row kernels: fusedSoftmax, fusedLayerNorm, fusedCrossEntropyLoss.
//
// Reference: include/jules/Kernel/FusedKernels.h:464-526 (softmax),
// :532-600 (layernorm), :766-854 (cross entropy), AVX-512 branches.  Each
// reference row is processed by one thread as 16-float vectors plus a scalar
// tail; the per-element arithmetic is kept here:
//   softmax  e = fast_exp(x - max) for j < N & ~15, expf(x - max) for the
//            tail; out = e * (1 / sum) for j < N & ~15, e / sum for the tail;
//   layernorm mean = sum / N, var = sum fma(d, d) / N, inv_std =
//            1 / sqrtf(var + eps), out = fma((x - mean) * inv_std, gamma, beta);
//   cross entropy  p = softmax row, loss_i = -logf(p[t] + 1e-10),
//            grad = (p - onehot(t)) / M, loss = sum_i loss_i / M.
// The sums are taken in a different (fixed, tree) order than the reference's
// 16 lane partials, so results match it to rounding, not bit for bit.
//
// All three are HBM-bound, and the row is held in registers so it is read
// from HBM once and written once: one wave per row for N <= 4096 (four rows
// per workgroup), one 1024-thread workgroup per row for N <= 65536 (up to 64
// elements per thread).  With N % 4 == 0 and 16-byte aligned rows each
// thread moves 16-byte pieces, otherwise single floats; either way every wave
// instruction covers contiguous bytes.  Rows longer than 65536 get a
// 1024-thread workgroup that keeps the row's first 65536 elements on chip
// (registers and LDS) and streams the rest in chunks of 16 elements per
// thread, in the reference's own three passes (softmax and cross entropy:
// max, sum of exponentials, write with the exponentials recomputed;
// layernorm: sum, squared deviations, write).  Reductions are a fixed butterfly within a wave and
// a fixed tree across waves, so results are deterministic.
#include <cfloat>
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"

namespace jh {
namespace {

constexpr int ROWS_PER_BLOCK = 4;
constexpr int MAX_CACHED = 4096;      // longest row held in one wave's registers
constexpr int BT = 1024;              // threads of a block that holds one row
constexpr int MAX_BLOCK_CACHED = 65536;  // longest row held in a block's registers

// Butterfly over the wave's 64 lanes: v of lane ^ o for o = 32, 16, .., 1.
// The lane id passes through an empty asm at each reduction, so the six
// permute addresses are rebuilt there (two instructions each) instead of
// being kept live between a row's reductions, where they would be spilled in
// the kernels that hold 64 elements per thread.
__device__ __forceinline__ int fresh_lane() {
    int lane = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    asm volatile("" : "+v"(lane));
    return lane;
}
__device__ __forceinline__ float lane_xor(float v, int lane, int o) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ o) << 2, __builtin_bit_cast(int, v)));
}
// the wave's index in the workgroup, in a scalar register
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6); }
__device__ __forceinline__ float wave_max(float v) {
    const int lane = fresh_lane();
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, lane_xor(v, lane, o));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
    const int lane = fresh_lane();
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += lane_xor(v, lane, o);
    return v;
}
// max as the reference's _mm512_max_ps(acc, x): acc > x ? acc : x
__device__ __forceinline__ float ref_max(float acc, float x) { return acc > x ? acc : x; }

// exp of the reference: fast_exp on the part of the row that fills whole
// 16-float vectors, libm expf on the tail
__device__ __forceinline__ float row_exp(float d, int j, int nv) {
    return j < nv ? fast_exp(d) : expf(d);
}
__device__ __forceinline__ float row_norm(float e, float inv, float sum, int j, int nv) {
    return j < nv ? e * inv : e / sum;
}

// ---- a row held in the registers of a group of G threads (one wave, or
// the BT threads of a block).  Thread `tid` holds ELEMS elements: with VEC,
// 16-byte pieces f = tid + G*t, elements 4f .. 4f+3 (rows 16-byte aligned,
// N % 4 == 0); without, elements j = tid + G*t.  Every load or store
// instruction of a wave covers contiguous bytes.
// The BT-thread rows use range-checked buffer accesses over the row (N * 4
// bytes, N <= 65536): a store past the row's end is dropped without a
// branch, and at 64 elements per thread the kernels fit in 128 registers.
// One wave per row uses plain global accesses, which measured 3-13 % faster
// there (many short rows per CU); a row's stores all take the same kind of
// access, so the same thread's later store to an address lands last. ----
template <int G, int ELEMS, bool VEC>
struct RowRegs {
    static constexpr int W = VEC ? 4 : 1;   // elements per access
    static constexpr int NA = ELEMS / W;    // accesses per thread
    static constexpr bool BUF = G != 64;
    using Access = std::conditional_t<VEC, f32x4_t, float>;
    float v[ELEMS];
    __device__ __forceinline__ static int elem(int tid, int a, int i) {
        return VEC ? 4 * (tid + G * a) + i : tid + G * a;
    }
    // access a of the group's threads covers elements [first(a), first(a + 1))
    static constexpr int first(int a) { return G * W * a; }
    // byte offset of this thread's access 0; access a adds 4 * first(a).  The
    // stores take it through an empty asm, so the compiler rebuilds their
    // offsets instead of keeping every load's offset live until the stores.
    __device__ __forceinline__ static uint32_t base_off(int tid) { return (uint32_t)elem(tid, 0, 0) * 4u; }
    __device__ __forceinline__ static uint32_t fresh_base_off(int tid) {
        uint32_t o = base_off(tid);
        asm volatile("" : "+v"(o));
        return o;
    }
    __device__ __forceinline__ static __amdgpu_buffer_rsrc_t row_rsrc(const float* p, int N) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), 0, (uint32_t)N * 4u,
                                                 0x00020000);
    }
    // one access of the row p at byte offset o (o + 4 W <= N * 4)
    __device__ __forceinline__ static Access load_at(const float* p, __amdgpu_buffer_rsrc_t src,
                                                     uint32_t o) {
        if constexpr (BUF) {
            if constexpr (VEC)
                return __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(src, o, 0, 0));
            else
                return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(src, o, 0, 0));
        } else {
            return *reinterpret_cast<const Access*>(reinterpret_cast<const char*>(p) + o);
        }
    }
    // one access stored at byte offset o; nothing if o is past the row
    __device__ __forceinline__ static void store_at(float* p, __amdgpu_buffer_rsrc_t dst, int N,
                                                    uint32_t o, Access q) {
        if constexpr (BUF) {
            if constexpr (VEC)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, q), dst, o, 0, 0);
            else
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, q), dst, o, 0, 0);
        } else if (o < (uint32_t)N * 4u) {
            *reinterpret_cast<Access*>(reinterpret_cast<char*>(p) + o) = q;
        }
    }
    // v[] = x[]; past the row's end, with LAST the row's last element (piece,
    // with VEC) again, else 0.  LAST leaves the row's max unchanged without a
    // select per element (in the BT-thread rows a compare per element held
    // until its load lands costs a pair of scalar registers each).  The
    // offsets are clamped into the row; the buffer form reads 0 past it.
    template <bool LAST>
    __device__ __forceinline__ void load(const float* x, int N, int tid) {
        const __amdgpu_buffer_rsrc_t src = row_rsrc(x, N);
        const uint32_t o0 = base_off(tid);
        const uint32_t last = (uint32_t)(N - W) * 4u;  // N >= W: with VEC, N % 4 == 0
#pragma unroll
        for (int a = 0; a < NA; ++a) {
            const uint32_t o = o0 + 4u * (uint32_t)first(a);
            Access q = load_at(x, src, (LAST || !BUF) ? (o < last ? o : last) : o);
            if constexpr (!LAST && !BUF) q = o <= last ? q : Access{};
            if constexpr (VEC) {
#pragma unroll
                for (int i = 0; i < 4; ++i) v[4 * a + i] = q[i];
            } else {
                v[a] = q;
            }
        }
    }
    // y[] = f(v[]), each access stored as soon as it is mapped
    template <typename F>
    __device__ __forceinline__ void store(float* y, int N, int tid, F&& f) const {
        const __amdgpu_buffer_rsrc_t dst = row_rsrc(y, N);
        const uint32_t o0 = fresh_base_off(tid);
#pragma unroll
        for (int a = 0; a < NA; ++a) {
            Access q;
            if constexpr (VEC)
                q = f32x4_t{f(v[4 * a]), f(v[4 * a + 1]), f(v[4 * a + 2]), f(v[4 * a + 3])};
            else
                q = f(v[a]);
            store_at(y, dst, N, o0 + 4u * (uint32_t)first(a), q);
        }
    }
    // f(element index, value) over this thread's elements inside the row
    template <typename F>
    __device__ __forceinline__ void each(int N, int tid, F&& f) {
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
            for (int i = 0; i < W; ++i) {
                const int j = elem(tid, a, i);
                f(j, v[W * a + i], j < N);
            }
    }
    // The row's tail [nv, N) (N % 16 elements; none when nv == N).  A thread
    // holds at most one access inside it: the tail has fewer than 16
    // elements and the group at least 64 threads (with VEC, nv % 16 == 0 and
    // N % 4 == 0, so a piece is wholly in or out).
    static constexpr uint32_t TAIL_NONE = 0x80000000u;  // past any row: no store
    // byte offset of this thread's tail access, or TAIL_NONE: the one element
    // (piece) u in [nv, N) (pieces [nv/4, N/4)) with u % G == tid
    __device__ __forceinline__ static uint32_t tail_off(int N, int nv, int tid) {
        const int u0 = nv / W, u1 = N / W;
        const int u = u0 + ((tid - u0) & (G - 1));
        return u < u1 ? (uint32_t)u * (uint32_t)(4 * W) : TAIL_NONE;
    }
    // values of that access (0 without one)
    __device__ __forceinline__ void tail(int N, int nv, int tid, float (&xt)[W]) const {
#pragma unroll
        for (int i = 0; i < W; ++i) xt[i] = 0.0f;
#pragma unroll
        for (int a = 0; a < NA; ++a) {
            const int j0 = elem(tid, a, 0);
            const bool t = j0 >= nv && j0 < N;
#pragma unroll
            for (int i = 0; i < W; ++i) xt[i] = t ? v[W * a + i] : xt[i];
        }
    }
    // y at byte offset off = q, one float, the same kind of access as store()
    __device__ __forceinline__ static void store1(float* y, int N, uint32_t off, float q) {
        RowRegs<G, 1, false>::store_at(y, row_rsrc(y, N), N, off, q);
    }
    // this thread's tail access, stored after store() (nothing for TAIL_NONE)
    __device__ __forceinline__ static void store_tail(float* y, int N, uint32_t toff, const float (&q)[W]) {
        Access w;
        if constexpr (VEC)
            w = f32x4_t{q[0], q[1], q[2], q[3]};
        else
            w = q[0];
        store_at(y, row_rsrc(y, N), N, toff, w);
    }
};

// group-wide reductions in a fixed order: a butterfly within each wave, then
// (G = BT) the wave partials combined as a balanced tree through LDS
template <int G>
__device__ __forceinline__ float group_max(float v, float* red) {
    v = wave_max(v);
    if constexpr (G == 64) {
        return v;
    } else {
        constexpr int NWV = G / 64;
        __syncthreads();  // red is reused by consecutive reductions
        if ((threadIdx.x & 63) == 0) red[wave_id()] = v;
        __syncthreads();
        float r[NWV];
#pragma unroll
        for (int w = 0; w < NWV; ++w) r[w] = red[w];
#pragma unroll
        for (int h = NWV / 2; h > 0; h >>= 1)
#pragma unroll
            for (int w = 0; w < h; ++w) r[w] = fmaxf(r[w], r[w + h]);
        return r[0];
    }
}
template <int G>
__device__ __forceinline__ float group_sum(float v, float* red) {
    v = wave_sum(v);
    if constexpr (G == 64) {
        return v;
    } else {
        constexpr int NWV = G / 64;
        __syncthreads();
        if ((threadIdx.x & 63) == 0) red[wave_id()] = v;
        __syncthreads();
        float r[NWV];
#pragma unroll
        for (int w = 0; w < NWV; ++w) r[w] = red[w];
#pragma unroll
        for (int h = NWV / 2; h > 0; h >>= 1)
#pragma unroll
            for (int w = 0; w < h; ++w) r[w] = r[w] + r[w + h];
        return r[0];
    }
}

// exponentials and sum of a held row (reference passes: max, exp and sum).
// Leaves e = fast_exp(x - max) in R.v for the part of the row that fills
// whole 16-float vectors (j < nv = N & ~15) and 0 elsewhere; the tail
// [nv, N), where the reference takes expf and divides by the sum instead of
// multiplying by its reciprocal, is this thread's et[] (its access there:
// RowRegs::tail_off), to be stored after R.  Each thread sums its own
// elements, then its tail ones.  FULL: N % 16 == 0, no tail (a kernel of
// its own, which carries neither the tail's extraction nor its expf).
template <bool FULL, int G, int ELEMS, bool VEC>
__device__ __forceinline__ void softmax_held(RowRegs<G, ELEMS, VEC>& R, const float* x, int N,
                                             int tid, float* red, float* mx_out, float* s_out,
                                             float (&et)[VEC ? 4 : 1]) {
    using RR = RowRegs<G, ELEMS, VEC>;
    const int nv = N & ~15;
    R.template load<true>(x, N, tid);
    float mx = -FLT_MAX;
#pragma unroll
    for (int k = 0; k < ELEMS; ++k) mx = ref_max(mx, R.v[k]);
    mx = group_max<G>(mx, red);
    if constexpr (FULL) {
#pragma unroll
        for (int i = 0; i < RR::W; ++i) et[i] = 0.0f;
    } else {
        R.tail(N, nv, tid, et);
    }
    // fast_exp clamps its argument to [-88, 88], so it is finite for every
    // element, pads included, and the select needs no branch
    float s = 0.0f;
#pragma unroll
    for (int a = 0; a < RR::NA; ++a)
#pragma unroll
        for (int i = 0; i < RR::W; ++i) {
            float& e = R.v[RR::W * a + i];
            const float f = fast_exp(e - mx);
            e = RR::elem(tid, a, i) < nv ? f : 0.0f;
            s += e;
        }
    if constexpr (!FULL) {
        const bool has_tail = RR::tail_off(N, nv, tid) != RR::TAIL_NONE;
#pragma unroll
        for (int i = 0; i < RR::W; ++i) {
            et[i] = expf(et[i] - mx);
            s += has_tail ? et[i] : 0.0f;
        }
    }
    *mx_out = mx;
    *s_out = group_sum<G>(s, red);
}

// row of this block: one per wave (G = 64, ROWS_PER_BLOCK rows) or one per block
template <int G>
__device__ __forceinline__ int held_row(int* tid) {
    if constexpr (G == 64) {
        *tid = threadIdx.x & 63;
        return blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
    } else {
        *tid = threadIdx.x;
        return blockIdx.x;
    }
}

template <int G, int ELEMS, bool VEC, bool FULL>
__global__ __launch_bounds__(G == 64 ? 64 * ROWS_PER_BLOCK : BT) void softmax_kernel(
    float* out, const float* in, int M, int N) {  // out may alias in
    __shared__ float red[G == 64 ? 1 : G / 64];
    int tid;
    const int row = held_row<G>(&tid);
    if (row >= M) return;  // whole wave (G = 64) or whole block
    RowRegs<G, ELEMS, VEC> R;
    float mx, s, pt[VEC ? 4 : 1];
    softmax_held<FULL>(R, in + (int64_t)row * N, N, tid, red, &mx, &s, pt);
    const float inv = 1.0f / s;
    float* y = out + (int64_t)row * N;
    R.store(y, N, tid, [&](float e) { return e * inv; });
    if constexpr (!FULL) {
#pragma unroll
        for (int i = 0; i < (VEC ? 4 : 1); ++i) pt[i] = pt[i] / s;
        R.store_tail(y, N, R.tail_off(N, N & ~15, tid), pt);  // after R's store of 0 there
    }
}

// ---- rows longer than a block holds: one BT-thread workgroup per row, the
// row streamed in chunks of LCH elements, LE per thread (16-byte accesses
// under the same conditions as the held rows, else single floats) ----
constexpr int LE = 16;          // elements per thread per chunk (its loads in flight)
constexpr int LCH = BT * LE;    // elements per chunk

template <bool VEC, int T = BT>
struct Chunk {
    static constexpr int W = VEC ? 4 : 1;
    static constexpr int NA = LE / W;
    float v[LE];
    // offset in the chunk of this thread's access a, element i (T threads,
    // T * LE elements); a chunk starts at a multiple of T * LE, so element j
    // of the row belongs to thread (VEC ? j / 4 : j) % T
    __device__ __forceinline__ static int off(int a, int i) {
        return VEC ? 4 * ((int)threadIdx.x + T * a) + i : (int)threadIdx.x + T * a;
    }
    // v[] = x[0 .. rem) of the chunk starting at x, pad past it (rem > 0;
    // with VEC rem % 4 == 0)
    __device__ __forceinline__ void load(const float* x, int rem, float pad) {
#pragma unroll
        for (int a = 0; a < NA; ++a) {
            const int o = off(a, 0);
            if constexpr (VEC) {
                f32x4_t q = {pad, pad, pad, pad};
                if (o < rem) q = *reinterpret_cast<const f32x4_t*>(x + o);
#pragma unroll
                for (int i = 0; i < 4; ++i) v[4 * a + i] = q[i];
            } else {
                v[a] = o < rem ? x[o] : pad;
            }
        }
    }
    __device__ __forceinline__ void store(float* y, int rem) const {
#pragma unroll
        for (int a = 0; a < NA; ++a) {
            const int o = off(a, 0);
            if (o < rem) {
                if constexpr (VEC) {
                    const f32x4_t q = {v[4 * a], v[4 * a + 1], v[4 * a + 2], v[4 * a + 3]};
                    *reinterpret_cast<f32x4_t*>(y + o) = q;
                } else {
                    y[o] = v[a];
                }
            }
        }
    }
    // f(offset in the chunk, value, inside the row)
    template <typename F>
    __device__ __forceinline__ void each(int rem, F&& f) {
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
            for (int i = 0; i < W; ++i) {
                const int o = off(a, i);
                f(o, v[W * a + i], o < rem);
            }
    }
};

// f(chunk start b, elements left rem) over the chunks of a row of N from b0
template <typename F>
__device__ __forceinline__ void chunks(int b0, int N, F&& f) {
    for (int64_t b = b0; b < N; b += LCH) f((int)b, (int)(N - b));
}

// The head of a long row, its first HEAD_CHUNKS chunks (65536 elements;
// every long row has all of them whole), stays on chip after the first read:
// chunks 0 and 1 in registers, chunks 2 and 3 in this thread's part of a
// dynamic LDS area (element k of chunk 2 + h at area[(h * LE + k) * BT +
// tid]: consecutive threads in consecutive banks, and no thread reads
// another's slots, so no barrier).  The later passes re-read only the rest
// of the row.  Every pass visits the head's elements in chunk order, each
// chunk in the order of Chunk::each, so sums are taken in the same order as
// over a streamed row.
constexpr int HEAD_CHUNKS = 4;
constexpr size_t HEAD_LDS = 2 * LE * BT * sizeof(float);  // 128 KiB
static_assert(HEAD_CHUNKS * LCH == MAX_BLOCK_CACHED, "long rows hold the whole head");

template <bool VEC>
struct Head {
    using C = Chunk<VEC>;
    C r[2];
    float* area;
    __device__ __forceinline__ explicit Head(float* lds) : area(lds + threadIdx.x) {}
    __device__ __forceinline__ float& slot(int h, int k) { return area[(h * LE + k) * BT]; }
    // offset in its chunk of this thread's element k
    __device__ __forceinline__ static int off(int k) { return C::off(k / C::W, k % C::W); }
    // loads the head, f(element index, value) over it in order
    template <typename F>
    __device__ __forceinline__ void load(const float* x, F&& f) {
        C c2, c3;
        r[0].load(x, LCH, 0.0f);
        r[1].load(x + LCH, LCH, 0.0f);
        c2.load(x + 2 * LCH, LCH, 0.0f);
        c3.load(x + 3 * LCH, LCH, 0.0f);
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int k = 0; k < LE; ++k) f(h * LCH + off(k), r[h].v[k]);
#pragma unroll
        for (int k = 0; k < LE; ++k) {
            f(2 * LCH + off(k), c2.v[k]);
            slot(0, k) = c2.v[k];
        }
#pragma unroll
        for (int k = 0; k < LE; ++k) {
            f(3 * LCH + off(k), c3.v[k]);
            slot(1, k) = c3.v[k];
        }
    }
    // f(element index, value&) over the head in order; with WB the LDS
    // values are written back
    template <bool WB, typename F>
    __device__ __forceinline__ void each(F&& f) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int k = 0; k < LE; ++k) f(h * LCH + off(k), r[h].v[k]);
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int k = 0; k < LE; ++k) {
                float v = slot(h, k);
                f((2 + h) * LCH + off(k), v);
                if constexpr (WB) slot(h, k) = v;
            }
    }
    // y = the head mapped chunk by chunk: f(chunk start, chunk) rewrites the
    // chunk's values, which are then stored
    template <typename F>
    __device__ __forceinline__ void map_store(float* y, F&& f) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            f(h * LCH, r[h]);
            r[h].store(y + h * LCH, LCH);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            C c;
#pragma unroll
            for (int k = 0; k < LE; ++k) c.v[k] = slot(h, k);
            f((2 + h) * LCH, c);
            c.store(y + (2 + h) * LCH, LCH);
        }
    }
};

// row max, then the sum of exp(x - max) (reference passes 1a and 1b); the
// head's exponentials are left in H (all of the head is in the vector part)
template <bool VEC>
__device__ __forceinline__ void long_row_stats(Head<VEC>& H, const float* x, int N, float* red,
                                               float* mx_out, float* s_out) {
    constexpr int B0 = HEAD_CHUNKS * LCH;
    const int nv = N & ~15;
    float mx = -FLT_MAX;
    H.load(x, [&](int, float v) { mx = ref_max(mx, v); });
    chunks(B0, N, [&](int b, int rem) {
        Chunk<VEC> C;
        C.load(x + b, rem, -FLT_MAX);
#pragma unroll
        for (int k = 0; k < LE; ++k) mx = ref_max(mx, C.v[k]);
    });
    mx = group_max<BT>(mx, red);
    float s = 0.0f;
    H.template each<true>([&](int, float& e) {
        e = fast_exp(e - mx);
        s += e;
    });
    chunks(B0, N, [&](int b, int rem) {
        Chunk<VEC> C;
        C.load(x + b, rem, 0.0f);
        C.each(rem, [&](int o, float e, bool in) { s += in ? row_exp(e - mx, b + o, nv) : 0.0f; });
    });
    *mx_out = mx;
    *s_out = group_sum<BT>(s, red);
}

template <bool VEC>
__global__ __launch_bounds__(BT) void softmax_long_kernel(float* out, const float* in, int N) {
    __shared__ float red[BT / 64];
    extern __shared__ float head_lds[];
    const float* x = in + (int64_t)blockIdx.x * N;
    float* y = out + (int64_t)blockIdx.x * N;
    const int nv = N & ~15;
    Head<VEC> H(head_lds);
    float mx, s;
    long_row_stats<VEC>(H, x, N, red, &mx, &s);
    const float inv = 1.0f / s;
    H.map_store(y, [&](int, Chunk<VEC>& c) {
#pragma unroll
        for (int k = 0; k < LE; ++k) c.v[k] *= inv;
    });
    chunks(HEAD_CHUNKS * LCH, N, [&](int b, int rem) {
        Chunk<VEC> C;
        C.load(x + b, rem, 0.0f);
        C.each(rem, [&](int o, float& e, bool) {
            e = row_norm(row_exp(e - mx, b + o, nv), inv, s, b + o, nv);
        });
        C.store(y + b, rem);
    });
}

// ---- layernorm ----
template <int G, int ELEMS, bool VEC, bool FULL>
__global__ __launch_bounds__(G == 64 ? 64 * ROWS_PER_BLOCK : BT) void layernorm_kernel(
    float* out, const float* in, const float* __restrict__ gamma,  // out may alias in
    const float* __restrict__ beta, int M, int N, float eps) {
    __shared__ float red[G == 64 ? 1 : G / 64];
    int tid;
    const int row = held_row<G>(&tid);
    if (row >= M) return;
    RowRegs<G, ELEMS, VEC> R;
    R.template load<false>(in + (int64_t)row * N, N, tid);
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < ELEMS; ++k) s += R.v[k];
    const float mean = group_sum<G>(s, red) / (float)N;
    float q = 0.0f;
    R.each(N, tid, [&](int, float& x, bool in) {
        const float d = x - mean;
        q = in ? __builtin_fmaf(d, d, q) : q;
    });
    const float var = group_sum<G>(q, red) / (float)N;
    const float inv_std = 1.0f / sqrtf(var + eps);
    using RR = RowRegs<G, ELEMS, VEC>;
    float* y = out + (int64_t)row * N;
    const __amdgpu_buffer_rsrc_t gs = RR::row_rsrc(gamma, N), bs = RR::row_rsrc(beta, N),
                                 ys = RR::row_rsrc(y, N);
    const uint32_t o0 = RR::fresh_base_off(tid);
    const uint32_t last = (uint32_t)(N - RR::W) * 4u;
#pragma unroll
    for (int a = 0; a < RR::NA; ++a) {
        if (RR::first(a) >= N) continue;  // the same for the whole group
        const uint32_t o = o0 + 4u * (uint32_t)RR::first(a), oc = o < last ? o : last;
        const typename RR::Access gq = RR::load_at(gamma, gs, oc), bq = RR::load_at(beta, bs, oc);
        typename RR::Access q;
        if constexpr (VEC) {
#pragma unroll
            for (int i = 0; i < 4; ++i) q[i] = __builtin_fmaf((R.v[4 * a + i] - mean) * inv_std, gq[i], bq[i]);
        } else {
            q = __builtin_fmaf((R.v[a] - mean) * inv_std, gq, bq);
        }
        RR::store_at(y, ys, N, o, q);  // nothing past the row
    }
}

// rows longer than a block holds: the reference's three passes (sum, sum of
// squared deviations, write), the head held on chip and the rest streamed
template <bool VEC>
__global__ __launch_bounds__(BT) void layernorm_long_kernel(float* out, const float* in,
                                                           const float* __restrict__ gamma,
                                                           const float* __restrict__ beta, int N,
                                                           float eps) {
    constexpr int B0 = HEAD_CHUNKS * LCH;
    __shared__ float red[BT / 64];
    extern __shared__ float head_lds[];
    const float* x = in + (int64_t)blockIdx.x * N;
    float* y = out + (int64_t)blockIdx.x * N;
    Head<VEC> H(head_lds);
    float s = 0.0f;
    H.load(x, [&](int, float v) { s += v; });
    chunks(B0, N, [&](int b, int rem) {
        Chunk<VEC> C;
        C.load(x + b, rem, 0.0f);
#pragma unroll
        for (int k = 0; k < LE; ++k) s += C.v[k];
    });
    const float mean = group_sum<BT>(s, red) / (float)N;
    float q = 0.0f;
    H.template each<false>([&](int, float& v) {
        const float d = v - mean;
        q = __builtin_fmaf(d, d, q);
    });
    chunks(B0, N, [&](int b, int rem) {
        Chunk<VEC> C;
        C.load(x + b, rem, 0.0f);
        C.each(rem, [&](int, float e, bool in) {
            const float d = e - mean;
            q = in ? __builtin_fmaf(d, d, q) : q;
        });
    });
    const float var = group_sum<BT>(q, red) / (float)N;
    const float inv_std = 1.0f / sqrtf(var + eps);
    auto write = [&](int b, int rem, Chunk<VEC>& C) {
        Chunk<VEC> G, B;
        G.load(gamma + b, rem, 0.0f);
        B.load(beta + b, rem, 0.0f);
#pragma unroll
        for (int k = 0; k < LE; ++k) C.v[k] = __builtin_fmaf((C.v[k] - mean) * inv_std, G.v[k], B.v[k]);
    };
    H.map_store(y, [&](int b, Chunk<VEC>& c) { write(b, LCH, c); });
    chunks(B0, N, [&](int b, int rem) {
        Chunk<VEC> C;
        C.load(x + b, rem, 0.0f);
        write(b, rem, C);
        C.store(y + b, rem);
    });
}

// ---- cross entropy: grad rows and per-row losses (row_loss[M]) ----
// A target outside [0, N) gives a NaN row loss and no onehot subtraction
// (the reference indexes out of bounds).  p[t] is recomputed from x[t] with
// the same operations as the row's own p (one cached load per row), and
// grad[t] is stored again after the row with the onehot subtracted (the
// same thread's later store to the same address wins).
template <int G, int ELEMS, bool VEC, bool FULL>
__global__ __launch_bounds__(G == 64 ? 64 * ROWS_PER_BLOCK : BT) void cross_entropy_kernel(
    const float* logits, const int32_t* __restrict__ targets,  // grad may alias logits
    float* grad, float* __restrict__ row_loss, int M, int N) {
    __shared__ float red[G == 64 ? 1 : G / 64];
    int tid;
    const int row = held_row<G>(&tid);
    if (row >= M) return;
    const float* x = logits + (int64_t)row * N;
    float* g = grad + (int64_t)row * N;
    const int t = targets[row];
    const bool valid = t >= 0 && t < N;
    // the thread whose elements include t stores its gradient; x[t] is read
    // (by every thread, a scalar load) before any store of this row (grad may
    // alias logits)
    const bool owner = valid && tid == (VEC ? (t >> 2) % G : t % G);
    const float xt = valid ? x[t] : 0.0f;
    RowRegs<G, ELEMS, VEC> R;
    float mx, s, ptl[VEC ? 4 : 1];
    softmax_held<FULL>(R, x, N, tid, red, &mx, &s, ptl);
    const int nv = N & ~15;
    const float inv = 1.0f / s;
    const float pt = row_norm(row_exp(xt - mx, t, nv), inv, s, t, nv);
    const float fm = (float)M;
#pragma unroll
    for (int i = 0; i < (VEC ? 4 : 1); ++i) ptl[i] = ptl[i] / s;
    // grad = p / M as the reference's division; for a power-of-two M the
    // product with 1/M (exact) is the same single rounding of p * 2^-k, bit
    // for bit, at a tenth of the instructions
    if ((M & (M - 1)) == 0) {
        const float rm = 1.0f / fm;
        R.store(g, N, tid, [&](float e) { return (e * inv) * rm; });
#pragma unroll
        for (int i = 0; i < (VEC ? 4 : 1); ++i) ptl[i] = ptl[i] * rm;
    } else {
        R.store(g, N, tid, [&](float e) { return (e * inv) / fm; });
#pragma unroll
        for (int i = 0; i < (VEC ? 4 : 1); ++i) ptl[i] = ptl[i] / fm;
    }
    if constexpr (!FULL) R.store_tail(g, N, R.tail_off(N, nv, tid), ptl);  // after R's store of 0 there
    if (owner) {
        // after this thread's own stores of g[t], through the same buffer path
        R.store1(g, N, (uint32_t)t * 4u, (pt - 1.0f) / fm);
        row_loss[row] = -logf(pt + 1e-10f);
    } else if (!valid && tid == 0) {
        row_loss[row] = __builtin_nanf("");
    }
}

template <bool VEC>
__global__ __launch_bounds__(BT) void cross_entropy_long_kernel(const float* logits,
                                                               const int32_t* targets, float* grad,
                                                               float* row_loss, int M, int N) {
    __shared__ float red[BT / 64];
    extern __shared__ float head_lds[];
    const int row = blockIdx.x;
    const float* x = logits + (int64_t)row * N;
    float* g = grad + (int64_t)row * N;
    const int nv = N & ~15;
    const int t = targets[row];
    const bool valid = t >= 0 && t < N;
    const bool owner = valid && (int)threadIdx.x == (VEC ? t >> 2 : t) % BT;  // Chunk's owner of t
    const float xt = valid ? x[t] : 0.0f;  // before any store of this row (grad may alias logits)
    Head<VEC> H(head_lds);
    float mx, s;
    long_row_stats<VEC>(H, x, N, red, &mx, &s);
    const float inv = 1.0f / s;
    const float fm = (float)M;
    const bool pow2 = (M & (M - 1)) == 0;  // exact product with 1/M, as in cross_entropy_kernel
    const float rm = 1.0f / fm;
    H.map_store(g, [&](int, Chunk<VEC>& c) {
#pragma unroll
        for (int k = 0; k < LE; ++k) c.v[k] = pow2 ? (c.v[k] * inv) * rm : (c.v[k] * inv) / fm;
    });
    chunks(HEAD_CHUNKS * LCH, N, [&](int b, int rem) {
        Chunk<VEC> C;
        C.load(x + b, rem, 0.0f);
        C.each(rem, [&](int o, float& e, bool) {
            const float p = row_norm(row_exp(e - mx, b + o, nv), inv, s, b + o, nv);
            e = pow2 ? p * rm : p / fm;
        });
        C.store(g + b, rem);
    });
    if (owner) {
        const float pt = row_norm(row_exp(xt - mx, t, nv), inv, s, t, nv);
        g[t] = (pt - 1.0f) / fm;  // after this thread's own store of g[t]
        row_loss[row] = -logf(pt + 1e-10f);
    } else if (!valid && threadIdx.x == 0) {
        row_loss[row] = __builtin_nanf("");
    }
}

// ---- few long rows: each row split into segments of SEG elements, one
// ST-thread workgroup per segment, in three launches (the reference's three
// passes), so that M rows fill M * ceil(N / SEG) workgroups instead of M.
// Launch 1 writes each segment's max (layernorm: its sum) to part1; launch 2
// reduces the row's part1 to the row max (mean) and writes each segment's
// sum of exponentials (squared deviations) to part2; launch 3 reduces both
// and writes the segment.  Every workgroup of a row reduces the row's
// partials with the same code in the same order, so all of them hold the
// same max and sum; results are deterministic (a row sum is taken within
// each segment, then over the segments in a fixed order).  The per-element
// arithmetic is the reference's, as in the other row kernels. ----
constexpr int ST = 256;       // threads per segment workgroup
constexpr int SEG = ST * LE;  // elements per segment

struct SegPos {
    int row, b, rem;  // row, segment start, elements from there to the row's end
};
__device__ __forceinline__ SegPos seg_pos(int N, int nseg) {
    SegPos p;
    p.row = (int)blockIdx.x / nseg;
    p.b = ((int)blockIdx.x - p.row * nseg) * SEG;
    p.rem = N - p.b;
    return p;
}
// a row's nseg partials reduced in a fixed order (thread i takes i, i + ST, ...)
__device__ __forceinline__ float parts_max(const float* part, int nseg, float* red) {
    float m = -FLT_MAX;
    for (int i = threadIdx.x; i < nseg; i += ST) m = ref_max(m, part[i]);
    return group_max<ST>(m, red);
}
__device__ __forceinline__ float parts_sum(const float* part, int nseg, float* red) {
    float s = 0.0f;
    for (int i = threadIdx.x; i < nseg; i += ST) s += part[i];
    return group_sum<ST>(s, red);
}

// launch 1: segment max (softmax, cross entropy) or sum (layernorm)
template <bool VEC, bool SUM>
__global__ __launch_bounds__(ST) void seg_pass1_kernel(const float* in, int N, int nseg,
                                                       float* __restrict__ part1) {
    __shared__ float red[ST / 64];
    const SegPos p = seg_pos(N, nseg);
    Chunk<VEC, ST> C;
    C.load(in + (int64_t)p.row * N + p.b, p.rem, SUM ? 0.0f : -FLT_MAX);
    float v = SUM ? 0.0f : -FLT_MAX;
#pragma unroll
    for (int k = 0; k < LE; ++k) v = SUM ? v + C.v[k] : ref_max(v, C.v[k]);
    v = SUM ? group_sum<ST>(v, red) : group_max<ST>(v, red);
    if (threadIdx.x == 0) part1[blockIdx.x] = v;
}

// launch 2: the segment's sum of exponentials at the row max (SUM = false) or
// of squared deviations from the row mean (SUM = true, layernorm)
template <bool VEC, bool SUM>
__global__ __launch_bounds__(ST) void seg_pass2_kernel(const float* in, int N, int nseg,
                                                       const float* __restrict__ part1,
                                                       float* __restrict__ part2) {
    __shared__ float red[ST / 64];
    const SegPos p = seg_pos(N, nseg);
    const int nv = N & ~15;
    Chunk<VEC, ST> C;
    C.load(in + (int64_t)p.row * N + p.b, p.rem, 0.0f);
    const float* pr = part1 + (int64_t)p.row * nseg;
    const float ref = SUM ? parts_sum(pr, nseg, red) / (float)N : parts_max(pr, nseg, red);
    float s = 0.0f;
    C.each(p.rem, [&](int o, float e, bool in) {
        if constexpr (SUM) {
            const float d = e - ref;
            s = in ? __builtin_fmaf(d, d, s) : s;
        } else {
            s += in ? row_exp(e - ref, p.b + o, nv) : 0.0f;
        }
    });
    s = group_sum<ST>(s, red);
    if (threadIdx.x == 0) part2[blockIdx.x] = s;
}

// launch 3, softmax
template <bool VEC>
__global__ __launch_bounds__(ST) void softmax_seg_write_kernel(float* out, const float* in, int N,
                                                               int nseg, const float* __restrict__ part1,
                                                               const float* __restrict__ part2) {
    __shared__ float red[ST / 64];
    const SegPos p = seg_pos(N, nseg);
    const int nv = N & ~15;
    Chunk<VEC, ST> C;
    C.load(in + (int64_t)p.row * N + p.b, p.rem, 0.0f);
    const float mx = parts_max(part1 + (int64_t)p.row * nseg, nseg, red);
    const float s = parts_sum(part2 + (int64_t)p.row * nseg, nseg, red);
    const float inv = 1.0f / s;
    C.each(p.rem, [&](int o, float& e, bool) {
        e = row_norm(row_exp(e - mx, p.b + o, nv), inv, s, p.b + o, nv);
    });
    C.store(out + (int64_t)p.row * N + p.b, p.rem);
}

// launch 3, layernorm
template <bool VEC>
__global__ __launch_bounds__(ST) void layernorm_seg_write_kernel(
    float* out, const float* in, const float* __restrict__ gamma, const float* __restrict__ beta,
    int N, float eps, int nseg, const float* __restrict__ part1, const float* __restrict__ part2) {
    __shared__ float red[ST / 64];
    const SegPos p = seg_pos(N, nseg);
    Chunk<VEC, ST> C, G, B;
    C.load(in + (int64_t)p.row * N + p.b, p.rem, 0.0f);
    G.load(gamma + p.b, p.rem, 0.0f);
    B.load(beta + p.b, p.rem, 0.0f);
    const float mean = parts_sum(part1 + (int64_t)p.row * nseg, nseg, red) / (float)N;
    const float var = parts_sum(part2 + (int64_t)p.row * nseg, nseg, red) / (float)N;
    const float inv_std = 1.0f / sqrtf(var + eps);
#pragma unroll
    for (int k = 0; k < LE; ++k) C.v[k] = __builtin_fmaf((C.v[k] - mean) * inv_std, G.v[k], B.v[k]);
    C.store(out + (int64_t)p.row * N + p.b, p.rem);
}

// launch 3, cross entropy: the segment's gradient; the workgroup whose
// segment holds the target also writes the row loss
template <bool VEC>
__global__ __launch_bounds__(ST) void cross_entropy_seg_write_kernel(
    const float* logits, const int32_t* targets, float* grad, float* row_loss, int M, int N,
    int nseg, const float* __restrict__ part1, const float* __restrict__ part2) {
    __shared__ float red[ST / 64];
    const SegPos p = seg_pos(N, nseg);
    const int nv = N & ~15;
    const float* x = logits + (int64_t)p.row * N;
    float* g = grad + (int64_t)p.row * N;
    const int t = targets[p.row];
    const bool valid = t >= 0 && t < N;
    const bool mine = valid && t >= p.b && t < p.b + SEG;  // the target is in this segment
    // the thread whose element t is (Chunk's layout from the segment start)
    const bool owner = mine && (int)threadIdx.x == (VEC ? (t - p.b) >> 2 : t - p.b) % ST;
    Chunk<VEC, ST> C;
    C.load(x + p.b, p.rem, 0.0f);
    const float xt = mine ? x[t] : 0.0f;  // before this workgroup's stores (grad may alias logits)
    const float mx = parts_max(part1 + (int64_t)p.row * nseg, nseg, red);
    const float s = parts_sum(part2 + (int64_t)p.row * nseg, nseg, red);
    const float inv = 1.0f / s;
    const float fm = (float)M;
    const bool pow2 = (M & (M - 1)) == 0;  // exact product with 1/M, as in cross_entropy_kernel
    const float rm = 1.0f / fm;
    C.each(p.rem, [&](int o, float& e, bool) {
        const float pv = row_norm(row_exp(e - mx, p.b + o, nv), inv, s, p.b + o, nv);
        e = pow2 ? pv * rm : pv / fm;
    });
    C.store(g + p.b, p.rem);
    if (owner) {
        const float pt = row_norm(row_exp(xt - mx, t, nv), inv, s, t, nv);
        g[t] = (pt - 1.0f) / fm;  // after this thread's own store of g[t]
        row_loss[p.row] = -logf(pt + 1e-10f);
    } else if (!valid && p.b == 0 && threadIdx.x == 0) {
        row_loss[p.row] = __builtin_nanf("");
    }
}

// loss = sum of row_loss in a fixed order / M (one workgroup of RT threads).
// Thread i adds rows i, i + RT, i + 2 RT, ..., RU of them per round with all
// RU loads in flight together (a loop of dependent load-add steps waited out
// one memory latency per row: ~25 us at M = 16384); then a butterfly within
// each wave and a fixed tree over the wave sums.
constexpr int RT = 1024, RU = 16;
__global__ __launch_bounds__(RT) void cross_entropy_reduce_kernel(const float* __restrict__ row_loss,
                                                                  float* __restrict__ loss, int M) {
    __shared__ float part[RT / 64];
    float s = 0.0f;
    // 64-bit row indices: i0 + RT * u would overflow int for M near INT_MAX
    for (int64_t i0 = threadIdx.x; i0 < M; i0 += RT * RU) {
        float v[RU];
#pragma unroll
        for (int u = 0; u < RU; ++u) {
            const int64_t i = i0 + (int64_t)RT * u;
            v[u] = i < M ? row_loss[i] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < RU; ++u) s += v[u];
    }
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        float w[RT / 64];
#pragma unroll
        for (int i = 0; i < RT / 64; ++i) w[i] = part[i];
#pragma unroll
        for (int h = RT / 128; h > 0; h >>= 1)
#pragma unroll
            for (int i = 0; i < h; ++i) w[i] = w[i] + w[i + h];
        loss[0] = w[0] / (float)M;
    }
}

// Launch plan for a row length: the smallest register-held size that fits
// (one wave per row up to MAX_CACHED, one BT-thread block per row up to
// MAX_BLOCK_CACHED), 16-byte accesses when every row is 16-byte aligned, the
// no-tail softmax when N % 16 == 0.  f(G, ELEMS, VEC, FULL) returns the
// launch status; rows past MAX_BLOCK_CACHED are left to the caller
// (streaming kernels).
template <int G, int E, typename F>
hipError_t with_flags(bool vec, bool full, F&& f) {
    using std::integral_constant;
    using g = integral_constant<int, G>;
    using e = integral_constant<int, E>;
    if constexpr (E < 4) {
        return full ? f(g{}, e{}, integral_constant<bool, false>{}, integral_constant<bool, true>{})
                    : f(g{}, e{}, integral_constant<bool, false>{}, integral_constant<bool, false>{});
    } else {
        if (vec)
            return full ? f(g{}, e{}, integral_constant<bool, true>{}, integral_constant<bool, true>{})
                        : f(g{}, e{}, integral_constant<bool, true>{}, integral_constant<bool, false>{});
        return full ? f(g{}, e{}, integral_constant<bool, false>{}, integral_constant<bool, true>{})
                    : f(g{}, e{}, integral_constant<bool, false>{}, integral_constant<bool, false>{});
    }
}
template <typename F>
hipError_t by_size(int N, bool vec, F&& f) {
    const bool full = N % 16 == 0;
    if (N <= 64) return with_flags<64, 1>(vec, full, f);
    if (N <= 128) return with_flags<64, 2>(vec, full, f);
    if (N <= 256) return with_flags<64, 4>(vec, full, f);
    if (N <= 512) return with_flags<64, 8>(vec, full, f);
    if (N <= 1024) return with_flags<64, 16>(vec, full, f);
    if (N <= 2048) return with_flags<64, 32>(vec, full, f);
    if (N <= MAX_CACHED) return with_flags<64, 64>(vec, full, f);
    if (N <= 8192) return with_flags<BT, 8>(vec, full, f);
    if (N <= 16384) return with_flags<BT, 16>(vec, full, f);
    if (N <= 32768) return with_flags<BT, 32>(vec, full, f);
    return with_flags<BT, MAX_BLOCK_CACHED / BT>(vec, full, f);
}

bool rows_vec4(int N, std::initializer_list<const void*> ptrs) {
    if (N % 4 != 0) return false;
    for (const void* p : ptrs)
        if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return false;
    return true;
}

template <int G>
unsigned row_blocks(int M) {
    return G == 64 ? (unsigned)((M + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK) : (unsigned)M;
}

// Few long rows: each row split over workgroups (three launches) when one
// workgroup per row would leave most CUs idle streaming it.  Measured: the
// three launches cost ~10 us together, so rows the block-held kernels take
// (N <= 65536) stay there (8 x 8192: 4.0 vs 10.8 us; 16 x 32000: 7.2 vs
// 11.4 us), while longer rows gain (1 x 128256: 30.2 -> 11.2 us; 64 x 128256:
// 34.6 -> 25.1 us) up to 64 rows (128 x 128256: 43.3 vs 46.3 us).
constexpr int SPLIT_MAX_ROWS = 64;
bool split_rows(int M, int N) { return M <= SPLIT_MAX_ROWS && N > MAX_BLOCK_CACHED; }

// launches 1 and 2 of a split row op; write(vec, grid, part1, part2) issues
// launch 3.  The partials (2 M ceil(N / SEG) floats) live in the stream's
// workspace.
template <typename W>
hipError_t launch_split(int M, int N, bool vec, bool layer, const float* x, hipStream_t s, W&& write) {
    const int nseg = (N + SEG - 1) / SEG;
    void* ws = nullptr;
    hipError_t e = stream_workspace(2 * (size_t)M * (size_t)nseg * sizeof(float), s, &ws);
    if (e != hipSuccess) return e;
    float* part1 = static_cast<float*>(ws);
    float* part2 = part1 + (size_t)M * (size_t)nseg;
    const dim3 grid((unsigned)(M * nseg)), blk(ST);
    if (vec) {
        if (layer) {
            hipLaunchKernelGGL((seg_pass1_kernel<true, true>), grid, blk, 0, s, x, N, nseg, part1);
            hipLaunchKernelGGL((seg_pass2_kernel<true, true>), grid, blk, 0, s, x, N, nseg, part1, part2);
        } else {
            hipLaunchKernelGGL((seg_pass1_kernel<true, false>), grid, blk, 0, s, x, N, nseg, part1);
            hipLaunchKernelGGL((seg_pass2_kernel<true, false>), grid, blk, 0, s, x, N, nseg, part1, part2);
        }
    } else {
        if (layer) {
            hipLaunchKernelGGL((seg_pass1_kernel<false, true>), grid, blk, 0, s, x, N, nseg, part1);
            hipLaunchKernelGGL((seg_pass2_kernel<false, true>), grid, blk, 0, s, x, N, nseg, part1, part2);
        } else {
            hipLaunchKernelGGL((seg_pass1_kernel<false, false>), grid, blk, 0, s, x, N, nseg, part1);
            hipLaunchKernelGGL((seg_pass2_kernel<false, false>), grid, blk, 0, s, x, N, nseg, part1, part2);
        }
    }
    if ((e = hipGetLastError()) != hipSuccess) return e;
    write(vec, grid, nseg, part1, part2);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_softmax(float* out, const float* in, int M, int N, hipStream_t s) {
    if (M <= 0 || N <= 0) return hipSuccess;  // no rows, or rows with nothing to load
    if (split_rows(M, N)) {
        return launch_split(M, N, rows_vec4(N, {out, in}), false, in, s,
                            [&](bool vec, dim3 grid, int nseg, const float* p1, const float* p2) {
                                if (vec)
                                    hipLaunchKernelGGL(softmax_seg_write_kernel<true>, grid, dim3(ST), 0, s,
                                                       out, in, N, nseg, p1, p2);
                                else
                                    hipLaunchKernelGGL(softmax_seg_write_kernel<false>, grid, dim3(ST), 0, s,
                                                       out, in, N, nseg, p1, p2);
                            });
    }
    if (N > MAX_BLOCK_CACHED) {
        if (rows_vec4(N, {out, in}))
            hipLaunchKernelGGL(softmax_long_kernel<true>, dim3(M), dim3(BT), HEAD_LDS, s, out, in, N);
        else
            hipLaunchKernelGGL(softmax_long_kernel<false>, dim3(M), dim3(BT), HEAD_LDS, s, out, in, N);
        return hipGetLastError();
    }
    return by_size(N, rows_vec4(N, {out, in}), [&](auto g, auto e, auto v, auto f) {
        constexpr int G = decltype(g)::value;
        hipLaunchKernelGGL((softmax_kernel<G, decltype(e)::value, decltype(v)::value, decltype(f)::value>),
                           dim3(row_blocks<G>(M)), dim3(G == 64 ? 64 * ROWS_PER_BLOCK : BT), 0, s,
                           out, in, M, N);
        return hipGetLastError();
    });
}

hipError_t launch_layernorm(float* out, const float* in, const float* gamma, const float* beta,
                            int M, int N, float eps, hipStream_t s) {
    if (M <= 0 || N <= 0) return hipSuccess;
    if (split_rows(M, N)) {
        return launch_split(M, N, rows_vec4(N, {out, in, gamma, beta}), true, in, s,
                            [&](bool vec, dim3 grid, int nseg, const float* p1, const float* p2) {
                                if (vec)
                                    hipLaunchKernelGGL(layernorm_seg_write_kernel<true>, grid, dim3(ST), 0,
                                                       s, out, in, gamma, beta, N, eps, nseg, p1, p2);
                                else
                                    hipLaunchKernelGGL(layernorm_seg_write_kernel<false>, grid, dim3(ST), 0,
                                                       s, out, in, gamma, beta, N, eps, nseg, p1, p2);
                            });
    }
    if (N > MAX_BLOCK_CACHED) {
        if (rows_vec4(N, {out, in, gamma, beta}))
            hipLaunchKernelGGL(layernorm_long_kernel<true>, dim3(M), dim3(BT), HEAD_LDS, s, out, in, gamma,
                               beta, N, eps);
        else
            hipLaunchKernelGGL(layernorm_long_kernel<false>, dim3(M), dim3(BT), HEAD_LDS, s, out, in, gamma,
                               beta, N, eps);
        return hipGetLastError();
    }
    return by_size(N, rows_vec4(N, {out, in, gamma, beta}), [&](auto g, auto e, auto v, auto) {
        constexpr int G = decltype(g)::value;
        hipLaunchKernelGGL((layernorm_kernel<G, decltype(e)::value, decltype(v)::value, false>),
                           dim3(row_blocks<G>(M)), dim3(G == 64 ? 64 * ROWS_PER_BLOCK : BT), 0, s,
                           out, in, gamma, beta, M, N, eps);
        return hipGetLastError();
    });
}

hipError_t launch_cross_entropy(const float* logits, const int32_t* targets, float* grad,
                                float* loss, float* row_loss, int M, int N, hipStream_t s) {
    hipError_t e = hipSuccess;
    if (M > 0 && N <= 0) return hipErrorInvalidValue;  // a target has no row to index
    if (M > 0) {
        if (split_rows(M, N)) {
            e = launch_split(M, N, rows_vec4(N, {logits, grad}), false, logits, s,
                             [&](bool vec, dim3 grid, int nseg, const float* p1, const float* p2) {
                                 if (vec)
                                     hipLaunchKernelGGL(cross_entropy_seg_write_kernel<true>, grid, dim3(ST),
                                                        0, s, logits, targets, grad, row_loss, M, N, nseg,
                                                        p1, p2);
                                 else
                                     hipLaunchKernelGGL(cross_entropy_seg_write_kernel<false>, grid, dim3(ST),
                                                        0, s, logits, targets, grad, row_loss, M, N, nseg,
                                                        p1, p2);
                             });
        } else if (N > MAX_BLOCK_CACHED) {
            if (rows_vec4(N, {logits, grad}))
                hipLaunchKernelGGL(cross_entropy_long_kernel<true>, dim3(M), dim3(BT), HEAD_LDS, s, logits,
                                   targets, grad, row_loss, M, N);
            else
                hipLaunchKernelGGL(cross_entropy_long_kernel<false>, dim3(M), dim3(BT), HEAD_LDS, s, logits,
                                   targets, grad, row_loss, M, N);
            e = hipGetLastError();
        } else {
            e = by_size(N, rows_vec4(N, {logits, grad}), [&](auto g, auto el, auto v, auto f) {
                constexpr int G = decltype(g)::value;
                hipLaunchKernelGGL((cross_entropy_kernel<G, decltype(el)::value, decltype(v)::value,
                                                         decltype(f)::value>),
                                   dim3(row_blocks<G>(M)), dim3(G == 64 ? 64 * ROWS_PER_BLOCK : BT), 0,
                                   s, logits, targets, grad, row_loss, M, N);
                return hipGetLastError();
            });
        }
    }
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(cross_entropy_reduce_kernel, dim3(1), dim3(RT), 0, s, row_loss, loss, M);
    return hipGetLastError();
}

}  // namespace jh
