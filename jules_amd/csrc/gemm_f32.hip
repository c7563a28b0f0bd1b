// gemm_f32.hip - fp32 fused GEMM + bias + activation for gfx950.
//
// Semantics follow the reference's tiled AVX-512 kernel
// (include/jules/Kernel/FusedKernels.h:378-458, bias epilogue :308-313):
// every output is ONE sequential fma chain over k = 0..K-1 starting from 0
// (the reference reloads the stored partial sum per K tile and keeps chaining,
// :401-406), followed by + bias[j] and the vector-path activation.  Each thread
// owns a TM x TN block of outputs and walks k in order, so the GPU reproduces
// those bits exactly; that rules out split-K and MFMA (whose internal
// accumulation order differs) for this dtype.  Parallelism comes from output
// tiles only.
//
// Data path: A and B tiles are staged through LDS (A transposed to k-major so
// a thread reads its TM rows as one vector), one barrier pair per BK slice.
// The global loads of slice k+1 are issued into registers before slice k is
// computed, so their latency is paid once per launch, not once per slice.
// The K tail is handled by a uniform trip count, never by zero padding (an
// extra fma(0, b, acc) could turn a -0 partial sum into +0).
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"
#include "tiles.hpp"

namespace jh {
namespace {

template <int BM, int BN, int BK, int TM, int TN, int ACT>
__global__ __launch_bounds__((BM / TM) * (BN / TN)) void gemm_f32_kernel(
    const float* __restrict__ A, const float* __restrict__ B, const float* __restrict__ bias,
    float* __restrict__ C, int M, int N, int K) {
    constexpr int TX = BN / TN;          // threads along N
    constexpr int NT = (BM / TM) * TX;   // threads per block
    __shared__ float As[BK][BM + 4];     // k-major copy of the A tile
    __shared__ float Bs[BK][BN + 4];

    const int tid = threadIdx.x;
    const int tx = tid % TX, ty = tid / TX;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

    float acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = 0.0f;

    constexpr int PA = (BM * BK + NT - 1) / NT;  // A elements per thread per slice
    constexpr int PB = (BK * BN + NT - 1) / NT;
    float ra[PA], rb[PB];
    auto gload = [&](int k0) {
        const int kc = min(BK, K - k0);
#pragma unroll
        for (int p = 0; p < PA; ++p) {
            const int e = tid + p * NT;
            const int m = e / BK, k = e % BK;
            ra[p] = (e < BM * BK && m0 + m < M && k < kc) ? A[(int64_t)(m0 + m) * K + k0 + k] : 0.0f;
        }
#pragma unroll
        for (int p = 0; p < PB; ++p) {
            const int e = tid + p * NT;
            const int k = e / BN, n = e % BN;
            rb[p] = (e < BK * BN && k < kc && n0 + n < N) ? B[(int64_t)(k0 + k) * N + n0 + n] : 0.0f;
        }
    };
    auto sstore = [&]() {
#pragma unroll
        for (int p = 0; p < PA; ++p) {
            const int e = tid + p * NT;
            if (e < BM * BK) As[e % BK][e / BK] = ra[p];
        }
#pragma unroll
        for (int p = 0; p < PB; ++p) {
            const int e = tid + p * NT;
            if (e < BK * BN) Bs[e / BN][e % BN] = rb[p];
        }
    };

    if (K > 0) gload(0);
    for (int k0 = 0; k0 < K; k0 += BK) {
        const int kc = min(BK, K - k0);
        sstore();
        __syncthreads();
        if (k0 + BK < K) gload(k0 + BK);
#pragma unroll 8
        for (int k = 0; k < kc; ++k) {
            float a[TM], b[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) a[i] = As[k][ty * TM + i];
#pragma unroll
            for (int j = 0; j < TN; ++j) b[j] = Bs[k][tx * TN + j];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int m = m0 + ty * TM + i;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int n = n0 + tx * TN + j;
            if (n >= N) continue;
            float v = acc[i][j];
            if (bias) v = v + bias[n];
            C[(int64_t)m * N + n] = activate<ACT>(v);
        }
    }
}

// Small problems (C1: 512^3): one wave per SIMD is all the outputs give at
// 2x2 per thread, and then the LDS reads of both operands (four values per
// four fmas, at most one read per ~30 cycles per wave) set the pace.  The
// row kernel instead gives a wave RW rows x 64 columns, lane = column, and
// stages the workgroup's RW*RWV rows of A in LDS once (K <= kF32RowsMaxK),
// read back as broadcasts (every lane the same address, one ds_read_b128 per
// row per four k).  Every output is still one fma chain over k = 0..K-1 in
// order.
constexpr int RWV = kF32RowsWaves;     // waves per workgroup (4 x RW rows x 64 columns)

// ---- row kernel: B streamed through an LDS ring by LDS DMA ----
// The B column block reaches LDS by LDS DMA through a ring of RD_NST stages of
// RD_KG k-rows, so the bytes in flight are not bounded by the wave's
// registers, and the workgroup's four waves share each B row (a register
// ring that each wave filled with its own loads ran C1 in 18.6 us, g2 in 6.7
// and 300x7x1500 in 30.2 against 16.0 / 5.7 / 24.9 us here).  The
// LDS reads (A as a broadcast b128 per row, B as two read2 per group of 4 k) run
// RD_PD groups ahead; they are inline asm with explicit waits (through
// builtins the compiler drains every DMA in flight before any LDS read).
// PIECE = 16 (N % 4 == 0 and B 16-byte aligned): a copy instruction moves 4
// rows of 64 columns.  PIECE = 4 (any N, B 4-byte aligned): one row per
// instruction, four times the instructions for the same bytes.
// At C1 (512^3): 16.0 us against 18.6 us for the register ring; g1 12.8 vs
// 17.0, g3 9.0 vs 11.9 (32-row stages with 6 stages: 17.6 / 14.8 / 10.2).
constexpr int RD_KG = 64;   // k rows per ring stage (16 KiB of B)
constexpr int RD_NST = 4;   // ring stages
constexpr int RD_PD = 3;    // groups of 4 k whose LDS reads are in flight
template <int I, int N, typename F>
__device__ __forceinline__ void static_for_f(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for_f<I + 1, N>(f);
    }
}
typedef __attribute__((address_space(3))) void lds_void_f;

template <int OFF>
__device__ __forceinline__ float rd_f32(uint32_t a) {
    float v;
    asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(v) : "v"(a), "n"(OFF) : "memory");
    return v;
}
typedef __attribute__((ext_vector_type(2))) float f32x2_t;
// two dwords 256 * O0 and 256 * O1 bytes past a (B rows O0 and O1 of a group)
template <int O0, int O1>
__device__ __forceinline__ f32x2_t rd_f32x2_st64(uint32_t a) {
    f32x2_t v;
    asm volatile("ds_read2st64_b32 %0, %1 offset0:%2 offset1:%3" : "=v"(v) : "v"(a), "n"(O0), "n"(O1) : "memory");
    return v;
}
template <int OFF>
__device__ __forceinline__ f32x4_t rd_f128(uint32_t a) {
    f32x4_t v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(a), "n"(OFF) : "memory");
    return v;
}

// Waits until at most N LDS reads are outstanding; the group's operands pass
// through the asm, so no fma that uses them is scheduled above the wait.
template <int N, int RW>
__device__ __forceinline__ void rd_wait(f32x4_t (&a)[RW], f32x2_t (&b)[2]) {
    static_assert(N >= 0 && N <= 15, "lgkmcnt is a 4-bit count");
    if constexpr (RW == 1)
        asm volatile("s_waitcnt lgkmcnt(%3)" : "+v"(a[0]), "+v"(b[0]), "+v"(b[1]) : "n"(N) : "memory");
    else
        asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(a[0]), "+v"(a[1]), "+v"(b[0]), "+v"(b[1]) : "n"(N) : "memory");
}

template <int ACT, int RW, int PIECE>
__global__ __launch_bounds__(64 * RWV) void gemm_f32_rowsdma_kernel(
    const float* __restrict__ A, const float* __restrict__ B, const float* __restrict__ bias,
    float* __restrict__ C, int M, int N, int K) {
    extern __shared__ __attribute__((aligned(16))) float sdyn[];  // ring [RD_NST][RD_KG][64], then A [RW*RWV][Kp]
    float* sB = sdyn;
    float* sA = sdyn + RD_NST * RD_KG * 64;
    const int Kp = (K + 3) & ~3;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = blockIdx.x * 64;
    const int n = n0 + lane;
    const int mb = blockIdx.y * RW * RWV;
    const int nst = (K + RD_KG - 1) / RD_KG;

    // stage rows mb .. mb + RW*RWV - 1 of A (rows past M repeat row M-1):
    // the rows unrolled, so a thread's loads of all of them are in flight
    // together (one load, its wait and its LDS store at a time took a memory
    // latency per element), 16-byte pieces when every row is 16-byte aligned
    constexpr int AR = RW * RWV;
    const float* arow[AR];
#pragma unroll
    for (int r = 0; r < AR; ++r) arow[r] = A + (int64_t)min(mb + r, M - 1) * K;
    if ((K & 3) == 0 && (reinterpret_cast<uintptr_t>(A) & 15) == 0) {
        for (int c = threadIdx.x; 4 * c < K; c += 64 * RWV) {
            f32x4_t v[AR];
#pragma unroll
            for (int r = 0; r < AR; ++r) v[r] = *reinterpret_cast<const f32x4_t*>(arow[r] + 4 * c);
#pragma unroll
            for (int r = 0; r < AR; ++r) *reinterpret_cast<f32x4_t*>(sA + r * Kp + 4 * c) = v[r];
        }
    } else {
        for (int k = threadIdx.x; k < K; k += 64 * RWV) {
            float v[AR];
#pragma unroll
            for (int r = 0; r < AR; ++r) v[r] = arow[r][k];
#pragma unroll
            for (int r = 0; r < AR; ++r) sA[r * Kp + k] = v[r];
        }
    }
    __syncthreads();

    // stage s of B: rows [RD_KG s, RD_KG (s + 1)) x columns [n0, n0 + 64) in
    // CPW instructions per wave.  PIECE 16: instruction i moves rows 4i ..
    // 4i+3, lane l row 4i + l/16, columns n0 + 4(l%16) .. +3.  PIECE 4:
    // instruction i moves row i, lane l column n0 + l.  The buffer covers the
    // stage's rows that exist (none past the last stage: no traffic), so every
    // call issues CPW instructions and the wait counts are constants.  Columns
    // past N read the next row (or 0 past the end): they only feed outputs
    // that are not stored.
    static_assert(PIECE == 16 || PIECE == 4, "16- or 4-byte copy pieces");
    constexpr int RPI = PIECE / 4;             // B rows per copy instruction
    constexpr int CPW = RD_KG / RPI / RWV;     // copy instructions per wave per stage
    auto copy_stage = [&](int s) {
        const bool live = s < nst;
        const int rows = live ? min(RD_KG, K - RD_KG * s) : 0;
        const __amdgpu_buffer_rsrc_t src = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(B) + (int64_t)RD_KG * (live ? s : 0) * N, 0, (uint32_t)rows * (uint32_t)N * 4u,
            0x00020000);
#pragma unroll
        for (int p = 0; p < CPW; ++p) {
            const int i = CPW * wave + p;
            const uint32_t row = (uint32_t)(RPI * i + (PIECE == 16 ? (lane >> 4) : 0));
            const uint32_t c = (uint32_t)(n0 + (PIECE == 16 ? 4 * (lane & 15) : lane));
            const uint32_t vo = (row * (uint32_t)N + c) * 4u;
            lds_void_f* dst = (lds_void_f*)(sB + ((s % RD_NST) * RD_KG + RPI * i) * 64);
            if constexpr (PIECE == 16)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(src, dst, 16, vo, 0, 0, 0);
            else
                __builtin_amdgcn_raw_ptr_buffer_load_lds(src, dst, 4, vo, 0, 0, 0);
        }
    };

    float acc[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) acc[r] = 0.0f;
    const uint32_t a0 = (uint32_t)(uintptr_t)(sA + wave * RW * Kp);
    const uint32_t b0 = (uint32_t)(uintptr_t)(sB + lane);

#pragma unroll
    for (int p = 0; p < RD_NST - 1; ++p) copy_stage(p);
    for (int s = 0; s < nst; ++s) {
        // this wave's pieces of stage s have landed once the CPW (RD_NST - 2)
        // instructions of the later stages are all that remain; the barrier
        // makes every wave's pieces visible and ends every wave's reads of
        // stage s - 1, whose slot the next copy reuses
        static_assert(CPW * (RD_NST - 2) <= 63, "vmcnt is a 6-bit count");
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(CPW * (RD_NST - 2)) : "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        copy_stage(s + RD_NST - 1);
        const int kv = min(RD_KG, K - RD_KG * s);   // k rows of this stage
        const int k0 = RD_KG * s;
        const uint32_t bs = b0 + (uint32_t)((s % RD_NST) * RD_KG * 64 * 4);
        const int ng = kv >> 2;
        // groups of 4 k: A as one b128 per row, B as two ds_read2st64_b32 (rows
        // 0-1 and 2-3 of the group, 256 bytes apart); a ring of RD_PD groups of
        // reads in flight.  The pairs stay whole until their wait, so no copy of
        // a register still being filled is scheduled before it.
        f32x4_t a[RD_PD][RW];
        f32x2_t b[RD_PD][2];  // B rows 0-1 and 2-3 of the group
        auto rd = [&](int g, int slot) {
#pragma unroll
            for (int r = 0; r < RW; ++r) a[slot][r] = rd_f128<0>(a0 + (uint32_t)((r * Kp + k0 + 4 * g) * 4));
            const uint32_t bg = bs + (uint32_t)(4 * g * 64 * 4);
            b[slot][0] = rd_f32x2_st64<0, 1>(bg);
            b[slot][1] = rd_f32x2_st64<2, 3>(bg);
        };
        if (ng == RD_KG / 4) {
            // a full stage: fully unrolled, compile-time ring slots and waits
            constexpr int NG = RD_KG / 4;
            static_for_f<0, RD_PD>([&](auto ic) { rd(decltype(ic)::value, decltype(ic)::value); });
            static_for_f<0, NG>([&](auto ic) {
                constexpr int g = decltype(ic)::value, slot = g % RD_PD;
                constexpr int later = (g + RD_PD - 1 < NG ? RD_PD - 1 : NG - 1 - g);  // groups read after g
                rd_wait<later * (RW + 2), RW>(a[slot], b[slot]);
#pragma unroll
                for (int r = 0; r < RW; ++r) {
                    acc[r] = __builtin_fmaf(a[slot][r].x, b[slot][0].x, acc[r]);
                    acc[r] = __builtin_fmaf(a[slot][r].y, b[slot][0].y, acc[r]);
                    acc[r] = __builtin_fmaf(a[slot][r].z, b[slot][1].x, acc[r]);
                    acc[r] = __builtin_fmaf(a[slot][r].w, b[slot][1].y, acc[r]);
                }
                if constexpr (g + RD_PD < NG) rd(g + RD_PD, slot);
            });
        } else {
            // the last, partial stage: one group at a time
            for (int g = 0; g < ng; ++g) {
                rd(g, 0);
                rd_wait<0, RW>(a[0], b[0]);
#pragma unroll
                for (int r = 0; r < RW; ++r) {
                    acc[r] = __builtin_fmaf(a[0][r].x, b[0][0].x, acc[r]);
                    acc[r] = __builtin_fmaf(a[0][r].y, b[0][0].y, acc[r]);
                    acc[r] = __builtin_fmaf(a[0][r].z, b[0][1].x, acc[r]);
                    acc[r] = __builtin_fmaf(a[0][r].w, b[0][1].y, acc[r]);
                }
            }
        }
        // the k rows past the last full group (K % 4 in the last stage)
        for (int k = 4 * ng; k < kv; ++k) {
            float bk = rd_f32<0>(bs + (uint32_t)(k * 64 * 4));
#pragma unroll
            for (int r = 0; r < RW; ++r) {
                float ak = rd_f32<0>(a0 + (uint32_t)((r * Kp + k0 + k) * 4));
                asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(ak), "+v"(bk)::"memory");
                acc[r] = __builtin_fmaf(ak, bk, acc[r]);
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the copies past the last stage (no traffic)
    if (n >= N) return;
    const float bv = bias ? bias[n] : 0.0f;
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const int m = mb + wave * RW + r;
        if (m >= M) continue;
        float v = acc[r];
        if (bias) v = v + bv;
        C[(int64_t)m * N + n] = activate<ACT>(v);
    }
}

template <int BM, int BN, int BK, int TM, int TN, int ACT>
hipError_t run(const float* A, const float* B, const float* bias, float* C, int M, int N, int K,
               hipStream_t s) {
    dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
    dim3 block((BM / TM) * (BN / TN));
    hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, BK, TM, TN, ACT>), grid, block, 0, s, A, B, bias,
                       C, M, N, K);
    return hipGetLastError();
}

template <int ACT>
__global__ void activation_kernel(float* out, const float* __restrict__ in, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = activate<ACT>(in[i]);
}

// fusedGelu (reference FusedKernels.h:606-627): gelu_zmm on the full groups
// of 16 elements, and on the last partial group (the n % 16 elements from
// n & ~15 on) the scalar formula with tanhf, evaluated left to right as the
// reference's tail loop is compiled: x + (0.044715*x*x)*x is one fma.
__global__ void fused_gelu_kernel(float* out, const float* __restrict__ in, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t nv = n & ~int64_t(15);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const float x = in[i];
        out[i] = i < nv ? gelu(x)
                        : 0.5f * x * (1.0f + tanhf(0.7978845608f * __builtin_fmaf(0.044715f * x * x, x, x)));
    }
}

}  // namespace

hipError_t launch_gemm_f32_variant(int variant, int act, const float* A, const float* B,
                                   const float* bias, float* C, int M, int N, int K,
                                   hipStream_t s) {
    hipError_t e = hipSuccess;
    // 16-byte copy pieces need whole 16-byte B rows; 4-byte pieces any N
    const bool p16 = (N % 4) == 0 && (reinterpret_cast<uintptr_t>(B) % 16) == 0;
    auto rowsdma = [&](auto kern, int rw) {
        dim3 grid((N + 63) / 64, (M + rw * RWV - 1) / (rw * RWV));
        const size_t lds = ((size_t)RD_NST * RD_KG * 64 + (size_t)rw * RWV * ((K + 3) & ~3)) * sizeof(float);
        hipLaunchKernelGGL(kern, grid, dim3(64 * RWV), lds, s, A, B, bias, C, M, N, K);
        return hipGetLastError();
    };
    if ((variant == GV_F32_ROWS1 || variant == GV_F32_ROWS2) &&
        (reinterpret_cast<uintptr_t>(B) % 4) != 0)
        return hipErrorInvalidValue;  // the C ABI requires 4-byte aligned operands
    switch (variant) {
    case GV_F32_ROWS1:
        if (p16) {
            JH_DISPATCH_ACT(act, ACT, e = rowsdma(gemm_f32_rowsdma_kernel<ACT, 1, 16>, 1));
        } else {
            JH_DISPATCH_ACT(act, ACT, e = rowsdma(gemm_f32_rowsdma_kernel<ACT, 1, 4>, 1));
        }
        break;
    case GV_F32_ROWS2:
        if (p16) {
            JH_DISPATCH_ACT(act, ACT, e = rowsdma(gemm_f32_rowsdma_kernel<ACT, 2, 16>, 2));
        } else {
            JH_DISPATCH_ACT(act, ACT, e = rowsdma(gemm_f32_rowsdma_kernel<ACT, 2, 4>, 2));
        }
        break;
    case GV_F32_T32:
        JH_DISPATCH_ACT(act, ACT, e = (run<32, 32, kF32SliceK, 2, 2, ACT>(A, B, bias, C, M, N, K, s)));
        break;
    case GV_F32_T64:
        JH_DISPATCH_ACT(act, ACT, e = (run<64, 64, kF32SliceK, 4, 4, ACT>(A, B, bias, C, M, N, K, s)));
        break;
    default: e = hipErrorInvalidValue;
    }
    return e;
}

hipError_t launch_gemm_f32(int act, const float* A, const float* B, const float* bias, float* C,
                           int M, int N, int K, hipStream_t s) {
    return launch_gemm_f32_variant(f32_gemm_tile(M, N, K).variant, act, A, B, bias, C, M, N, K, s);
}

hipError_t launch_activation(int act, float* out, const float* in, int64_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const int threads = 256;
    int64_t blocks = (n + threads - 1) / threads;
    if (blocks > 4096) blocks = 4096;
    if (act == JH_ACT_GELU) {
        hipLaunchKernelGGL(fused_gelu_kernel, dim3((unsigned)blocks), dim3(threads), 0, s, out, in, n);
        return hipGetLastError();
    }
    hipError_t e = hipSuccess;
    JH_DISPATCH_ACT(act, ACT, {
        hipLaunchKernelGGL(activation_kernel<ACT>, dim3((unsigned)blocks), dim3(threads), 0, s,
                           out, in, n);
        e = hipGetLastError();
    });
    return e;
}

}  // namespace jh
