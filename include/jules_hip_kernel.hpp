// jules_hip_kernel.hpp - the jules::kernel C++ entry points, on MI355X.
//
// Drop-in for the reference's header-defined kernels
// (include/jules/Kernel/FusedKernels.h, FlashAttention.h, TilePlanner.h,
// ExecutionArena.h): same namespace, names, argument order and argument
// meaning, so a caller such as the reference's benchmarks/bench_kernel.cpp
// switches by including this header instead and linking libjules_hip.so.
//
// Like the reference these are synchronous and take caller-owned buffers.
// Buffers may be host memory (copied to and from the GPU around the call) or
// device memory (used in place).  The reference returns void and validates
// nothing; here a failed call leaves the output unspecified and records a
// jh_status readable with lastStatus() / lastError().  Nothing aborts.
#pragma once

#include <cstddef>
#include <cstdint>
#include <unordered_map>
#include <vector>

#include "jules_hip.h"

namespace jules {
namespace kernel {

// reference FusedKernels.h:61-67; Silu appended (value 5, C ABI JH_ACT_SILU)
enum class ActivationType { None, Relu, Sigmoid, Tanh, Gelu, Silu };

// reference TilePlanner.h:39-56.  On the GPU a TileConfig names one kernel of
// the library's gfx950 tile table (jules_hip_gemm_tile): fp32 rows x 64 x K
// with 4 or 8 rows (the row kernel), 32x32x32 or 64x64x32.  Every table tile
// gives the same bits (each output is one fma chain over k in order), as in
// the reference, whose results do not depend on the tile either.
struct TileConfig {
    int tile_m;
    int tile_n;
    int tile_k;
    size_t footprintBytes(int M, int N, int K) const;
    bool fitsInCache(size_t cacheBytes, int M = 0, int N = 0, int K = 0) const;
};

// reference ExecutionArena.h:41-83, describing the GPU instead of sysfs:
// l1d = LDS per CU, l2 = L2 per XCD, l3 = last-level (MALL) size.
struct CacheInfo {
    size_t l1d_bytes;
    size_t l2_bytes;
    size_t l3_bytes;
    size_t line_bytes;
    int num_cores;  // compute units
    static CacheInfo detect();
};

// reference TilePlanner.h:59-72: the key of the planner's per-shape cache
struct ShapeSignature {
    int m, n, k;
    bool operator==(const ShapeSignature& o) const { return m == o.m && n == o.n && k == o.k; }
    struct Hash {
        size_t operator()(const ShapeSignature& s) const {
            return ((size_t)s.m << 32) | ((size_t)s.n << 16) | (size_t)s.k;
        }
    };
};

// reference TilePlanner.h:74-294.  computeAnalytical returns the tile the
// fp32 GEMM launch uses by default (the library's table); getTileConfig
// caches per shape and, with auto-tuning on (the default, as in the
// reference) and M, N >= 32, times every table kernel that can run the
// shape on the current GPU (one warm-up and 10 timed launches each, HIP
// events) and keeps the fastest.  Like the reference, one planner object is
// not safe to use from two threads at once.
//
// setBenchmarkKernel (reference TilePlanner.h:141-148) registers the function
// that auto-tuning times instead: as in the reference it is called with HOST
// buffers (A, B filled with 1.0f, C of M*N floats), M, N, K and each
// candidate TileConfig, one warm-up and 10 timed calls per candidate on the
// host clock, and must be synchronous.  The candidates stay the GPU table's
// tiles; a captureless lambda that calls tiledMatmulWithActivation below is a
// valid registration.
class TilePlanner {
public:
    using BenchmarkKernelFn = void (*)(const float*, const float*, float*, int, int, int,
                                       const TileConfig&);
    explicit TilePlanner(const CacheInfo& cache = CacheInfo::detect());
    TileConfig getTileConfig(int M, int N, int K);
    TileConfig computeAnalytical(int M, int N, int K) const;
    void setAutoTune(bool enabled) { autoTune_ = enabled; }
    void setVerbose(bool v) { verbose_ = v; }
    const CacheInfo& cacheInfo() const { return cache_; }
    void setBenchmarkKernel(BenchmarkKernelFn fn) { benchmarkKernel_ = fn; }

private:
    TileConfig autoTune(int M, int N, int K, const TileConfig& defaultConfig);
    TileConfig autoTuneWith(BenchmarkKernelFn fn, int M, int N, int K,
                            const TileConfig& defaultConfig);
    CacheInfo cache_;
    bool autoTune_ = true;
    bool verbose_ = false;
    BenchmarkKernelFn benchmarkKernel_ = nullptr;
    std::unordered_map<ShapeSignature, TileConfig, ShapeSignature::Hash> configCache_;
};

// reference ExecutionArena.h:94-199: bump allocator over one DEVICE buffer
// (allocated once, 256-byte aligned blocks); reset() frees everything.
// Overflow returns nullptr and records JH_ERR_WORKSPACE instead of abort().
class ExecutionArena {
public:
    static constexpr size_t DEFAULT_MAX_SIZE = 256UL * 1024 * 1024;
    explicit ExecutionArena(size_t maxSize = DEFAULT_MAX_SIZE);
    ~ExecutionArena();
    ExecutionArena(const ExecutionArena&) = delete;
    ExecutionArena& operator=(const ExecutionArena&) = delete;

    template <typename T>
    T* allocate(size_t count) { return static_cast<T*>(allocateBytes(count * sizeof(T))); }
    void* allocateBytes(size_t bytes);
    void reset() { offset_ = 0; }
    void resetAndZero();
    // reference ExecutionArena.h:170-187 issues CPU cache-prefetch hints over
    // [addr, addr + size).  The kernels here stream their operands from HBM
    // through the GPU's own caches, and a host-side hint would warm the CPU
    // caches with data the GPU does not read from there, so these do nothing.
    void prefetch(const void* addr, size_t size, int level = 1) const {
        (void)addr;
        (void)size;
        (void)level;
    }
    template <typename T>
    void prefetchTensor(const T* data, size_t count, int level = 1) const {
        prefetch(data, count * sizeof(T), level);
    }
    size_t usedBytes() const { return offset_; }
    size_t highWaterMark() const { return highWaterMark_; }
    size_t capacity() const { return maxSize_; }
    char* rawBuffer() { return buffer_; }
    const char* rawBuffer() const { return buffer_; }

private:
    char* buffer_ = nullptr;
    size_t maxSize_ = 0;
    size_t offset_ = 0;
    size_t highWaterMark_ = 0;
};

// status of the last jules::kernel call on this thread (JH_OK on success)
int lastStatus();
const char* lastError();

// reference FusedKernels.h:203
void fusedMatmulRelu(const float* X, const float* W, float* output, int M, int K, int N);
// reference FusedKernels.h:265
void fusedMatmulBiasRelu(const float* X, const float* W, const float* bias, float* output, int M,
                         int K, int N);
// reference FusedKernels.h:378.  A cfg naming a kernel of the tile table
// (what TilePlanner returns) runs that kernel; any other cfg runs the
// table's default for the shape.  The bits are the same either way.
void tiledMatmulWithActivation(const float* A, const float* B, float* C, int M, int N, int K,
                               const TileConfig& cfg, ActivationType act = ActivationType::None);
// reference FusedKernels.h:633-644: C = alpha op(A) op(B) + beta C with the
// reference's leading dimensions (A [M,K] or [K,M], B [K,N] or [N,K], C
// [M,N], all dense); jules_hip_sgemm
void blasMatmul(const float* A, const float* B, float* C, int M, int N, int K, float alpha = 1.0f,
                float beta = 0.0f, bool transA = false, bool transB = false);
// reference FusedKernels.h:606
void fusedGelu(float* output, const float* input, int N);
// reference FusedKernels.h:464
void fusedSoftmax(float* output, const float* input, int M, int N);
// reference FusedKernels.h:532
void fusedLayerNorm(float* output, const float* input, const float* gamma, const float* beta,
                    int M, int N, float epsilon = 1e-5f);
// reference FusedKernels.h:766; returns the mean loss (NaN on failure)
float fusedCrossEntropyLoss(const float* logits, const int32_t* targets, float* grad, int M, int N);
// reference FusedKernels.h:650-657, :659
struct MLPParams {
    const float* W1;
    const float* b1;
    const float* W2;
    const float* b2;
    int batch_size;
    int in_features;
    int hidden_features;
    int out_features;
};
void fusedMLPForward(float* output, const float* X, const MLPParams& params, ExecutionArena& arena,
                     TilePlanner& planner);
// reference InterleavedAutodiff.h:41-53
struct MLPGradients {
    float* dW1;
    float* db1;
    float* dW2;
    float* db2;
    float* dX;
};
struct InterleavedMLPResult {
    float loss;
    MLPGradients grads;
};
// reference InterleavedAutodiff.h:55-62: 2-layer MLP forward, softmax cross
// entropy and backward; dX may be null; loss is NaN on failure
InterleavedMLPResult interleavedMLPForwardBackward(const float* X, const float* W1,
                                                   const float* b1, const float* W2,
                                                   const float* b2, const int32_t* targets,
                                                   float* output, float* dW1, float* db1,
                                                   float* dW2, float* db2, float* dX, int M,
                                                   int K1, int N1, int N2, ExecutionArena& arena,
                                                   TilePlanner& planner);
// reference FusedKernels.h:867 (scalar-path semantics)
void matmulInt8(const int8_t* A, const int8_t* B, float* C, int M, int N, int K, float scale_A,
                float scale_B, const float* bias = nullptr, ExecutionArena* arena = nullptr);
// reference FlashAttention.h:130 (non-causal, scale 1/sqrtf(head_dim))
void flashAttention(float* output, const float* Q, const float* K, const float* V, int batch,
                    int heads, int seq, int head_dim, ExecutionArena& arena, TilePlanner& planner);
// reference FusedKernels.h:1085-1115: flash attention when the [S,S] fp32
// score matrix exceeds l3_bytes, or when seq_len >= 64 and head_dim <= 256
inline bool shouldUseFlashAttention(int seq_len, int head_dim, size_t l3_bytes) {
    const size_t attn_matrix_bytes = (size_t)seq_len * seq_len * sizeof(float);
    if (attn_matrix_bytes > l3_bytes) return true;
    return seq_len >= 64 && head_dim <= 256;
}
// reference FlashAttention.h:114-124: chooses with shouldUseFlashAttention and
// planner.cacheInfo().l3_bytes between flashAttention and standardAttention
void attention(float* output, const float* Q, const float* K, const float* V, int batch,
               int heads, int seq, int head_dim, ExecutionArena& arena, TilePlanner& planner);
// reference FlashAttention.h:52-100: softmax(Q K^T / sqrt(D)) V, non-causal.
// On the GPU it runs the flash kernel (the same function; the reference
// materialises the [S,S] matrix only because that is faster on a CPU for
// small S), then resets the arena as the reference does.
void standardAttention(float* output, const float* Q, const float* K, const float* V, int batch,
                       int heads, int seq, int head_dim, ExecutionArena& arena);

}  // namespace kernel
}  // namespace jules
