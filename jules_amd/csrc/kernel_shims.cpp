// kernel_shims.cpp - jules::kernel C++ entry points (include/jules_hip_kernel.hpp)
// implemented on the C ABI.  Host buffers are staged through device memory
// and the call is synchronous, as the reference's CPU kernels are.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <limits>
#include <string>
#include <vector>

#include "jules_hip.h"
#include "jules_hip_kernel.hpp"
#include "launch.hpp"
#include "tiles.hpp"

namespace jh {
int set_last_error(int status, const std::string& message);  // capi.cpp
}

namespace jules {
namespace kernel {
namespace {

thread_local int g_status = JH_OK;
thread_local std::string g_error;

void record(int st) {
    g_status = st;
    g_error = st == JH_OK ? std::string() : std::string(jules_hip_last_error());
}

bool is_device_ptr(const void* p) {
    if (!p) return false;
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeDevice;
}

// A device view of a caller buffer: the buffer itself when it already lives
// on the device, otherwise a device copy (copied in if `in`, back if `out`).
class DevBuf {
public:
    DevBuf(const void* host, size_t bytes, bool in, bool out)
        : host_(const_cast<void*>(host)), bytes_(bytes), out_(out) {
        if (!host || bytes == 0) return;
        if (is_device_ptr(host)) {
            dev_ = host_;
            return;
        }
        if (hipMalloc(&dev_, bytes) != hipSuccess) {
            dev_ = nullptr;
            ok_ = false;
            return;
        }
        owned_ = true;
        if (in && hipMemcpy(dev_, host, bytes, hipMemcpyHostToDevice) != hipSuccess) ok_ = false;
    }
    ~DevBuf() {
        if (owned_) (void)hipFree(dev_);
    }
    bool finish() {  // copy results back; false on failure
        if (!ok_) return false;
        if (owned_ && out_ && hipMemcpy(host_, dev_, bytes_, hipMemcpyDeviceToHost) != hipSuccess)
            return false;
        return true;
    }
    bool ok() const { return ok_; }
    void* get() const { return dev_; }

private:
    void* host_;
    void* dev_ = nullptr;
    size_t bytes_;
    bool out_;
    bool owned_ = false;
    bool ok_ = true;
};

// variant: a kernel of the tile table, or -1 for the table's default
void run_gemm(const float* A, const float* B, const float* bias, float* C, int M, int N, int K,
              int act, int variant = -1) {
    if (M < 0 || N < 0 || K < 0) return record(JH_ERR_SHAPE);
    DevBuf a(A, sizeof(float) * (size_t)M * K, true, false);
    DevBuf b(B, sizeof(float) * (size_t)K * N, true, false);
    DevBuf bi(bias, bias ? sizeof(float) * (size_t)N : 0, true, false);
    DevBuf c(C, sizeof(float) * (size_t)M * N, false, true);
    if (!a.ok() || !b.ok() || !bi.ok() || !c.ok()) return record(JH_ERR_HIP);
    int st = jh::gemm_f32_with_variant(variant, act, static_cast<const float*>(a.get()),
                                       static_cast<const float*>(b.get()),
                                       static_cast<const float*>(bi.get()),
                                       static_cast<float*>(c.get()), M, N, K, nullptr);
    if (st == JH_OK && hipDeviceSynchronize() != hipSuccess) st = JH_ERR_HIP;
    if (st == JH_OK && !c.finish()) st = JH_ERR_HIP;
    record(st);
}

// the table kernel a TileConfig names at depth K, or -1
int variant_of(const TileConfig& cfg, int K) {
    for (int v = jh::GV_F32_ROWS1; v <= jh::GV_F32_T64; ++v) {
        const jh::GemmTile t = jh::f32_variant_tile(v, K);
        if (jh::f32_variant_valid(v, K) && t.tile_m == cfg.tile_m && t.tile_n == cfg.tile_n &&
            t.tile_k == cfg.tile_k)
            return v;
    }
    return -1;
}

TileConfig to_config(const jh::GemmTile& t) { return TileConfig{t.tile_m, t.tile_n, t.tile_k}; }

void run_attention(float* out, const float* Q, const float* K, const float* V, int B, int H,
                   int S, int D) {
    if (B < 0 || H < 0 || S < 0 || D <= 0) return record(JH_ERR_SHAPE);
    const size_t bytes = sizeof(float) * (size_t)B * H * S * D;
    DevBuf q(Q, bytes, true, false), k(K, bytes, true, false), v(V, bytes, true, false);
    DevBuf o(out, bytes, false, true);
    if (!q.ok() || !k.ok() || !v.ok() || !o.ok()) return record(JH_ERR_HIP);
    const float scale = 1.0f / sqrtf((float)D);  // reference FlashAttention.h:135
    int st = jules_hip_flash_attn_fwd(JH_F32, 0, scale, q.get(), k.get(), v.get(), o.get(),
                                      nullptr, B, H, S, D, nullptr);
    if (st == JH_OK && hipDeviceSynchronize() != hipSuccess) st = JH_ERR_HIP;
    if (st == JH_OK && !o.finish()) st = JH_ERR_HIP;
    record(st);
}

}  // namespace

int lastStatus() { return g_status; }
const char* lastError() { return g_error.c_str(); }

size_t TileConfig::footprintBytes(int, int, int) const {
    return ((size_t)tile_m * tile_k + (size_t)tile_k * tile_n + (size_t)tile_m * tile_n) * 4;
}
bool TileConfig::fitsInCache(size_t cacheBytes, int M, int N, int K) const {
    return footprintBytes(M, N, K) <= cacheBytes;
}

CacheInfo CacheInfo::detect() {
    CacheInfo c{160 * 1024, 4 * 1024 * 1024, 256UL * 1024 * 1024, 128, 256};
    int dev = 0;
    hipDeviceProp_t p;
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&p, dev) == hipSuccess) {
        if (p.maxSharedMemoryPerMultiProcessor > 0) c.l1d_bytes = p.maxSharedMemoryPerMultiProcessor;
        if (p.l2CacheSize > 0) c.l2_bytes = (size_t)p.l2CacheSize;
        if (p.multiProcessorCount > 0) c.num_cores = p.multiProcessorCount;
    } else {
        (void)hipGetLastError();
    }
    return c;
}

TilePlanner::TilePlanner(const CacheInfo& cache) : cache_(cache) {}

TileConfig TilePlanner::computeAnalytical(int M, int N, int K) const {
    return to_config(jh::f32_gemm_tile(M, N, K));
}

TileConfig TilePlanner::getTileConfig(int M, int N, int K) {
    const ShapeSignature sig{M, N, K};
    auto it = configCache_.find(sig);
    if (it != configCache_.end()) return it->second;
    TileConfig cfg = computeAnalytical(M, N, K);
    if (autoTune_ && M >= 32 && N >= 32)  // TilePlanner.h:88-90
        cfg = benchmarkKernel_ ? autoTuneWith(benchmarkKernel_, M, N, K, cfg)
                               : autoTune(M, N, K, cfg);
    configCache_[sig] = cfg;
    return cfg;
}

// The registered benchmark function over the table's tiles for this depth,
// on host buffers of ones (TilePlanner.h:188-236), host-clock timed.
TileConfig TilePlanner::autoTuneWith(BenchmarkKernelFn fn, int M, int N, int K,
                                     const TileConfig& defaultConfig) {
    std::vector<float> A((size_t)M * K, 1.0f), B((size_t)K * N, 1.0f), C((size_t)M * N, 0.0f);
    TileConfig best = defaultConfig;
    double best_ms = 1e18;
    for (int v = jh::GV_F32_ROWS1; v <= jh::GV_F32_T64; ++v) {
        if (!jh::f32_variant_valid(v, K)) continue;
        const TileConfig cfg = to_config(jh::f32_variant_tile(v, K));
        fn(A.data(), B.data(), C.data(), M, N, K, cfg);  // warm-up, not timed
        constexpr int iters = 10;
        const auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < iters; ++i) fn(A.data(), B.data(), C.data(), M, N, K, cfg);
        const double ms =
            std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count() /
            iters;
        if (ms < best_ms) {
            best_ms = ms;
            best = cfg;
        }
    }
    if (verbose_)
        std::printf("Auto-tune [%d,%d]x[%d,%d]: tile=(%d,%d,%d) %.3fms\n", M, K, K, N, best.tile_m,
                    best.tile_n, best.tile_k, best_ms);
    return best;
}

// Times each table kernel that can run the shape (TilePlanner.h:158-236 does
// the same over CPU tile candidates): zero-filled device operands, one
// warm-up and 10 timed launches per kernel between HIP events.  Any HIP
// failure keeps the table's default.
TileConfig TilePlanner::autoTune(int M, int N, int K, const TileConfig& defaultConfig) {
    float *A = nullptr, *B = nullptr, *C = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    const size_t fa = (size_t)M * K, fb = (size_t)K * N, fc = (size_t)M * N;
    TileConfig best = defaultConfig;
    float best_ms = 0.0f;
    bool ok = hipMalloc(&A, 4 * (fa ? fa : 1)) == hipSuccess &&
              hipMalloc(&B, 4 * (fb ? fb : 1)) == hipSuccess &&
              hipMalloc(&C, 4 * (fc ? fc : 1)) == hipSuccess &&
              hipMemset(A, 0, 4 * (fa ? fa : 1)) == hipSuccess &&
              hipMemset(B, 0, 4 * (fb ? fb : 1)) == hipSuccess &&
              hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess;
    for (int v = jh::GV_F32_ROWS1; ok && v <= jh::GV_F32_T64; ++v) {
        if (!jh::f32_variant_valid(v, K)) continue;
        constexpr int iters = 10;
        ok = jh::launch_gemm_f32_variant(v, JH_ACT_NONE, A, B, nullptr, C, M, N, K, nullptr) ==
                 hipSuccess &&
             hipEventRecord(e0, nullptr) == hipSuccess;
        for (int i = 0; ok && i < iters; ++i)
            ok = jh::launch_gemm_f32_variant(v, JH_ACT_NONE, A, B, nullptr, C, M, N, K, nullptr) ==
                 hipSuccess;
        float ms = 0.0f;
        ok = ok && hipEventRecord(e1, nullptr) == hipSuccess &&
             hipEventSynchronize(e1) == hipSuccess && hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
        if (ok && (best_ms == 0.0f || ms < best_ms)) {
            best_ms = ms;
            best = to_config(jh::f32_variant_tile(v, K));
        }
    }
    if (!ok) {
        (void)hipGetLastError();
        best = defaultConfig;
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (A) (void)hipFree(A);
    if (B) (void)hipFree(B);
    if (C) (void)hipFree(C);
    if (verbose_ && ok)
        std::printf("Auto-tune [%d,%d]x[%d,%d]: tile=(%d,%d,%d) %.3fms\n", M, K, K, N, best.tile_m,
                    best.tile_n, best.tile_k, best_ms / 10.0f);
    return best;
}

ExecutionArena::ExecutionArena(size_t maxSize) : maxSize_(maxSize) {
    void* p = nullptr;
    if (hipMalloc(&p, maxSize_) != hipSuccess || hipMemset(p, 0, maxSize_) != hipSuccess) {
        (void)hipGetLastError();
        if (p) (void)hipFree(p);
        p = nullptr;
        maxSize_ = 0;
    }
    buffer_ = static_cast<char*>(p);
}
ExecutionArena::~ExecutionArena() {
    if (buffer_) (void)hipFree(buffer_);
}
void* ExecutionArena::allocateBytes(size_t bytes) {
    const size_t aligned_offset = (offset_ + 255) & ~size_t(255);
    // written so that a huge request cannot wrap around the size check
    if (!buffer_ || aligned_offset > maxSize_ || bytes > maxSize_ - aligned_offset) {
        record(JH_ERR_WORKSPACE);
        return nullptr;
    }
    offset_ = aligned_offset + bytes;
    if (offset_ > highWaterMark_) highWaterMark_ = offset_;
    return buffer_ + aligned_offset;
}
void ExecutionArena::resetAndZero() {
    if (buffer_ && offset_) (void)hipMemset(buffer_, 0, offset_);
    offset_ = 0;
}

void fusedMatmulRelu(const float* X, const float* W, float* output, int M, int K, int N) {
    run_gemm(X, W, nullptr, output, M, N, K, JH_ACT_RELU);
}

void fusedMatmulBiasRelu(const float* X, const float* W, const float* bias, float* output, int M,
                         int K, int N) {
    run_gemm(X, W, bias, output, M, N, K, JH_ACT_RELU);
}

void tiledMatmulWithActivation(const float* A, const float* B, float* C, int M, int N, int K,
                               const TileConfig& cfg, ActivationType act) {
    if (K == 0 && M > 0 && N > 0) {
        // The reference zeroes C (FusedKernels.h:382) and applies the
        // activation only inside its K-slice loop (:407), which K = 0 never
        // enters: C stays 0 for every activation (act(0) is 0.5 for sigmoid).
        const size_t bytes = sizeof(float) * (size_t)M * (size_t)N;
        int st = JH_OK;
        if (is_device_ptr(C)) {
            if (hipMemset(C, 0, bytes) != hipSuccess || hipDeviceSynchronize() != hipSuccess)
                st = JH_ERR_HIP;
        } else if (C) {
            std::memset(C, 0, bytes);
        } else {
            st = JH_ERR_NULL;
        }
        if (st == JH_ERR_HIP) (void)hipGetLastError();
        if (st != JH_OK)
            jh::set_last_error(st, st == JH_ERR_NULL ? "tiledMatmulWithActivation: C is null"
                                                     : "tiledMatmulWithActivation: zeroing C failed");
        return record(st);
    }
    run_gemm(A, B, nullptr, C, M, N, K, static_cast<int>(act), variant_of(cfg, K));
}

void blasMatmul(const float* A, const float* B, float* C, int M, int N, int K, float alpha,
                float beta, bool transA, bool transB) {
    if (M < 0 || N < 0 || K < 0) return record(JH_ERR_SHAPE);
    const size_t f = sizeof(float);
    DevBuf a(A, f * (size_t)M * K, true, false), b(B, f * (size_t)K * N, true, false);
    // C is read when beta != 0 (FusedKernels.h:637-643 passes beta to sgemm)
    DevBuf c(C, f * (size_t)M * N, beta != 0.0f, true);
    if (!a.ok() || !b.ok() || !c.ok()) return record(JH_ERR_HIP);
    // leading dimensions as the reference passes them: transA ? M : K,
    // transB ? K : N, N
    int st = jules_hip_sgemm(transA ? 1 : 0, transB ? 1 : 0, M, N, K, alpha,
                             static_cast<const float*>(a.get()), transA ? M : K,
                             static_cast<const float*>(b.get()), transB ? K : N, beta,
                             static_cast<float*>(c.get()), N, nullptr);
    if (st == JH_OK && hipDeviceSynchronize() != hipSuccess) st = JH_ERR_HIP;
    if (st == JH_OK && !c.finish()) st = JH_ERR_HIP;
    record(st);
}

void fusedGelu(float* output, const float* input, int N) {
    if (N < 0) return record(JH_ERR_SHAPE);
    const size_t bytes = sizeof(float) * (size_t)N;
    DevBuf in(input, bytes, true, false), out(output, bytes, false, true);
    if (!in.ok() || !out.ok()) return record(JH_ERR_HIP);
    int st = jules_hip_activation(JH_ACT_GELU, static_cast<float*>(out.get()),
                                  static_cast<const float*>(in.get()), N, nullptr);
    if (st == JH_OK && hipDeviceSynchronize() != hipSuccess) st = JH_ERR_HIP;
    if (st == JH_OK && !out.finish()) st = JH_ERR_HIP;
    record(st);
}

void fusedSoftmax(float* output, const float* input, int M, int N) {
    if (M < 0 || N < 0) return record(JH_ERR_SHAPE);
    const size_t bytes = sizeof(float) * (size_t)M * (size_t)N;
    DevBuf in(input, bytes, true, false), out(output, bytes, false, true);
    if (!in.ok() || !out.ok()) return record(JH_ERR_HIP);
    int st = jules_hip_softmax(static_cast<float*>(out.get()), static_cast<const float*>(in.get()),
                               M, N, nullptr);
    if (st == JH_OK && hipDeviceSynchronize() != hipSuccess) st = JH_ERR_HIP;
    if (st == JH_OK && !out.finish()) st = JH_ERR_HIP;
    record(st);
}

void fusedLayerNorm(float* output, const float* input, const float* gamma, const float* beta,
                    int M, int N, float epsilon) {
    if (M < 0 || N < 0) return record(JH_ERR_SHAPE);
    const size_t bytes = sizeof(float) * (size_t)M * (size_t)N;
    const size_t nb = sizeof(float) * (size_t)N;
    DevBuf in(input, bytes, true, false), out(output, bytes, false, true);
    DevBuf g(gamma, nb, true, false), b(beta, nb, true, false);
    if (!in.ok() || !out.ok() || !g.ok() || !b.ok()) return record(JH_ERR_HIP);
    int st = jules_hip_layernorm(static_cast<float*>(out.get()), static_cast<const float*>(in.get()),
                                 static_cast<const float*>(g.get()),
                                 static_cast<const float*>(b.get()), M, N, epsilon, nullptr);
    if (st == JH_OK && hipDeviceSynchronize() != hipSuccess) st = JH_ERR_HIP;
    if (st == JH_OK && !out.finish()) st = JH_ERR_HIP;
    record(st);
}

void fusedMLPForward(float* output, const float* X, const MLPParams& p, ExecutionArena&,
                     TilePlanner&) {
    const int M = p.batch_size, K1 = p.in_features, N1 = p.hidden_features, N2 = p.out_features;
    if (M < 0 || K1 < 1 || N1 < 1 || N2 < 1) {
        record(JH_ERR_SHAPE);
        return;
    }
    const size_t f = sizeof(float), m = (size_t)M, k1 = (size_t)K1, n1 = (size_t)N1, n2 = (size_t)N2;
    std::vector<char> ws_host(std::max<size_t>(16, jules_hip_mlp_forward_workspace_size(M, K1, N1, N2)));
    DevBuf x(X, f * m * k1, true, false), w1(p.W1, f * k1 * n1, true, false),
        b1(p.b1, f * n1, true, false), w2(p.W2, f * n1 * n2, true, false), b2(p.b2, f * n2, true, false),
        o(output, f * m * n2, false, true), ws(ws_host.data(), ws_host.size(), false, false);
    if (!x.ok() || !w1.ok() || !b1.ok() || !w2.ok() || !b2.ok() || !o.ok() || !ws.ok()) {
        record(JH_ERR_HIP);
        return;
    }
    int st = jules_hip_mlp_forward(static_cast<const float*>(x.get()), static_cast<const float*>(w1.get()),
                                   static_cast<const float*>(b1.get()), static_cast<const float*>(w2.get()),
                                   static_cast<const float*>(b2.get()), static_cast<float*>(o.get()), M,
                                   K1, N1, N2, ws.get(), ws_host.size(), nullptr);
    if (st == JH_OK && hipDeviceSynchronize() != hipSuccess) st = JH_ERR_HIP;
    if (st == JH_OK && !o.finish()) st = JH_ERR_HIP;
    record(st);
}

InterleavedMLPResult interleavedMLPForwardBackward(const float* X, const float* W1,
                                                   const float* b1, const float* W2,
                                                   const float* b2, const int32_t* targets,
                                                   float* output, float* dW1, float* db1,
                                                   float* dW2, float* db2, float* dX, int M,
                                                   int K1, int N1, int N2, ExecutionArena&,
                                                   TilePlanner&) {
    const float nan = std::numeric_limits<float>::quiet_NaN();
    InterleavedMLPResult res{nan, MLPGradients{dW1, db1, dW2, db2, dX}};
    if (M < 0 || K1 < 1 || N1 < 1 || N2 < 1) {
        record(JH_ERR_SHAPE);
        return res;
    }
    const size_t f = sizeof(float), m = (size_t)M, k1 = (size_t)K1, n1 = (size_t)N1,
                 n2 = (size_t)N2;
    float loss = nan;
    std::vector<char> ws_host(std::max<size_t>(16, jules_hip_mlp_workspace_size(M, K1, N1, N2)));
    DevBuf x(X, f * m * k1, true, false), w1(W1, f * k1 * n1, true, false),
        bb1(b1, f * n1, true, false), w2(W2, f * n1 * n2, true, false), bb2(b2, f * n2, true, false),
        t(targets, sizeof(int32_t) * m, true, false), o(output, f * m * n2, false, true),
        g1(dW1, f * k1 * n1, false, true), gb1(db1, f * n1, false, true),
        g2(dW2, f * n1 * n2, false, true), gb2(db2, f * n2, false, true),
        gx(dX, f * m * k1, false, true), l(&loss, f, false, true),
        ws(ws_host.data(), ws_host.size(), false, false);
    const DevBuf* all[] = {&x, &w1, &bb1, &w2, &bb2, &t, &o, &g1, &gb1, &g2, &gb2, &gx, &l, &ws};
    for (const DevBuf* d : all)
        if (!d->ok()) {
            record(JH_ERR_HIP);
            return res;
        }
    int st = jules_hip_mlp_forward_backward(
        static_cast<const float*>(x.get()), static_cast<const float*>(w1.get()),
        static_cast<const float*>(bb1.get()), static_cast<const float*>(w2.get()),
        static_cast<const float*>(bb2.get()), static_cast<const int32_t*>(t.get()),
        static_cast<float*>(o.get()), static_cast<float*>(g1.get()), static_cast<float*>(gb1.get()),
        static_cast<float*>(g2.get()), static_cast<float*>(gb2.get()),
        dX ? static_cast<float*>(gx.get()) : nullptr, M, K1, N1, N2, static_cast<float*>(l.get()),
        ws.get(), ws_host.size(), nullptr);
    if (st == JH_OK && hipDeviceSynchronize() != hipSuccess) st = JH_ERR_HIP;
    DevBuf* outs[] = {&o, &g1, &gb1, &g2, &gb2, &gx, &l};
    for (DevBuf* d : outs)
        if (st == JH_OK && !d->finish()) st = JH_ERR_HIP;
    record(st);
    if (st == JH_OK) res.loss = loss;
    return res;
}

float fusedCrossEntropyLoss(const float* logits, const int32_t* targets, float* grad, int M,
                            int N) {
    const float nan = std::numeric_limits<float>::quiet_NaN();
    if (M < 0 || N < 0) {
        record(JH_ERR_SHAPE);
        return nan;
    }
    const size_t bytes = sizeof(float) * (size_t)M * (size_t)N;
    float loss = nan;
    std::vector<float> ws_host(std::max<size_t>(1, (size_t)M));
    DevBuf x(logits, bytes, true, false), t(targets, sizeof(int32_t) * (size_t)M, true, false);
    DevBuf g(grad, bytes, false, true), l(&loss, sizeof(float), false, true);
    DevBuf ws(ws_host.data(), sizeof(float) * ws_host.size(), false, false);
    if (!x.ok() || !t.ok() || !g.ok() || !l.ok() || !ws.ok()) {
        record(JH_ERR_HIP);
        return nan;
    }
    int st = jules_hip_cross_entropy(static_cast<const float*>(x.get()),
                                     static_cast<const int32_t*>(t.get()),
                                     static_cast<float*>(g.get()), static_cast<float*>(l.get()), M,
                                     N, ws.get(), sizeof(float) * ws_host.size(), nullptr);
    if (st == JH_OK && hipDeviceSynchronize() != hipSuccess) st = JH_ERR_HIP;
    if (st == JH_OK && (!g.finish() || !l.finish())) st = JH_ERR_HIP;
    record(st);
    return st == JH_OK ? loss : nan;
}

void matmulInt8(const int8_t* A, const int8_t* B, float* C, int M, int N, int K, float scale_A,
                float scale_B, const float* bias, ExecutionArena*) {
    if (M < 0 || N < 0 || K < 0) return record(JH_ERR_SHAPE);
    DevBuf a(A, (size_t)M * K, true, false), b(B, (size_t)K * N, true, false);
    DevBuf bi(bias, bias ? sizeof(float) * (size_t)N : 0, true, false);
    DevBuf c(C, sizeof(float) * (size_t)M * N, false, true);
    if (!a.ok() || !b.ok() || !bi.ok() || !c.ok()) return record(JH_ERR_HIP);
    int st = jules_hip_matmul_int8(static_cast<const int8_t*>(a.get()),
                                   static_cast<const int8_t*>(b.get()),
                                   static_cast<float*>(c.get()), M, N, K, scale_A, scale_B,
                                   static_cast<const float*>(bi.get()), nullptr);
    if (st == JH_OK && hipDeviceSynchronize() != hipSuccess) st = JH_ERR_HIP;
    if (st == JH_OK && !c.finish()) st = JH_ERR_HIP;
    record(st);
}

void flashAttention(float* output, const float* Q, const float* K, const float* V, int batch,
                    int heads, int seq, int head_dim, ExecutionArena&, TilePlanner&) {
    run_attention(output, Q, K, V, batch, heads, seq, head_dim);
}

void attention(float* output, const float* Q, const float* K, const float* V, int batch, int heads,
               int seq, int head_dim, ExecutionArena& arena, TilePlanner& planner) {
    if (shouldUseFlashAttention(seq, head_dim, planner.cacheInfo().l3_bytes))
        flashAttention(output, Q, K, V, batch, heads, seq, head_dim, arena, planner);
    else
        standardAttention(output, Q, K, V, batch, heads, seq, head_dim, arena);
}

void standardAttention(float* output, const float* Q, const float* K, const float* V, int batch,
                       int heads, int seq, int head_dim, ExecutionArena& arena) {
    run_attention(output, Q, K, V, batch, heads, seq, head_dim);
    arena.reset();  // reference FlashAttention.h:99
}

}  // namespace kernel
}  // namespace jules
