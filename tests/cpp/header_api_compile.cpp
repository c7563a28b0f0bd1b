// header_api_compile.cpp - every public member of the reference's kernel
// headers, called through include/jules_hip_kernel.hpp.  TEST
// INFRASTRUCTURE ONLY: tests/test_capi.py compiles and links this file
// against libjules_hip.so (no GPU needed) to show that a caller written
// against the reference's ExecutionArena.h, TilePlanner.h, FusedKernels.h,
// FlashAttention.h and InterleavedAutodiff.h builds against this header.
// The program runs nothing unless given arguments.
#include <cstdio>
#include <unordered_map>
#include <vector>

#include "jules_hip_kernel.hpp"

using namespace jules::kernel;

namespace {

// TilePlanner::BenchmarkKernelFn (TilePlanner.h:144-145)
void bench_fn(const float* A, const float* B, float* C, int M, int N, int K, const TileConfig& cfg) {
    tiledMatmulWithActivation(A, B, C, M, N, K, cfg);
}

int exercise() {
    // ExecutionArena.h:41-83
    CacheInfo ci = CacheInfo::detect();
    size_t cache_sum = ci.l1d_bytes + ci.l2_bytes + ci.l3_bytes + ci.line_bytes + (size_t)ci.num_cores;

    // ExecutionArena.h:94-199
    static_assert(ExecutionArena::DEFAULT_MAX_SIZE == 256UL * 1024 * 1024, "default arena size");
    ExecutionArena arena;
    ExecutionArena small(1 << 20);
    float* f = arena.allocate<float>(64);
    void* raw = arena.allocateBytes(128);
    arena.prefetch(raw, 128);
    arena.prefetch(raw, 128, 2);
    arena.prefetchTensor(f, 64);
    arena.prefetchTensor(f, 64, 0);
    size_t used = arena.usedBytes() + arena.highWaterMark() + arena.capacity();
    char* buf = arena.rawBuffer();
    const ExecutionArena& carena = arena;
    const char* cbuf = carena.rawBuffer();
    carena.prefetch(cbuf, 16);
    arena.resetAndZero();
    arena.reset();
    small.reset();

    // TilePlanner.h:39-72
    TileConfig tc{32, 32, 128};
    size_t fp = tc.footprintBytes(64, 64, 64);
    bool fits = tc.fitsInCache(ci.l1d_bytes) && tc.fitsInCache(ci.l2_bytes, 64, 64, 64);
    ShapeSignature sig{64, 64, 64};
    std::unordered_map<ShapeSignature, TileConfig, ShapeSignature::Hash> cache;
    cache[sig] = tc;
    bool same = sig == ShapeSignature{64, 64, 64};

    // TilePlanner.h:74-148
    TilePlanner planner;
    TilePlanner planner2(ci);
    planner.setAutoTune(false);
    planner.setVerbose(true);
    TilePlanner::BenchmarkKernelFn fn = &bench_fn;
    planner2.setBenchmarkKernel(fn);
    TileConfig got = planner.getTileConfig(64, 64, 64);
    TileConfig ana = planner.computeAnalytical(64, 64, 64);
    const CacheInfo& pci = planner.cacheInfo();

    // FusedKernels.h
    std::vector<float> A(64 * 64, 1.0f), B(64 * 64, 1.0f), C(64 * 64), bias(64, 0.0f);
    fusedMatmulRelu(A.data(), B.data(), C.data(), 64, 64, 64);
    fusedMatmulBiasRelu(A.data(), B.data(), bias.data(), C.data(), 64, 64, 64);
    tiledMatmulWithActivation(A.data(), B.data(), C.data(), 64, 64, 64, got);
    for (ActivationType act : {ActivationType::None, ActivationType::Relu, ActivationType::Sigmoid,
                               ActivationType::Tanh, ActivationType::Gelu})
        tiledMatmulWithActivation(A.data(), B.data(), C.data(), 64, 64, 64, ana, act);
    fusedSoftmax(C.data(), A.data(), 64, 64);
    fusedLayerNorm(C.data(), A.data(), bias.data(), bias.data(), 64, 64);
    fusedLayerNorm(C.data(), A.data(), bias.data(), bias.data(), 64, 64, 1e-6f);
    fusedGelu(C.data(), A.data(), 64 * 64);
    blasMatmul(A.data(), B.data(), C.data(), 64, 64, 64);
    blasMatmul(A.data(), B.data(), C.data(), 64, 64, 64, 0.5f, 1.0f, true, true);
    MLPParams p{B.data(), bias.data(), B.data(), bias.data(), 64, 64, 64, 64};
    fusedMLPForward(C.data(), A.data(), p, arena, planner);
    std::vector<int32_t> targets(64, 0);
    float loss = fusedCrossEntropyLoss(A.data(), targets.data(), C.data(), 64, 64);
    std::vector<int8_t> qa(64 * 64, 1), qb(64 * 64, 1);
    matmulInt8(qa.data(), qb.data(), C.data(), 64, 64, 64, 0.1f, 0.1f);
    matmulInt8(qa.data(), qb.data(), C.data(), 64, 64, 64, 0.1f, 0.1f, bias.data(), &arena);
    bool flash = shouldUseFlashAttention(1024, 64, ci.l3_bytes);

    // FlashAttention.h:42-124
    std::vector<float> Q(1 * 2 * 64 * 32, 0.5f), O(Q.size());
    flashAttention(O.data(), Q.data(), Q.data(), Q.data(), 1, 2, 64, 32, arena, planner);
    standardAttention(O.data(), Q.data(), Q.data(), Q.data(), 1, 2, 64, 32, arena);
    attention(O.data(), Q.data(), Q.data(), Q.data(), 1, 2, 64, 32, arena, planner);

    // InterleavedAutodiff.h:41-62
    std::vector<float> out(64 * 64), dW1(64 * 64), db1(64), dW2(64 * 64), db2(64), dX(64 * 64);
    InterleavedMLPResult r = interleavedMLPForwardBackward(
        A.data(), B.data(), bias.data(), B.data(), bias.data(), targets.data(), out.data(),
        dW1.data(), db1.data(), dW2.data(), db2.data(), dX.data(), 64, 64, 64, 64, arena, planner);
    MLPGradients g = r.grads;

    std::printf("%zu %zu %zu %p %p %d %d %d %zu %d %d %f %f %p %d\n", cache_sum, used, fp,
                (void*)buf, (const void*)cbuf, (int)fits, (int)same, pci.num_cores,
                cache.size(), got.tile_m + ana.tile_n, (int)flash, loss, r.loss, (void*)g.dW1,
                lastStatus());
    return lastStatus();
}

}  // namespace

int main(int argc, char**) { return argc > 1 ? exercise() : 0; }
