// host_sanitize.cpp - drives the library's host code (argument checks, error
// strings, the kernel registry and its descriptor/backend_config parsing, the
// tile table and TilePlanner, ExecutionArena, PJRT program parsing, the
// cblas_sgemm front end) with valid, invalid and extreme arguments, in a
// build of those sources with AddressSanitizer and UndefinedBehaviorSanitizer.
// It needs no GPU: every call either fails its checks or reaches the HIP
// runtime, which reports that there is no device.  Exit status 0 and no
// sanitizer report means the host code stayed in bounds and free of undefined
// behaviour on all of these inputs.
#include <climits>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "jules_cblas.h"
#include "jules_hip.h"
#include "jules_hip_kernel.hpp"

static int g_fail = 0;
#define EXPECT(cond)                                                          \
    do {                                                                      \
        if (!(cond)) {                                                        \
            std::fprintf(stderr, "%s:%d: expected %s\n", __FILE__, __LINE__, #cond); \
            ++g_fail;                                                         \
        }                                                                     \
    } while (0)

// every failing call leaves a readable message
static void touch_error() {
    const char* e = jules_hip_last_error();
    EXPECT(e != nullptr);
    volatile size_t n = std::strlen(e);
    (void)n;
}

static const int kDims[] = {INT_MIN, -1, 0, 1, 2, 7, 8, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129,
                            255, 256, 257, 1023, 1024, 4096, 8192, 65535, 65536, 131071, 131072,
                            (1 << 26), (1 << 26) + 16, INT_MAX - 15, INT_MAX};

static void status_strings() {
    for (int s = -3; s < 20; ++s) {
        const char* t = jules_hip_status_string(s);
        EXPECT(t != nullptr);
        if (t) {
            volatile size_t n = std::strlen(t);
            (void)n;
        }
    }
    EXPECT(jules_hip_abi_version() > 0);
}

static void workspace_sizes() {
    for (int a : kDims)
        for (int b : kDims)
            for (int c : kDims) {
                (void)jules_hip_w8a16_workspace_size(a % 17, b, c);
                (void)jules_hip_flash_attn_bwd_workspace_size(a, b, c);
                (void)jules_hip_mlp_forward_workspace_size(a, b, c, 10);
                (void)jules_hip_mlp_workspace_size(a, b, c, 10);
            }
    for (int a : kDims) (void)jules_hip_cross_entropy_workspace_size(a);
    (void)jules_hip_w8a16_noalloc_max_bytes();
}

static void tile_table() {
    int out[4];
    for (int dt = -1; dt <= 2; ++dt)
        for (int m : kDims)
            for (int n : kDims)
                for (int k : kDims) {
                    const int st = jules_hip_gemm_tile(dt, m, n, k, out);
                    // tile_k is 0 only for K = 0 (the row kernel keeps all of K)
                    if (st == JH_OK)
                        EXPECT(out[0] >= 0 && out[0] <= 5 && out[1] > 0 && out[2] > 0 &&
                               (out[3] > 0 || (k == 0 && out[3] == 0)));
                    else touch_error();
                }
    EXPECT(jules_hip_gemm_tile(JH_F32, 64, 64, 64, nullptr) != JH_OK);
}

// Invalid requests must fail before touching a device; shapes that pass the
// checks reach the HIP runtime (no device here) and must fail cleanly too.
static void entry_point_checks() {
    alignas(16) static float buf[4096];
    float* f = buf;
    const void* odd = reinterpret_cast<const char*>(buf) + 2;
    for (int dt = -1; dt <= 2; ++dt)
        for (int act = -1; act <= 6; ++act)
            for (int m : {-1, 0, 1, 64, INT_MAX})
                for (int n : {-1, 0, 1, 64, INT_MAX})
                    for (int k : {-1, 0, 1, 64, INT_MAX}) {
                        int st = jules_hip_gemm_bias_act(dt, act, f, f, f, f, m, n, k, nullptr);
                        if (st != JH_OK) touch_error();
                        st = jules_hip_gemm_bias_act(dt, act, nullptr, odd, f, f, m, n, k, nullptr);
                        if (st != JH_OK) touch_error();
                    }
    for (int ta : {-1, 0, 1, 2})
        for (int tb : {0, 1, 7})
            for (int ld : {-1, 0, 1, 64, INT_MAX}) {
                const int st = jules_hip_sgemm(ta, tb, 64, 64, 64, 1.0f, f, ld, f, ld, 0.0f, f, ld, nullptr);
                if (st != JH_OK) touch_error();
            }
    for (int act = -1; act <= 6; ++act)
        for (int64_t n : {int64_t(-1), int64_t(0), int64_t(17), int64_t(1) << 41})
            if (jules_hip_activation(act, f, f, n, nullptr) != JH_OK) touch_error();
    for (int dt = -1; dt <= 2; ++dt)
        for (int causal = -1; causal <= 2; ++causal)
            for (float scale : {-1.0f, 0.0f, 0.125f, INFINITY, NAN})
                for (int d : {-1, 0, 1, 63, 64, 100, 128, 129, INT_MAX})
                    for (int s : {-1, 0, 1, 4097, INT_MAX}) {
                        int st = jules_hip_flash_attn_fwd(dt, causal, scale, f, f, f, f, nullptr, 2, 3, s, d,
                                                          nullptr);
                        if (st != JH_OK) touch_error();
                        st = jules_hip_flash_attn_bwd(dt, causal, scale, f, f, f, f, f, f, f, f, f, 2, 3, s, d,
                                                      f, 64, nullptr);
                        if (st != JH_OK) touch_error();
                    }
    for (int act = -1; act <= 6; ++act)
        for (int m : {-1, 0, 1, 8, 16, 17})
            for (int n : kDims)
                for (int k : {-1, 0, 8, 12, 8192, (1 << 26) + 8, INT_MAX - 7}) {
                    int st = jules_hip_w8a16_gemm_bias_act(act, f, reinterpret_cast<const int8_t*>(f), f, f, f, m,
                                                           n, k, f, 16, nullptr);
                    if (st != JH_OK) touch_error();
                    st = jules_hip_w8a16_gemm_bias_act_noalloc(act, f, reinterpret_cast<const int8_t*>(f), f,
                                                               nullptr, f, m, n, k, nullptr);
                    if (st != JH_OK) touch_error();
                }
    const int8_t* i8 = reinterpret_cast<const int8_t*>(buf);
    for (int m : {-1, 0, 1, 8, 4096})
        for (int k : {-1, 0, 16, 131071, 131072, INT_MAX}) {
            int st = jules_hip_matmul_int8(i8, i8, f, m, 64, k, 1.0f, 1.0f, nullptr, nullptr);
            if (st != JH_OK) touch_error();
            st = jules_hip_matmul_w8a8(i8, i8, f, m, 64, k, nullptr, f, nullptr, nullptr);
            if (st != JH_OK) touch_error();
        }
    for (int m : {-1, 0, 1, INT_MAX})
        for (int n : {-1, 0, 1, INT_MAX}) {
            if (jules_hip_softmax(f, f, m, n, nullptr) != JH_OK) touch_error();
            if (jules_hip_layernorm(f, f, f, f, m, n, 1e-5f, nullptr) != JH_OK) touch_error();
            if (jules_hip_layernorm(f, f, f, f, m, n, -1.0f, nullptr) != JH_OK) touch_error();
            if (jules_hip_layernorm(f, f, f, f, m, n, NAN, nullptr) != JH_OK) touch_error();
            const int32_t* tg = reinterpret_cast<const int32_t*>(buf);
            if (jules_hip_cross_entropy(f, tg, f, f, m, n, f, 4, nullptr) != JH_OK) touch_error();
            if (jules_hip_mlp_forward(f, f, f, f, f, f, m, n, 3, 4, f, 64, nullptr) != JH_OK) touch_error();
            if (jules_hip_mlp_forward_backward(f, f, f, f, f, tg, f, f, f, f, f, f, m, n, 3, 4, f, f, 64,
                                               nullptr) != JH_OK)
                touch_error();
        }
    for (int wg : {-1, 0, 1, 65536})
        for (int it : {-1, 0, 1}) {
            if (jules_hip_mfma_ceiling(f, wg, it, nullptr) != JH_OK) touch_error();
            if (jules_hip_hbm_read_floor(f, it * 1024, reinterpret_cast<uint32_t*>(f), wg, nullptr) != JH_OK)
                touch_error();
        }
}

static jh_tensor desc(void* p, std::initializer_list<int64_t> sizes, int dtype) {
    jh_tensor t;
    std::memset(&t, 0, sizeof t);
    t.data = p;
    t.rank = (int32_t)sizes.size();
    t.dtype = dtype;
    int i = 0;
    for (int64_t s : sizes) t.sizes[i++] = s;
    int64_t st = 1;
    for (int j = t.rank - 1; j >= 0; --j) {
        t.strides[j] = st;
        if (t.sizes[j] > 0 && st <= INT64_MAX / t.sizes[j]) st *= t.sizes[j];
    }
    return t;
}

// every registry kernel with well-formed, malformed and hostile descriptors
// and backend_config strings
static void registry() {
    alignas(16) static float buf[4096];
    const int n = jules_hip_kernel_count();
    EXPECT(n > 0);
    EXPECT(jules_hip_kernel_name(-1) == nullptr);
    EXPECT(jules_hip_kernel_name(n) == nullptr);
    EXPECT(jules_hip_lookup(nullptr) == nullptr);
    EXPECT(jules_hip_lookup("") == nullptr);
    EXPECT(jules_hip_lookup(std::string(5000, 'x').c_str()) == nullptr);
    touch_error();
    const std::string longcfg = "scale=" + std::string(3000, '9');
    const char* cfgs[] = {nullptr, "", "scale=", "scale=abc", "scale=1e40", "scale=-1", "scale=0.125",
                          "epsilon=", "epsilon=1e-5", "epsilon=nan", "scale_a=2,scale_b=", "scale_a=,scale_b=3",
                          "scale_a=2,scale_b=3", "scale_a=2;scale_b=3", "=,=,=", ",,,,", longcfg.c_str()};
    for (int i = 0; i < n; ++i) {
        const char* name = jules_hip_kernel_name(i);
        EXPECT(name != nullptr);
        jh_kernel_fn fn = jules_hip_lookup(name);
        EXPECT(fn != nullptr);
        if (!fn) continue;
        std::vector<std::vector<jh_tensor>> shapes;
        for (int dt : {(int)JH_F32, (int)JH_BF16, 9}) {
            shapes.push_back({desc(buf, {4, 8}, dt), desc(buf, {8, 16}, dt), desc(buf, {16}, dt),
                              desc(buf, {16}, dt), desc(buf, {16}, dt)});
            shapes.push_back({desc(buf, {1, 2, 16, 64}, dt), desc(buf, {1, 2, 16, 64}, dt),
                              desc(buf, {1, 2, 16, 64}, dt), desc(buf, {1}, dt), desc(buf, {1}, dt)});
            shapes.push_back({desc(buf, {}, dt), desc(buf, {}, dt), desc(buf, {}, dt), desc(buf, {}, dt),
                              desc(buf, {}, dt)});
            shapes.push_back({desc(buf, {-1, 8}, dt), desc(buf, {8, INT64_MAX}, dt), desc(nullptr, {16}, dt),
                              desc(buf, {16}, dt), desc(buf, {16}, dt)});
        }
        // ranks outside 0..6
        std::vector<jh_tensor> bad = {desc(buf, {4, 8}, JH_F32), desc(buf, {8, 16}, JH_F32),
                                      desc(buf, {16}, JH_F32), desc(buf, {16}, JH_F32), desc(buf, {16}, JH_F32)};
        bad[0].rank = 7;
        bad[1].rank = -1;
        bad[2].rank = INT32_MAX;
        shapes.push_back(bad);
        for (auto& in : shapes)
            for (int ni = 0; ni <= 5; ++ni)
                for (int no = 0; no <= 3; ++no)
                    for (const char* cfg : cfgs) {
                        std::vector<jh_tensor> out(3, desc(buf, {4, 16}, in[0].dtype));
                        const int st = fn(ni, in.data(), no, out.data(), cfg, nullptr);
                        if (st != JH_OK) touch_error();
                    }
        // null descriptor arrays
        if (fn(2, nullptr, 1, nullptr, nullptr, nullptr) != JH_OK) touch_error();
    }
}

static void cpp_api() {
    using namespace jules::kernel;
    const CacheInfo ci = CacheInfo::detect();
    (void)ci;
    TilePlanner planner;
    planner.setAutoTune(false);
    for (int m : kDims)
        for (int n : kDims)
            for (int k : kDims) {
                const TileConfig a = planner.computeAnalytical(m, n, k);
                (void)a.footprintBytes(m, n, k);
                (void)a.fitsInCache(1 << 20, m, n, k);
                if (m > 0 && n > 0 && k > 0 && m < 70000 && n < 70000 && k < 70000) {
                    const TileConfig b = planner.getTileConfig(m, n, k);
                    (void)b;
                }
            }
    for (int s : kDims)
        for (int d : {-1, 0, 64, 128, 256, 257})
            for (size_t l3 : {size_t(0), size_t(1) << 20, SIZE_MAX})
                (void)shouldUseFlashAttention(s, d, l3);
    {
        // no device: the arena holds no buffer and refuses every allocation
        ExecutionArena arena(1 << 20);
        for (size_t b : {size_t(0), size_t(1), size_t(255), size_t(1) << 19, size_t(1) << 21, SIZE_MAX,
                         SIZE_MAX - 300})
            (void)arena.allocateBytes(b);
        arena.reset();
        arena.resetAndZero();
        (void)arena.highWaterMark();
    }
    alignas(16) static float buf[1024];
    const int32_t* tg = reinterpret_cast<const int32_t*>(buf);
    const int8_t* i8 = reinterpret_cast<const int8_t*>(buf);
    ExecutionArena arena(1 << 16);
    fusedMatmulRelu(buf, buf, buf, -1, 4, 4);
    EXPECT(lastStatus() != JH_OK);
    fusedMatmulBiasRelu(buf, buf, nullptr, buf, 4, 4, 4);
    tiledMatmulWithActivation(buf, buf, buf, 4, -4, 4, TileConfig{}, ActivationType::Gelu);
    EXPECT(lastStatus() != JH_OK);
    tiledMatmulWithActivation(buf, buf, buf, 4, 4, 4, TileConfig{-1, 0, INT_MAX}, ActivationType::Silu);
    blasMatmul(buf, buf, buf, 4, 4, -1);
    EXPECT(lastStatus() != JH_OK);
    blasMatmul(buf, buf, buf, 4, 4, 4, 2.0f, 1.0f, true, true);
    fusedGelu(buf, buf, -5);
    fusedSoftmax(buf, buf, -1, 3);
    fusedLayerNorm(buf, buf, buf, buf, 2, -3);
    (void)fusedCrossEntropyLoss(buf, tg, buf, -2, 3);
    matmulInt8(i8, i8, buf, 4, 4, INT_MAX, 1.0f, 1.0f);
    flashAttention(buf, buf, buf, buf, 1, 1, -4, 64, arena, planner);
    attention(buf, buf, buf, buf, 1, 1, 4, 300, arena, planner);
    standardAttention(buf, buf, buf, buf, 1, 1, -1, 64, arena);
    MLPParams mp{buf, buf, buf, buf, -1, 4, 4, 4};
    fusedMLPForward(buf, buf, mp, arena, planner);
    (void)interleavedMLPForwardBackward(buf, buf, buf, buf, buf, tg, buf, buf, buf, buf, buf, buf, 4, -1,
                                        4, 4, arena, planner);
    EXPECT(lastError() != nullptr);
}

static void pjrt() {
    const std::string deep(2000, '(');
    const std::string many = [] {
        std::string p;
        for (int i = 0; i < 200; ++i)
            p += "%" + std::to_string(i + 2) + " = stablehlo.add %arg0, %" + std::to_string(i + 1) +
                 " : tensor<4xf32>\n";
        return p;
    }();
    const char* programs[] = {
        nullptr,
        "",
        "garbage",
        "%0 = stablehlo.add %arg0, %arg1 : tensor<4xf32>",
        "%0 = stablehlo.dot_general %arg0, %arg1, contracting_dims = [1] x [0] : "
        "(tensor<2x3xf32>, tensor<3x4xf32>) -> tensor<2x4xf32>",
        "%0 = stablehlo.transpose %arg0, dims = [1, 0] : (tensor<2x3xf32>) -> tensor<3x2xf32>",
        "%0 = stablehlo.transpose %arg0, dims = [7, -1, 99999999999] : (tensor<2x3xf32>) -> tensor<3x2xf32>",
        "%0 = stablehlo.reduce(%arg0 init: %arg1) applies stablehlo.add across dimensions = [9] : "
        "(tensor<2x3xf32>, tensor<f32>) -> tensor<2xf32>",
        "%0 = stablehlo.constant dense<[1.0, 2.0, nan, 1e400]> : tensor<4xf32>",
        "%0 = stablehlo.reshape %arg0 : (tensor<2x3xf32>) -> tensor<99999999999999999999x6xf32>",
        "%0 = \"stablehlo.custom_call\"(%arg0) {call_target_name = \"gelu\"} : (tensor<4xf32>) -> tensor<4xf32>",
        "%0 = \"stablehlo.custom_call\"(%arg0) {call_target_name = \"nope\", backend_config = \"scale=\"} "
        ": (tensor<4xf32>) -> tensor<4xf32>",
        "%r:2 = \"stablehlo.custom_call\"(%arg0, %arg1) {call_target_name = \"fusedCrossEntropyLoss\"} : "
        "(tensor<2x3xf32>, tensor<2xi32>) -> (tensor<2x3xf32>, tensor<f32>)\n%1 = stablehlo.add %r#1, %r#7 : "
        "tensor<f32>",
        "%0 = stablehlo.add %arg99999999999999999999, %arg1 : tensor<4xf32>",
        "%0 = stablehlo.add %arg0, %arg1 : tensor<>",
        "%0 = stablehlo.add %arg0, %arg1 : tensor<4x",
        many.c_str(),
        deep.c_str()};
    for (const char* p : programs)
        for (int ni : {-1, 0, 1, 3, 64})
            for (size_t len : {size_t(0), size_t(1), size_t(8), size_t(4096)}) {
                std::vector<char> out(len + 1, 'Z');
                const int st = jules_hip_pjrt_describe(p, ni, len ? out.data() : nullptr, len);
                if (st != JH_OK) touch_error();
                if (st == JH_OK && len) EXPECT(std::memchr(out.data(), 0, len) != nullptr);
                EXPECT(out[len] == 'Z');  // nothing written past buf_len
            }
    jh_pjrt_exe* exe = nullptr;
    if (jules_hip_pjrt_compile(programs[3], 0, &exe) == JH_OK && exe) (void)jules_hip_pjrt_destroy(exe);
    EXPECT(jules_hip_pjrt_compile(nullptr, 0, &exe) != JH_OK);
    EXPECT(jules_hip_pjrt_destroy(nullptr) != JH_OK || true);
    int nout = 0;
    EXPECT(jules_hip_pjrt_execute(nullptr, 0, nullptr, 0, nullptr, &nout) != JH_OK);
}

static void cblas() {
    alignas(16) static float buf[256];
    for (int order : {0, 101, 102})
        for (int ta : {0, 111, 112, 113, 114})
            for (int m : {-1, 0, 4})
                for (int ld : {-1, 0, 1, 4, INT_MAX}) {
                    cblas_sgemm(order, ta, 111, m, 4, 4, 1.0f, buf, ld, buf, ld, 0.0f, buf, ld);
                    (void)jules_cblas_last_status();
                }
    cblas_sgemm(101, 111, 111, 4, 4, 4, 1.0f, nullptr, 4, buf, 4, 0.0f, buf, 4);
    EXPECT(jules_cblas_last_status() != JH_OK);
}

int main() {
    status_strings();
    workspace_sizes();
    tile_table();
    entry_point_checks();
    registry();
    cpp_api();
    pjrt();
    cblas();
    std::printf("host_sanitize: %d failed expectations\n", g_fail);
    return g_fail == 0 ? 0 : 1;
}
