// capi.cpp - the extern "C" boundary of libjules_hip.so (declared in
// include/jules_hip.h): argument validation, status codes, and the
// extern_kernel / custom_call name registry.
//
// Every entry point checks its arguments before touching the device and
// returns a jh_status; nothing here aborts (the reference kernels validate
// nothing and abort() on arena overflow, ExecutionArena.h:140-143).
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstdint>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include "jules_hip.h"
#include "launch.hpp"
#include "tiles.hpp"

namespace {

thread_local std::string g_last_error;

int fail(int status, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return status;
}

int check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return JH_OK;
    return fail(JH_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
bool valid_act(int act) { return act >= JH_ACT_NONE && act <= JH_ACT_SILU; }

// element-count limit: every index is computed in 64-bit, this only guards
// against sizes whose products overflow int64 in the caller's arithmetic.
constexpr int64_t kMaxElems = int64_t(1) << 40;

// largest int8 GEMM depth whose int32 sums cannot overflow: every product
// is at most (-128)*(-128) = 2^14, and 131071 * 2^14 < 2^31
constexpr int kMaxInt8K = 131071;
// W8A16 decode: x and one k-step of W are addressed with 32-bit buffer offsets
constexpr int kMaxDecodeDim = 1 << 26;

}  // namespace

namespace jh {
// Lets other translation units of the library (pjrt.cpp) report through
// jules_hip_last_error().
int set_last_error(int status, const std::string& message) {
    g_last_error = message;
    return status;
}

// jules_hip_gemm_bias_act for fp32 with a chosen kernel of the tile table
// (variant < 0: the table's default for the shape).  Every variant gives the
// same bits, so the choice changes speed only.
int gemm_f32_with_variant(int variant, int act, const float* A, const float* B, const float* bias,
                          float* C, int M, int N, int K, hipStream_t s) {
    if (!valid_act(act)) return fail(JH_ERR_ACT, "gemm: activation code %d", act);
    if (M < 0 || N < 0 || K < 0) return fail(JH_ERR_SHAPE, "gemm: M=%d N=%d K=%d", M, N, K);
    if ((int64_t)M * K > kMaxElems || (int64_t)K * N > kMaxElems || (int64_t)M * N > kMaxElems)
        return fail(JH_ERR_SHAPE, "gemm: M=%d N=%d K=%d too large", M, N, K);
    if (variant < 0) variant = f32_gemm_tile(M, N, K).variant;
    if (!f32_variant_valid(variant, K))
        return fail(JH_ERR_ARG, "gemm f32: kernel variant %d cannot run K=%d", variant, K);
    if (M == 0 || N == 0) return JH_OK;
    if (!C || (K > 0 && (!A || !B))) return fail(JH_ERR_NULL, "gemm: null A, B or C");
    if (!aligned(A, 4) || !aligned(B, 4) || !aligned(C, 4) || !aligned(bias, 4))
        return fail(JH_ERR_ALIGN, "gemm f32: operands must be 4-byte aligned");
    return check_hip(launch_gemm_f32_variant(variant, act, A, B, bias, C, M, N, K, s),
                     "gemm f32 launch");
}
}  // namespace jh

extern "C" {

int jules_hip_abi_version(void) { return JULES_HIP_ABI_VERSION; }

const char* jules_hip_status_string(int status) {
    switch (status) {
    case JH_OK: return "ok";
    case JH_ERR_NULL: return "null pointer";
    case JH_ERR_SHAPE: return "invalid shape";
    case JH_ERR_DTYPE: return "unsupported dtype";
    case JH_ERR_ALIGN: return "misaligned pointer";
    case JH_ERR_ACT: return "unknown activation";
    case JH_ERR_WORKSPACE: return "workspace missing or too small";
    case JH_ERR_HIP: return "HIP runtime error";
    case JH_ERR_UNSUPPORTED: return "unsupported configuration";
    case JH_ERR_NOT_FOUND: return "unknown kernel name";
    case JH_ERR_ARG: return "invalid argument";
    default: return "unknown status";
    }
}

const char* jules_hip_last_error(void) { return g_last_error.c_str(); }

int jules_hip_gemm_bias_act(int dtype, int act, const void* A, const void* B, const float* bias,
                            void* C, int M, int N, int K, void* stream) {
    if (!valid_act(act)) return fail(JH_ERR_ACT, "gemm: activation code %d", act);
    if (M < 0 || N < 0 || K < 0) return fail(JH_ERR_SHAPE, "gemm: M=%d N=%d K=%d", M, N, K);
    if ((int64_t)M * K > kMaxElems || (int64_t)K * N > kMaxElems || (int64_t)M * N > kMaxElems)
        return fail(JH_ERR_SHAPE, "gemm: M=%d N=%d K=%d too large", M, N, K);
    if (dtype != JH_F32 && dtype != JH_BF16) return fail(JH_ERR_DTYPE, "gemm: dtype %d", dtype);
    if (dtype == JH_F32)
        return jh::gemm_f32_with_variant(-1, act, static_cast<const float*>(A),
                                         static_cast<const float*>(B), bias, static_cast<float*>(C),
                                         M, N, K, static_cast<hipStream_t>(stream));
    if (M == 0 || N == 0) return JH_OK;
    if (!C || (K > 0 && (!A || !B))) return fail(JH_ERR_NULL, "gemm: null A, B or C");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (M % 8 || N % 8 || K % 8)
        return fail(JH_ERR_UNSUPPORTED, "gemm bf16: M, N, K must be multiples of 8 (got %d %d %d)",
                    M, N, K);
    if (!aligned(A, 16) || !aligned(B, 16) || !aligned(C, 2) || !aligned(bias, 4))
        return fail(JH_ERR_ALIGN, "gemm bf16: A and B must be 16-byte aligned");
    return check_hip(jh::launch_gemm_bf16(act, static_cast<const uint16_t*>(A),
                                          static_cast<const uint16_t*>(B), bias,
                                          static_cast<uint16_t*>(C), M, N, K, s),
                     "gemm bf16 launch");
}

int jules_hip_gemm_tile(int dtype, int M, int N, int K, int* out) {
    if (!out) return fail(JH_ERR_NULL, "gemm_tile: null out");
    if (M < 0 || N < 0 || K < 0) return fail(JH_ERR_SHAPE, "gemm_tile: M=%d N=%d K=%d", M, N, K);
    if (dtype != JH_F32 && dtype != JH_BF16) return fail(JH_ERR_DTYPE, "gemm_tile: dtype %d", dtype);
    const jh::GemmTile t = dtype == JH_F32 ? jh::f32_gemm_tile(M, N, K) : jh::bf16_gemm_tile(M, N, K);
    out[0] = t.variant;
    out[1] = t.tile_m;
    out[2] = t.tile_n;
    out[3] = t.tile_k;
    return JH_OK;
}

int jules_hip_sgemm(int transA, int transB, int M, int N, int K, float alpha, const float* A,
                    int lda, const float* B, int ldb, float beta, float* C, int ldc, void* stream) {
    if ((transA != 0 && transA != 1) || (transB != 0 && transB != 1))
        return fail(JH_ERR_ARG, "sgemm: transA/transB must be 0 or 1 (got %d, %d)", transA, transB);
    if (M < 0 || N < 0 || K < 0) return fail(JH_ERR_SHAPE, "sgemm: M=%d N=%d K=%d", M, N, K);
    // BLAS leading-dimension rules for row-major storage
    const int a_cols = transA ? M : K, b_cols = transB ? K : N;
    if (lda < (a_cols > 1 ? a_cols : 1) || ldb < (b_cols > 1 ? b_cols : 1) || ldc < (N > 1 ? N : 1))
        return fail(JH_ERR_SHAPE, "sgemm: lda=%d ldb=%d ldc=%d below the row lengths %d %d %d", lda,
                    ldb, ldc, a_cols, b_cols, N);
    const int64_t a_rows = transA ? K : M, b_rows = transB ? N : K;
    if (a_rows * lda > kMaxElems || b_rows * ldb > kMaxElems || (int64_t)M * ldc > kMaxElems)
        return fail(JH_ERR_SHAPE, "sgemm: too large");
    if (M == 0 || N == 0) return JH_OK;
    const bool product = K > 0 && alpha != 0.0f;
    if (!C || (product && (!A || !B))) return fail(JH_ERR_NULL, "sgemm: null A, B or C");
    if (!aligned(A, 4) || !aligned(B, 4) || !aligned(C, 4))
        return fail(JH_ERR_ALIGN, "sgemm: operands must be 4-byte aligned");
    hipStream_t s = static_cast<hipStream_t>(stream);
    // The call LLVMBackend emits (LLVMBackend.cpp:1242-1255): plain C = A B
    // on dense operands.  It runs the fp32 fma-chain GEMM, whose bits equal
    // the reference's tiledMatmulWithActivation.
    if (!transA && !transB && alpha == 1.0f && beta == 0.0f && lda == K && ldb == N && ldc == N)
        return check_hip(jh::launch_gemm_f32(JH_ACT_NONE, A, B, nullptr, C, M, N, K, s),
                         "sgemm launch");
    return check_hip(jh::launch_sgemm(transA, transB, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s),
                     "sgemm launch");
}

int jules_hip_activation(int act, float* out, const float* in, int64_t n, void* stream) {
    if (!valid_act(act)) return fail(JH_ERR_ACT, "activation: code %d", act);
    if (n < 0 || n > kMaxElems) return fail(JH_ERR_SHAPE, "activation: n=%lld", (long long)n);
    if (n == 0) return JH_OK;
    if (!out || !in) return fail(JH_ERR_NULL, "activation: null pointer");
    if (!aligned(out, 4) || !aligned(in, 4)) return fail(JH_ERR_ALIGN, "activation: alignment");
    return check_hip(jh::launch_activation(act, out, in, n, static_cast<hipStream_t>(stream)),
                     "activation launch");
}

int jules_hip_flash_attn_fwd(int dtype, int causal, float scale, const void* Q, const void* K,
                             const void* V, void* O, float* lse, int B, int H, int S, int D,
                             void* stream) {
    if (dtype != JH_F32 && dtype != JH_BF16) return fail(JH_ERR_DTYPE, "flash: dtype %d", dtype);
    if (B < 0 || H < 0 || S < 0) return fail(JH_ERR_SHAPE, "flash: B=%d H=%d S=%d", B, H, S);
    if (D < 1) return fail(JH_ERR_SHAPE, "flash: head_dim %d", D);
    if (D > 128) return fail(JH_ERR_UNSUPPORTED, "flash: head_dim %d (at most 128)", D);
    if (!(std::isfinite(scale) && scale > 0.0f)) return fail(JH_ERR_ARG, "flash: scale %g", scale);
    if (causal != 0 && causal != 1) return fail(JH_ERR_ARG, "flash: causal must be 0 or 1");
    if ((int64_t)B * H * S * D > kMaxElems) return fail(JH_ERR_SHAPE, "flash: too large");
    if (B == 0 || H == 0 || S == 0) return JH_OK;
    if (!Q || !K || !V || !O) return fail(JH_ERR_NULL, "flash: null Q, K, V or O");
    if (!aligned(Q, 16) || !aligned(K, 16) || !aligned(V, 16) || !aligned(O, 16) ||
        !aligned(lse, 4))
        return fail(JH_ERR_ALIGN, "flash: Q, K, V, O must be 16-byte aligned");
    if (D != 64 && D != 128)
        return check_hip(jh::launch_flash_fwd_padded(dtype, causal, scale, Q, K, V, O, lse, B, H, S, D,
                                                     static_cast<hipStream_t>(stream)),
                         "flash launch (padded head dim)");
    return check_hip(jh::launch_flash_fwd(dtype, causal, scale, Q, K, V, O, lse, B, H, S, D,
                                          static_cast<hipStream_t>(stream)),
                     "flash launch");
}

size_t jules_hip_flash_attn_bwd_workspace_size(int B, int H, int S) {
    if (B < 0 || H < 0 || S < 0) return 0;
    return jh::flash_bwd_workspace_size(B, H, S);
}

int jules_hip_flash_attn_bwd(int dtype, int causal, float scale, const void* Q, const void* K,
                             const void* V, const void* O, const void* dO, const float* lse,
                             void* dQ, void* dK, void* dV, int B, int H, int S, int D,
                             void* workspace, size_t workspace_bytes, void* stream) {
    if (dtype != JH_F32 && dtype != JH_BF16) return fail(JH_ERR_DTYPE, "flash bwd: dtype %d", dtype);
    if (B < 0 || H < 0 || S < 0) return fail(JH_ERR_SHAPE, "flash bwd: B=%d H=%d S=%d", B, H, S);
    if (D < 1) return fail(JH_ERR_SHAPE, "flash bwd: head_dim %d", D);
    if (D > 128) return fail(JH_ERR_UNSUPPORTED, "flash bwd: head_dim %d (at most 128)", D);
    if (dtype != JH_BF16) return fail(JH_ERR_UNSUPPORTED, "flash bwd: only bf16 is implemented");
    if (!(std::isfinite(scale) && scale > 0.0f)) return fail(JH_ERR_ARG, "flash bwd: scale %g", scale);
    if (causal != 0 && causal != 1) return fail(JH_ERR_ARG, "flash bwd: causal must be 0 or 1");
    if ((int64_t)B * H * S * D > kMaxElems) return fail(JH_ERR_SHAPE, "flash bwd: too large");
    if (B == 0 || H == 0 || S == 0) return JH_OK;
    if (!Q || !K || !V || !O || !dO || !lse || !dQ || !dK || !dV)
        return fail(JH_ERR_NULL, "flash bwd: null operand");
    const void* t16[] = {Q, K, V, O, dO, dQ, dK, dV};
    for (const void* q : t16)
        if (!aligned(q, 16)) return fail(JH_ERR_ALIGN, "flash bwd: tensors must be 16-byte aligned");
    if (!aligned(lse, 4)) return fail(JH_ERR_ALIGN, "flash bwd: lse alignment");
    const size_t need = jh::flash_bwd_workspace_size(B, H, S);
    if (!workspace || workspace_bytes < need)
        return fail(JH_ERR_WORKSPACE, "flash bwd: workspace %zu bytes, need %zu", workspace_bytes, need);
    if (!aligned(workspace, 4)) return fail(JH_ERR_ALIGN, "flash bwd: workspace alignment");
    if (D != 64 && D != 128)
        return check_hip(jh::launch_flash_bwd_padded(dtype, causal, scale, Q, K, V, O, dO, lse, dQ, dK,
                                                     dV, B, H, S, D, workspace,
                                                     static_cast<hipStream_t>(stream)),
                         "flash bwd launch (padded head dim)");
    return check_hip(jh::launch_flash_bwd(dtype, causal, scale, Q, K, V, O, dO, lse, dQ, dK, dV, B,
                                          H, S, D, workspace, static_cast<hipStream_t>(stream)),
                     "flash bwd launch");
}

size_t jules_hip_w8a16_workspace_size(int M, int N, int K) {
    if (M < 1 || M > 16 || N < 16 || N % 16 || K < 8 || K % 8) return 0;
    return jh::w8a16_workspace_size(M, N, K);
}

// argument checks shared by the two W8A16 entry points; *done is set when
// there is nothing to compute (M = 0 or N = 0)
static int w8a16_check(const char* who, int act, const void* x, const int8_t* W, const float* scale,
                       const float* bias, const void* y, int M, int N, int K, bool* done) {
    *done = false;
    if (!valid_act(act)) return fail(JH_ERR_ACT, "%s: activation code %d", who, act);
    if (M < 0 || N < 0 || K < 0) return fail(JH_ERR_SHAPE, "%s: M=%d N=%d K=%d", who, M, N, K);
    if (M == 0 || N == 0) {
        *done = true;
        return JH_OK;
    }
    if (M > 16 || N % 16 || K % 8 || K == 0 || N > kMaxDecodeDim || K > kMaxDecodeDim)
        return fail(JH_ERR_UNSUPPORTED,
                    "%s: needs 1<=M<=16, N%%16==0, K%%8==0, 0<K<=2^26, N<=2^26 (got %d %d %d)", who, M,
                    N, K);
    if ((int64_t)K * N > kMaxElems) return fail(JH_ERR_SHAPE, "%s: too large", who);
    if (!x || !W || !scale || !y) return fail(JH_ERR_NULL, "%s: null x, W, scale or y", who);
    if (!aligned(W, 16) || !aligned(x, 16) || !aligned(y, 8) || !aligned(scale, 4) ||
        !aligned(bias, 4))
        return fail(JH_ERR_ALIGN, "%s: W, x 16-byte, y 8-byte, scale/bias 4-byte alignment", who);
    return JH_OK;
}

int jules_hip_w8a16_gemm_bias_act(int act, const void* x, const int8_t* W, const float* scale,
                                  const float* bias, void* y, int M, int N, int K,
                                  void* workspace, size_t workspace_bytes, void* stream) {
    bool done = false;
    const int st = w8a16_check("w8a16", act, x, W, scale, bias, y, M, N, K, &done);
    if (st != JH_OK || done) return st;
    const size_t need = jh::w8a16_workspace_size(M, N, K);
    if (need > 0 && (!workspace || workspace_bytes < need))
        return fail(JH_ERR_WORKSPACE, "w8a16: workspace %zu bytes, need %zu", workspace_bytes, need);
    if (!aligned(workspace, 16)) return fail(JH_ERR_ALIGN, "w8a16: workspace alignment");
    return check_hip(jh::launch_w8a16(act, static_cast<const uint16_t*>(x), W, scale, bias,
                                      static_cast<uint16_t*>(y), M, N, K, workspace,
                                      static_cast<hipStream_t>(stream)),
                     "w8a16 launch");
}

size_t jules_hip_w8a16_packed_size(int K, int N) {
    if (K <= 0 || N <= 0 || K > kMaxDecodeDim || N > kMaxDecodeDim || (int64_t)K * N > kMaxElems)
        return 0;
    return jh::w8a16_packed_bytes(K, N);
}

int jules_hip_w8a16_pack(const int8_t* W, int K, int N, void* Wp, size_t Wp_bytes, void* stream) {
    if (K < 0 || N < 0) return fail(JH_ERR_SHAPE, "w8a16 pack: K=%d N=%d", K, N);
    if (K == 0 || N == 0) return JH_OK;
    if (N % 16 || K % 8 || N > kMaxDecodeDim || K > kMaxDecodeDim)
        return fail(JH_ERR_UNSUPPORTED, "w8a16 pack: needs N%%16==0, K%%8==0, K,N<=2^26 (got %d %d)", K,
                    N);
    if ((int64_t)K * N > kMaxElems) return fail(JH_ERR_SHAPE, "w8a16 pack: too large");
    if (!W || !Wp) return fail(JH_ERR_NULL, "w8a16 pack: null W or Wp");
    if (!aligned(Wp, 16)) return fail(JH_ERR_ALIGN, "w8a16 pack: Wp 16-byte alignment");
    const size_t need = jh::w8a16_packed_bytes(K, N);
    if (Wp_bytes < need)
        return fail(JH_ERR_WORKSPACE, "w8a16 pack: Wp holds %zu bytes, need %zu", Wp_bytes, need);
    return check_hip(jh::launch_w8a16_pack(W, K, N, static_cast<int8_t*>(Wp),
                                           static_cast<hipStream_t>(stream)),
                     "w8a16 pack launch");
}

int jules_hip_w8a16_packed_gemm_bias_act(int act, const void* x, const void* Wp, const float* scale,
                                         const float* bias, void* y, int M, int N, int K,
                                         void* stream) {
    bool done = false;
    const int st = w8a16_check("w8a16 packed", act, x, static_cast<const int8_t*>(Wp), scale, bias, y,
                               M, N, K, &done);
    if (st != JH_OK || done) return st;
    return check_hip(jh::launch_w8a16_packed(act, static_cast<const uint16_t*>(x),
                                             static_cast<const int8_t*>(Wp), scale, bias,
                                             static_cast<uint16_t*>(y), M, N, K,
                                             static_cast<hipStream_t>(stream)),
                     "w8a16 packed launch");
}

size_t jules_hip_w8a16_noalloc_max_bytes(void) { return jh::static_scratch_bytes(); }

int jules_hip_w8a16_gemm_bias_act_noalloc(int act, const void* x, const int8_t* W,
                                          const float* scale, const float* bias, void* y, int M,
                                          int N, int K, void* stream) {
    bool done = false;
    const int st = w8a16_check("w8a16 noalloc", act, x, W, scale, bias, y, M, N, K, &done);
    if (st != JH_OK || done) return st;
    const size_t need = jh::w8a16_partials_size(M, N, K);
    if (need > jh::static_scratch_partial_bytes() || N > 16384)
        return fail(JH_ERR_WORKSPACE,
                    "w8a16 noalloc: M=%d N=%d K=%d needs %zu bytes of partials, the library's "
                    "static scratch holds %zu (N <= 16384 fits at any K)",
                    M, N, K, need, jh::static_scratch_partial_bytes());
    void* ws = nullptr;
    const int hst = check_hip(jh::static_scratch(&ws), "w8a16 noalloc: scratch address");
    if (hst != JH_OK) return hst;
    // partials first, the per-tile counters at a fixed offset after them
    char* base = static_cast<char*>(ws);
    return check_hip(jh::launch_w8a16_counters(
                         act, static_cast<const uint16_t*>(x), W, scale, bias,
                         static_cast<uint16_t*>(y), M, N, K, reinterpret_cast<float*>(base),
                         reinterpret_cast<uint32_t*>(base + jh::static_scratch_partial_bytes()),
                         static_cast<hipStream_t>(stream)),
                     "w8a16 noalloc launch");
}

int jules_hip_w8a16_noalloc_counters(uint32_t* out, int n) {
    const int words = 4096 / (int)sizeof(uint32_t);
    if (n < 0 || n > words) return fail(JH_ERR_ARG, "w8a16 noalloc counters: n=%d (0..%d)", n, words);
    if (n == 0) return JH_OK;
    if (!out) return fail(JH_ERR_NULL, "w8a16 noalloc counters: out is NULL");
    void* ws = nullptr;
    int st = check_hip(jh::static_scratch(&ws), "w8a16 noalloc counters: scratch address");
    if (st != JH_OK) return st;
    st = check_hip(hipDeviceSynchronize(), "w8a16 noalloc counters: device");
    if (st != JH_OK) return st;
    return check_hip(hipMemcpy(out, static_cast<char*>(ws) + jh::static_scratch_partial_bytes(),
                               sizeof(uint32_t) * (size_t)n, hipMemcpyDeviceToHost),
                     "w8a16 noalloc counters: copy");
}

int jules_hip_matmul_int8(const int8_t* A, const int8_t* B, float* C, int M, int N, int K,
                          float scale_A, float scale_B, const float* bias, void* stream) {
    if (M < 0 || N < 0 || K < 0) return fail(JH_ERR_SHAPE, "matmulInt8: M=%d N=%d K=%d", M, N, K);
    // |sum| <= K * 128 * 128 < 2^31 for K <= 131071: the int32 sum is exact
    if (K > kMaxInt8K) return fail(JH_ERR_SHAPE, "matmulInt8: K=%d exceeds exact int32 range", K);
    if ((int64_t)M * K > kMaxElems || (int64_t)K * N > kMaxElems || (int64_t)M * N > kMaxElems)
        return fail(JH_ERR_SHAPE, "matmulInt8: too large");
    if (M == 0 || N == 0) return JH_OK;
    if (!C || (K > 0 && (!A || !B))) return fail(JH_ERR_NULL, "matmulInt8: null A, B or C");
    if (!aligned(C, 4) || !aligned(bias, 4)) return fail(JH_ERR_ALIGN, "matmulInt8: alignment");
    return check_hip(jh::launch_matmul_int8(A, B, C, M, N, K, scale_A, scale_B, bias,
                                            static_cast<hipStream_t>(stream)),
                     "matmulInt8 launch");
}

int jules_hip_matmul_w8a8(const int8_t* A, const int8_t* B, float* C, int M, int N, int K,
                          const float* scale_A, const float* scale_B, const float* bias,
                          void* stream) {
    if (M < 0 || N < 0 || K < 0) return fail(JH_ERR_SHAPE, "matmulW8A8: M=%d N=%d K=%d", M, N, K);
    if (K > kMaxInt8K) return fail(JH_ERR_SHAPE, "matmulW8A8: K=%d exceeds exact int32 range", K);
    if ((int64_t)M * K > kMaxElems || (int64_t)K * N > kMaxElems || (int64_t)M * N > kMaxElems)
        return fail(JH_ERR_SHAPE, "matmulW8A8: too large");
    if (M == 0 || N == 0) return JH_OK;
    if (!C || !scale_B || (K > 0 && (!A || !B)))
        return fail(JH_ERR_NULL, "matmulW8A8: null A, B, C or scale_B");
    if (!aligned(C, 4) || !aligned(bias, 4) || !aligned(scale_A, 4) || !aligned(scale_B, 4))
        return fail(JH_ERR_ALIGN, "matmulW8A8: alignment");
    return check_hip(jh::launch_matmul_w8a8(A, B, C, M, N, K, scale_A, scale_B, bias,
                                            static_cast<hipStream_t>(stream)),
                     "matmulW8A8 launch");
}

// Row kernels (reference FusedKernels.h:464-526, :532-600, :766-854).
static int row_shape(const char* who, int M, int N) {
    if (M < 0 || N < 0) return fail(JH_ERR_SHAPE, "%s: M=%d N=%d", who, M, N);
    if ((int64_t)M * N > kMaxElems) return fail(JH_ERR_SHAPE, "%s: M=%d N=%d too large", who, M, N);
    return JH_OK;
}

int jules_hip_softmax(float* out, const float* in, int M, int N, void* stream) {
    int st = row_shape("softmax", M, N);
    if (st != JH_OK) return st;
    if (M == 0 || N == 0) return JH_OK;
    if (!out || !in) return fail(JH_ERR_NULL, "softmax: null pointer");
    if (!aligned(out, 4) || !aligned(in, 4)) return fail(JH_ERR_ALIGN, "softmax: alignment");
    return check_hip(jh::launch_softmax(out, in, M, N, static_cast<hipStream_t>(stream)),
                     "softmax launch");
}

int jules_hip_layernorm(float* out, const float* in, const float* gamma, const float* beta,
                        int M, int N, float epsilon, void* stream) {
    int st = row_shape("layernorm", M, N);
    if (st != JH_OK) return st;
    if (!(std::isfinite(epsilon) && epsilon >= 0.0f))
        return fail(JH_ERR_ARG, "layernorm: epsilon %g", epsilon);
    if (M == 0 || N == 0) return JH_OK;
    if (!out || !in || !gamma || !beta) return fail(JH_ERR_NULL, "layernorm: null pointer");
    if (!aligned(out, 4) || !aligned(in, 4) || !aligned(gamma, 4) || !aligned(beta, 4))
        return fail(JH_ERR_ALIGN, "layernorm: alignment");
    return check_hip(jh::launch_layernorm(out, in, gamma, beta, M, N, epsilon,
                                          static_cast<hipStream_t>(stream)),
                     "layernorm launch");
}

int jules_hip_mfma_ceiling(float* out, int workgroups, int iters, void* stream) {
    if (!out) return fail(JH_ERR_NULL, "mfma_ceiling: null out");
    if (!aligned(out, 4)) return fail(JH_ERR_ALIGN, "mfma_ceiling: out must be 4-byte aligned");
    if (workgroups < 1 || workgroups > 65535 || iters < 1 || iters > (1 << 20))
        return fail(JH_ERR_SHAPE, "mfma_ceiling: workgroups %d (1..65535), iters %d (1..1048576)",
                    workgroups, iters);
    return check_hip(jh::launch_mfma_ceiling(out, workgroups, iters, static_cast<hipStream_t>(stream)),
                     "mfma_ceiling");
}

int jules_hip_hbm_read_floor(const void* buf, int64_t bytes, uint32_t* out, int workgroups,
                             void* stream) {
    if (!buf || !out) return fail(JH_ERR_NULL, "hbm_read_floor: null buffer or out");
    if (!aligned(buf, 16) || !aligned(out, 4))
        return fail(JH_ERR_ALIGN, "hbm_read_floor: buf 16-byte, out 4-byte alignment");
    if (bytes < 16 || bytes % 16 || bytes > (int64_t(1) << 40))
        return fail(JH_ERR_SHAPE, "hbm_read_floor: bytes %lld (a multiple of 16, >= 16)",
                    (long long)bytes);
    if (workgroups < 1 || workgroups > 65535)
        return fail(JH_ERR_SHAPE, "hbm_read_floor: workgroups %d (1..65535)", workgroups);
    return check_hip(jh::launch_hbm_read(buf, bytes, out, workgroups, static_cast<hipStream_t>(stream)),
                     "hbm_read_floor");
}

size_t jules_hip_cross_entropy_workspace_size(int M) {
    return M > 0 ? (size_t)M * sizeof(float) : sizeof(float);
}

int jules_hip_cross_entropy(const float* logits, const int32_t* targets, float* grad, float* loss,
                            int M, int N, void* workspace, size_t workspace_bytes, void* stream) {
    int st = row_shape("cross_entropy", M, N);
    if (st != JH_OK) return st;
    if (M > 0 && N == 0) return fail(JH_ERR_SHAPE, "cross_entropy: N=0 with M=%d rows", M);
    if (!loss) return fail(JH_ERR_NULL, "cross_entropy: null loss");
    if (M > 0 && (!logits || !targets || !grad))
        return fail(JH_ERR_NULL, "cross_entropy: null logits, targets or grad");
    if (!workspace || workspace_bytes < jules_hip_cross_entropy_workspace_size(M))
        return fail(JH_ERR_WORKSPACE, "cross_entropy: workspace needs %zu bytes",
                    jules_hip_cross_entropy_workspace_size(M));
    if (!aligned(logits, 4) || !aligned(targets, 4) || !aligned(grad, 4) || !aligned(loss, 4) ||
        !aligned(workspace, 4))
        return fail(JH_ERR_ALIGN, "cross_entropy: alignment");
    return check_hip(jh::launch_cross_entropy(logits, targets, grad, loss,
                                              static_cast<float*>(workspace), M, N,
                                              static_cast<hipStream_t>(stream)),
                     "cross_entropy launch");
}

size_t jules_hip_mlp_forward_workspace_size(int M, int K1, int N1, int N2) {
    if (M < 0 || K1 < 1 || N1 < 1 || N2 < 1) return 0;
    return jh::mlp_forward_workspace_size(M, K1, N1, N2);
}

int jules_hip_mlp_forward(const float* X, const float* W1, const float* b1, const float* W2,
                          const float* b2, float* output, int M, int K1, int N1, int N2,
                          void* workspace, size_t workspace_bytes, void* stream) {
    if (M < 0 || K1 < 1 || N1 < 1 || N2 < 1)
        return fail(JH_ERR_SHAPE, "mlp forward: needs M >= 0 and K1, N1, N2 >= 1 (got %d %d %d %d)",
                    M, K1, N1, N2);
    if ((int64_t)M * K1 > kMaxElems || (int64_t)M * N1 > kMaxElems || (int64_t)M * N2 > kMaxElems ||
        (int64_t)K1 * N1 > kMaxElems || (int64_t)N1 * N2 > kMaxElems)
        return fail(JH_ERR_SHAPE, "mlp forward: too large");
    if (M == 0) return JH_OK;
    if (!X || !W1 || !b1 || !W2 || !b2 || !output) return fail(JH_ERR_NULL, "mlp forward: null operand");
    const void* ptrs[] = {X, W1, b1, W2, b2, output};
    for (const void* q : ptrs)
        if (!aligned(q, 4)) return fail(JH_ERR_ALIGN, "mlp forward: operands must be 4-byte aligned");
    const size_t need = jh::mlp_forward_workspace_size(M, K1, N1, N2);
    if (!workspace || workspace_bytes < need)
        return fail(JH_ERR_WORKSPACE, "mlp forward: workspace %zu bytes, need %zu", workspace_bytes, need);
    if (!aligned(workspace, 16)) return fail(JH_ERR_ALIGN, "mlp forward: workspace alignment");
    return check_hip(jh::launch_mlp_forward(X, W1, b1, W2, b2, output, M, K1, N1, N2, workspace,
                                            static_cast<hipStream_t>(stream)),
                     "mlp forward launch");
}

size_t jules_hip_mlp_workspace_size(int M, int K1, int N1, int N2) {
    if (M < 0 || K1 < 1 || N1 < 1 || N2 < 1) return 0;
    return jh::mlp_workspace_size(M, K1, N1, N2);
}

int jules_hip_mlp_forward_backward(const float* X, const float* W1, const float* b1,
                                   const float* W2, const float* b2, const int32_t* targets,
                                   float* output, float* dW1, float* db1, float* dW2, float* db2,
                                   float* dX, int M, int K1, int N1, int N2, float* loss,
                                   void* workspace, size_t workspace_bytes, void* stream) {
    if (M < 0 || K1 < 1 || N1 < 1 || N2 < 1)
        return fail(JH_ERR_SHAPE, "mlp: needs M >= 0 and K1, N1, N2 >= 1 (got %d %d %d %d)", M, K1,
                    N1, N2);
    if ((int64_t)M * K1 > kMaxElems || (int64_t)M * N1 > kMaxElems || (int64_t)M * N2 > kMaxElems ||
        (int64_t)K1 * N1 > kMaxElems || (int64_t)N1 * N2 > kMaxElems)
        return fail(JH_ERR_SHAPE, "mlp: too large");
    if (!W1 || !b1 || !W2 || !b2 || !dW1 || !db1 || !dW2 || !db2 || !loss)
        return fail(JH_ERR_NULL, "mlp: null weight, bias, gradient or loss pointer");
    if (M > 0 && (!X || !targets || !output)) return fail(JH_ERR_NULL, "mlp: null X, targets or output");
    const void* ptrs[] = {X, W1, b1, W2, b2, targets, output, dW1, db1, dW2, db2, dX, loss};
    for (const void* q : ptrs)
        if (!aligned(q, 4)) return fail(JH_ERR_ALIGN, "mlp: operands must be 4-byte aligned");
    const size_t need = jh::mlp_workspace_size(M, K1, N1, N2);
    if (M > 0 && (!workspace || workspace_bytes < need))
        return fail(JH_ERR_WORKSPACE, "mlp: workspace %zu bytes, need %zu", workspace_bytes, need);
    if (!aligned(workspace, 16)) return fail(JH_ERR_ALIGN, "mlp: workspace alignment");
    return check_hip(jh::launch_mlp_forward_backward(X, W1, b1, W2, b2, targets, output, dW1, db1,
                                                     dW2, db2, dX, loss, M, K1, N1, N2, workspace,
                                                     static_cast<hipStream_t>(stream)),
                     "mlp launch");
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Registry: extern_kernel / custom_call names -> descriptor entry points.
// ---------------------------------------------------------------------------
namespace {

const void* addr(const jh_tensor& t) {
    int esz = t.dtype == JH_F32 || t.dtype == JH_I32 ? 4 : t.dtype == JH_BF16 ? 2 : 1;
    return static_cast<const char*>(t.data) + t.offset * esz;
}
void* addr_mut(jh_tensor& t) { return const_cast<void*>(addr(t)); }

bool contiguous(const jh_tensor& t) {
    if (t.rank < 0 || t.rank > 6) return false;
    int64_t s = 1;
    for (int i = t.rank - 1; i >= 0; --i) {
        if (t.sizes[i] < 0) return false;
        if (t.sizes[i] != 1 && t.strides[i] != s) return false;
        s *= t.sizes[i];
    }
    return true;
}

int64_t numel(const jh_tensor& t) {
    int64_t n = 1;
    for (int i = 0; i < t.rank; ++i) n *= t.sizes[i];
    return n;
}

// parse "key=value" out of a comma separated backend_config
bool config_float(const char* cfg, const char* key, float* out) {
    if (!cfg) return false;
    const size_t kl = strlen(key);
    const char* p = cfg;
    while (*p) {
        while (*p == ' ' || *p == ',') ++p;
        if (strncmp(p, key, kl) == 0 && p[kl] == '=') {
            char* end = nullptr;
            const float v = strtof(p + kl + 1, &end);
            if (end == p + kl + 1) return false;
            *out = v;
            return true;
        }
        while (*p && *p != ',') ++p;
    }
    return false;
}

int matmul_desc(int act, bool with_bias, int n_in, const jh_tensor* in, int n_out,
                jh_tensor* out, void* stream) {
    if (n_in != (with_bias ? 3 : 2) || n_out != 1 || !in || !out)
        return fail(JH_ERR_ARG, "matmul: expected %d inputs and 1 output", with_bias ? 3 : 2);
    const jh_tensor &a = in[0], &b = in[1];
    jh_tensor& c = out[0];
    if (a.rank != 2 || b.rank != 2 || c.rank != 2) return fail(JH_ERR_SHAPE, "matmul: rank != 2");
    if (!contiguous(a) || !contiguous(b) || !contiguous(c))
        return fail(JH_ERR_UNSUPPORTED, "matmul: non-contiguous operand");
    const int64_t M = a.sizes[0], K = a.sizes[1], N = b.sizes[1];
    if (b.sizes[0] != K || c.sizes[0] != M || c.sizes[1] != N)
        return fail(JH_ERR_SHAPE, "matmul: shape mismatch");
    if (a.dtype != b.dtype || a.dtype != c.dtype) return fail(JH_ERR_DTYPE, "matmul: dtype mismatch");
    const float* bias = nullptr;
    if (with_bias) {
        if (in[2].dtype != JH_F32 || numel(in[2]) != N || !contiguous(in[2]))
            return fail(JH_ERR_SHAPE, "matmul: bias must be fp32 [N]");
        bias = static_cast<const float*>(addr(in[2]));
    }
    if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return fail(JH_ERR_SHAPE, "matmul: dims");
    return jules_hip_gemm_bias_act(a.dtype, act, addr(a), addr(b), bias, addr_mut(c), (int)M,
                                   (int)N, (int)K, stream);
}

#define MATMUL_ENTRY(fname, ACT, BIAS)                                                      \
    int fname(int ni, const jh_tensor* in, int no, jh_tensor* out, const char*, void* s) { \
        return matmul_desc(ACT, BIAS, ni, in, no, out, s);                                  \
    }
MATMUL_ENTRY(k_matmul, JH_ACT_NONE, false)
MATMUL_ENTRY(k_matmul_relu, JH_ACT_RELU, false)
MATMUL_ENTRY(k_matmul_sigmoid, JH_ACT_SIGMOID, false)
MATMUL_ENTRY(k_matmul_tanh, JH_ACT_TANH, false)
MATMUL_ENTRY(k_matmul_gelu, JH_ACT_GELU, false)
MATMUL_ENTRY(k_matmul_bias, JH_ACT_NONE, true)
MATMUL_ENTRY(k_matmul_bias_relu, JH_ACT_RELU, true)
MATMUL_ENTRY(k_matmul_bias_sigmoid, JH_ACT_SIGMOID, true)
MATMUL_ENTRY(k_matmul_bias_tanh, JH_ACT_TANH, true)
MATMUL_ENTRY(k_matmul_bias_gelu, JH_ACT_GELU, true)
MATMUL_ENTRY(k_matmul_bias_silu, JH_ACT_SILU, true)

int k_gelu(int ni, const jh_tensor* in, int no, jh_tensor* out, const char*, void* s) {
    if (ni != 1 || no != 1 || !in || !out) return fail(JH_ERR_ARG, "fusedGelu: 1 in, 1 out");
    if (in[0].dtype != JH_F32 || out[0].dtype != JH_F32)
        return fail(JH_ERR_DTYPE, "fusedGelu: fp32 only");
    if (!contiguous(in[0]) || !contiguous(out[0]) || numel(in[0]) != numel(out[0]))
        return fail(JH_ERR_SHAPE, "fusedGelu: shape");
    return jules_hip_activation(JH_ACT_GELU, static_cast<float*>(addr_mut(out[0])),
                                static_cast<const float*>(addr(in[0])), numel(in[0]), s);
}

int attention_desc(int causal, int ni, const jh_tensor* in, int no, jh_tensor* out,
                   const char* cfg, void* s) {
    if (ni != 3 || no != 1 || !in || !out) return fail(JH_ERR_ARG, "attention: 3 in, 1 out");
    for (int i = 0; i < 3; ++i)
        if (in[i].rank != 4 || !contiguous(in[i])) return fail(JH_ERR_SHAPE, "attention: [B,H,S,D]");
    if (out[0].rank != 4 || !contiguous(out[0])) return fail(JH_ERR_SHAPE, "attention: out");
    for (int d = 0; d < 4; ++d)
        if (in[1].sizes[d] != in[0].sizes[d] || in[2].sizes[d] != in[0].sizes[d] ||
            out[0].sizes[d] != in[0].sizes[d])
            return fail(JH_ERR_SHAPE, "attention: Q, K, V, O shapes differ");
    const int dt = in[0].dtype;
    if (in[1].dtype != dt || in[2].dtype != dt || out[0].dtype != dt)
        return fail(JH_ERR_DTYPE, "attention: dtype mismatch");
    const int D = (int)in[0].sizes[3];
    float scale = 1.0f / sqrtf((float)D);  // reference FlashAttention.h:135
    config_float(cfg, "scale", &scale);
    return jules_hip_flash_attn_fwd(dt, causal, scale, addr(in[0]), addr(in[1]), addr(in[2]),
                                    addr_mut(out[0]), nullptr, (int)in[0].sizes[0],
                                    (int)in[0].sizes[1], (int)in[0].sizes[2], D, s);
}
int k_attn(int ni, const jh_tensor* in, int no, jh_tensor* out, const char* c, void* s) {
    return attention_desc(0, ni, in, no, out, c, s);
}
int k_attn_causal(int ni, const jh_tensor* in, int no, jh_tensor* out, const char* c, void* s) {
    return attention_desc(1, ni, in, no, out, c, s);
}

// Workspace for registry callers, who cannot pass one (W8A16 partials and
// flags, cross-entropy row losses, MLP activations): the library's buffer
// for the caller's (device, stream), grown on demand.  Calls on one stream
// run in stream order and may share it; calls on another stream get their
// own buffer, so registry calls on two streams of one device do not race.
int registry_workspace(size_t need, void* stream, void** ws) {
    return check_hip(jh::stream_workspace(need, static_cast<hipStream_t>(stream), ws),
                     "registry workspace");
}

int k_w8a16_silu(int ni, const jh_tensor* in, int no, jh_tensor* out, const char*, void* s) {
    if ((ni != 3 && ni != 4) || no != 1 || !in || !out)
        return fail(JH_ERR_ARG, "matmulW8A16BiasSilu: (x, W, scale[, bias]) -> y");
    const jh_tensor &x = in[0], &w = in[1], &sc = in[2];
    jh_tensor& y = out[0];
    if (x.rank != 2 || w.rank != 2 || y.rank != 2 || !contiguous(x) || !contiguous(w) ||
        !contiguous(y) || !contiguous(sc))
        return fail(JH_ERR_SHAPE, "matmulW8A16BiasSilu: 2-D contiguous operands");
    if (x.dtype != JH_BF16 || w.dtype != JH_I8 || sc.dtype != JH_F32 || y.dtype != JH_BF16)
        return fail(JH_ERR_DTYPE, "matmulW8A16BiasSilu: x bf16, W int8, scale fp32, y bf16");
    const int64_t M = x.sizes[0], K = x.sizes[1], N = w.sizes[1];
    if (w.sizes[0] != K || y.sizes[0] != M || y.sizes[1] != N || numel(sc) != N)
        return fail(JH_ERR_SHAPE, "matmulW8A16BiasSilu: shape mismatch");
    const float* bias = nullptr;
    if (ni == 4) {
        if (in[3].dtype != JH_F32 || numel(in[3]) != N || !contiguous(in[3]))
            return fail(JH_ERR_SHAPE, "matmulW8A16BiasSilu: bias fp32 [N]");
        bias = static_cast<const float*>(addr(in[3]));
    }
    const size_t need = jules_hip_w8a16_workspace_size((int)M, (int)N, (int)K);
    void* ws = nullptr;
    if (need) {
        const int st = registry_workspace(need, s, &ws);
        if (st != JH_OK) return st;
    }
    return jules_hip_w8a16_gemm_bias_act(JH_ACT_SILU, addr(x), static_cast<const int8_t*>(addr(w)),
                                         static_cast<const float*>(addr(sc)), bias, addr_mut(y),
                                         (int)M, (int)N, (int)K, ws, need, s);
}

int k_int8(int ni, const jh_tensor* in, int no, jh_tensor* out, const char* cfg, void* s) {
    if ((ni != 2 && ni != 3) || no != 1 || !in || !out)
        return fail(JH_ERR_ARG, "matmulInt8: (A, B[, bias]) -> C");
    const jh_tensor &a = in[0], &b = in[1];
    jh_tensor& c = out[0];
    if (a.rank != 2 || b.rank != 2 || c.rank != 2 || !contiguous(a) || !contiguous(b) ||
        !contiguous(c))
        return fail(JH_ERR_SHAPE, "matmulInt8: 2-D contiguous operands");
    if (a.dtype != JH_I8 || b.dtype != JH_I8 || c.dtype != JH_F32)
        return fail(JH_ERR_DTYPE, "matmulInt8: int8 x int8 -> fp32");
    const int64_t M = a.sizes[0], K = a.sizes[1], N = b.sizes[1];
    if (b.sizes[0] != K || c.sizes[0] != M || c.sizes[1] != N)
        return fail(JH_ERR_SHAPE, "matmulInt8: shape mismatch");
    float sa = 1.0f, sb = 1.0f;
    config_float(cfg, "scale_a", &sa);
    config_float(cfg, "scale_b", &sb);
    const float* bias = nullptr;
    if (ni == 3) {
        if (in[2].dtype != JH_F32 || numel(in[2]) != N || !contiguous(in[2]))
            return fail(JH_ERR_SHAPE, "matmulInt8: bias fp32 [N]");
        bias = static_cast<const float*>(addr(in[2]));
    }
    return jules_hip_matmul_int8(static_cast<const int8_t*>(addr(a)),
                                 static_cast<const int8_t*>(addr(b)),
                                 static_cast<float*>(addr_mut(c)), (int)M, (int)N, (int)K, sa, sb,
                                 bias, s);
}

int k_w8a8(int ni, const jh_tensor* in, int no, jh_tensor* out, const char*, void* s) {
    if ((ni != 4 && ni != 5) || no != 1 || !in || !out)
        return fail(JH_ERR_ARG, "matmulW8A8: (A, B, scale_A, scale_B[, bias]) -> C");
    const jh_tensor &a = in[0], &b = in[1], &sa = in[2], &sb = in[3];
    jh_tensor& c = out[0];
    if (a.rank != 2 || b.rank != 2 || c.rank != 2 || !contiguous(a) || !contiguous(b) ||
        !contiguous(c))
        return fail(JH_ERR_SHAPE, "matmulW8A8: 2-D contiguous A, B, C");
    if (a.dtype != JH_I8 || b.dtype != JH_I8 || c.dtype != JH_F32 || sa.dtype != JH_F32 ||
        sb.dtype != JH_F32)
        return fail(JH_ERR_DTYPE, "matmulW8A8: int8 x int8 -> fp32, fp32 scales");
    const int64_t M = a.sizes[0], K = a.sizes[1], N = b.sizes[1];
    if (b.sizes[0] != K || c.sizes[0] != M || c.sizes[1] != N)
        return fail(JH_ERR_SHAPE, "matmulW8A8: shape mismatch");
    if (numel(sa) != M || numel(sb) != N || !contiguous(sa) || !contiguous(sb))
        return fail(JH_ERR_SHAPE, "matmulW8A8: scale_A [M], scale_B [N]");
    const float* bias = nullptr;
    if (ni == 5) {
        if (in[4].dtype != JH_F32 || numel(in[4]) != N || !contiguous(in[4]))
            return fail(JH_ERR_SHAPE, "matmulW8A8: bias fp32 [N]");
        bias = static_cast<const float*>(addr(in[4]));
    }
    return jules_hip_matmul_w8a8(static_cast<const int8_t*>(addr(a)), static_cast<const int8_t*>(addr(b)),
                                 static_cast<float*>(addr_mut(c)), (int)M, (int)N, (int)K,
                                 static_cast<const float*>(addr(sa)), static_cast<const float*>(addr(sb)),
                                 bias, s);
}

// rows of a descriptor: product of all but the last dimension
int64_t rows_of(const jh_tensor& t) {
    int64_t r = 1;
    for (int d = 0; d + 1 < t.rank; ++d) r *= t.sizes[d];
    return r;
}

int k_softmax(int ni, const jh_tensor* in, int no, jh_tensor* out, const char*, void* s) {
    if (ni != 1 || no != 1 || !in || !out) return fail(JH_ERR_ARG, "fusedSoftmax: (x) -> y");
    const jh_tensor& x = in[0];
    jh_tensor& y = out[0];
    if (x.rank < 1 || y.rank < 1 || !contiguous(x) || !contiguous(y) || numel(x) != numel(y) ||
        y.sizes[y.rank - 1] != x.sizes[x.rank - 1])
        return fail(JH_ERR_SHAPE, "fusedSoftmax: contiguous x and y of one shape");
    if (x.dtype != JH_F32 || y.dtype != JH_F32) return fail(JH_ERR_DTYPE, "fusedSoftmax: fp32");
    const int64_t N = x.sizes[x.rank - 1], M = rows_of(x);
    if (M > INT32_MAX || N > INT32_MAX) return fail(JH_ERR_SHAPE, "fusedSoftmax: too large");
    return jules_hip_softmax(static_cast<float*>(addr_mut(y)), static_cast<const float*>(addr(x)),
                             (int)M, (int)N, s);
}

int k_layernorm(int ni, const jh_tensor* in, int no, jh_tensor* out, const char* cfg, void* s) {
    if (ni != 3 || no != 1 || !in || !out)
        return fail(JH_ERR_ARG, "fusedLayerNorm: (x, gamma, beta) -> y");
    const jh_tensor &x = in[0], &g = in[1], &b = in[2];
    jh_tensor& y = out[0];
    if (x.rank < 1 || !contiguous(x) || !contiguous(y) || !contiguous(g) || !contiguous(b) ||
        numel(x) != numel(y))
        return fail(JH_ERR_SHAPE, "fusedLayerNorm: contiguous operands");
    const int64_t N = x.sizes[x.rank - 1], M = rows_of(x);
    if (numel(g) != N || numel(b) != N) return fail(JH_ERR_SHAPE, "fusedLayerNorm: gamma/beta [N]");
    if (x.dtype != JH_F32 || y.dtype != JH_F32 || g.dtype != JH_F32 || b.dtype != JH_F32)
        return fail(JH_ERR_DTYPE, "fusedLayerNorm: fp32");
    if (M > INT32_MAX || N > INT32_MAX) return fail(JH_ERR_SHAPE, "fusedLayerNorm: too large");
    float eps = 1e-5f;  // reference default, FusedKernels.h:534
    config_float(cfg, "epsilon", &eps);
    return jules_hip_layernorm(static_cast<float*>(addr_mut(y)), static_cast<const float*>(addr(x)),
                               static_cast<const float*>(addr(g)),
                               static_cast<const float*>(addr(b)), (int)M, (int)N, eps, s);
}

int k_cross_entropy(int ni, const jh_tensor* in, int no, jh_tensor* out, const char*, void* s) {
    if (ni != 2 || no != 2 || !in || !out)
        return fail(JH_ERR_ARG, "fusedCrossEntropyLoss: (logits, targets) -> (grad, loss)");
    const jh_tensor &x = in[0], &t = in[1];
    jh_tensor &g = out[0], &l = out[1];
    if (x.rank < 1 || !contiguous(x) || !contiguous(t) || !contiguous(g) || !contiguous(l) ||
        numel(g) != numel(x) || numel(l) != 1)
        return fail(JH_ERR_SHAPE, "fusedCrossEntropyLoss: contiguous operands, one loss element");
    const int64_t N = x.sizes[x.rank - 1], M = rows_of(x);
    if (numel(t) != M) return fail(JH_ERR_SHAPE, "fusedCrossEntropyLoss: one target per row");
    if (x.dtype != JH_F32 || g.dtype != JH_F32 || l.dtype != JH_F32 || t.dtype != JH_I32)
        return fail(JH_ERR_DTYPE, "fusedCrossEntropyLoss: fp32 logits/grad/loss, int32 targets");
    if (M > INT32_MAX || N > INT32_MAX) return fail(JH_ERR_SHAPE, "fusedCrossEntropyLoss: too large");
    const size_t need = jules_hip_cross_entropy_workspace_size((int)M);
    void* ws = nullptr;
    const int st = registry_workspace(need, s, &ws);
    if (st != JH_OK) return st;
    return jules_hip_cross_entropy(static_cast<const float*>(addr(x)),
                                   static_cast<const int32_t*>(addr(t)),
                                   static_cast<float*>(addr_mut(g)),
                                   static_cast<float*>(addr_mut(l)), (int)M, (int)N, ws, need, s);
}

int k_mlp_forward(int ni, const jh_tensor* in, int no, jh_tensor* out, const char*, void* s) {
    if (ni != 5 || no != 1 || !in || !out)
        return fail(JH_ERR_ARG, "fusedMLPForward: (X, W1, b1, W2, b2) -> output");
    const jh_tensor &x = in[0], &w1 = in[1], &b1 = in[2], &w2 = in[3], &b2 = in[4];
    jh_tensor& y = out[0];
    for (int i = 0; i < ni; ++i)
        if (!contiguous(in[i]) || in[i].dtype != JH_F32)
            return fail(JH_ERR_DTYPE, "fusedMLPForward: contiguous fp32 operands");
    if (!contiguous(y) || y.dtype != JH_F32) return fail(JH_ERR_DTYPE, "fusedMLPForward: fp32 output");
    if (x.rank != 2 || w1.rank != 2 || w2.rank != 2)
        return fail(JH_ERR_SHAPE, "fusedMLPForward: X, W1, W2 rank 2");
    const int64_t M = x.sizes[0], K1 = x.sizes[1], N1 = w1.sizes[1], N2 = w2.sizes[1];
    if (w1.sizes[0] != K1 || w2.sizes[0] != N1 || numel(b1) != N1 || numel(b2) != N2 ||
        numel(y) != M * N2)
        return fail(JH_ERR_SHAPE, "fusedMLPForward: operand shapes disagree");
    if (M > INT32_MAX || K1 > INT32_MAX || N1 > INT32_MAX || N2 > INT32_MAX)
        return fail(JH_ERR_SHAPE, "fusedMLPForward: too large");
    const size_t need = jules_hip_mlp_forward_workspace_size((int)M, (int)K1, (int)N1, (int)N2);
    void* ws = nullptr;
    if (need > 0) {
        const int st = registry_workspace(need, s, &ws);
        if (st != JH_OK) return st;
    }
    return jules_hip_mlp_forward(static_cast<const float*>(addr(x)), static_cast<const float*>(addr(w1)),
                                 static_cast<const float*>(addr(b1)), static_cast<const float*>(addr(w2)),
                                 static_cast<const float*>(addr(b2)), static_cast<float*>(addr_mut(y)),
                                 (int)M, (int)K1, (int)N1, (int)N2, ws, need, s);
}

int k_mlp(int ni, const jh_tensor* in, int no, jh_tensor* out, const char*, void* s) {
    if (ni != 6 || (no != 6 && no != 7) || !in || !out)
        return fail(JH_ERR_ARG, "interleavedMLPForwardBackward: (X, W1, b1, W2, b2, targets) -> "
                                "(output, dW1, db1, dW2, db2, loss[, dX])");
    const jh_tensor &x = in[0], &w1 = in[1], &b1 = in[2], &w2 = in[3], &b2 = in[4], &t = in[5];
    for (int i = 0; i < ni; ++i)
        if (!contiguous(in[i])) return fail(JH_ERR_SHAPE, "interleavedMLPForwardBackward: contiguous inputs");
    for (int i = 0; i < no; ++i)
        if (!contiguous(out[i]) || out[i].dtype != JH_F32)
            return fail(JH_ERR_SHAPE, "interleavedMLPForwardBackward: contiguous fp32 outputs");
    if (x.rank != 2 || w1.rank != 2 || w2.rank != 2)
        return fail(JH_ERR_SHAPE, "interleavedMLPForwardBackward: X, W1, W2 rank 2");
    for (int i = 0; i < 5; ++i)
        if (in[i].dtype != JH_F32) return fail(JH_ERR_DTYPE, "interleavedMLPForwardBackward: fp32 X, W, b");
    if (t.dtype != JH_I32) return fail(JH_ERR_DTYPE, "interleavedMLPForwardBackward: int32 targets");
    const int64_t M = x.sizes[0], K1 = x.sizes[1], N1 = w1.sizes[1], N2 = w2.sizes[1];
    if (w1.sizes[0] != K1 || w2.sizes[0] != N1 || numel(b1) != N1 || numel(b2) != N2 ||
        numel(t) != M || numel(out[0]) != M * N2 || numel(out[1]) != K1 * N1 ||
        numel(out[2]) != N1 || numel(out[3]) != N1 * N2 || numel(out[4]) != N2 ||
        numel(out[5]) != 1 || (no == 7 && numel(out[6]) != M * K1))
        return fail(JH_ERR_SHAPE, "interleavedMLPForwardBackward: operand shapes disagree");
    if (M > INT32_MAX || K1 > INT32_MAX || N1 > INT32_MAX || N2 > INT32_MAX)
        return fail(JH_ERR_SHAPE, "interleavedMLPForwardBackward: too large");
    const size_t need = jules_hip_mlp_workspace_size((int)M, (int)K1, (int)N1, (int)N2);
    void* ws = nullptr;
    if (need > 0) {
        const int st = registry_workspace(need, s, &ws);
        if (st != JH_OK) return st;
    }
    float* f[7];
    for (int i = 0; i < no; ++i) f[i] = static_cast<float*>(addr_mut(out[i]));
    return jules_hip_mlp_forward_backward(
        static_cast<const float*>(addr(x)), static_cast<const float*>(addr(w1)),
        static_cast<const float*>(addr(b1)), static_cast<const float*>(addr(w2)),
        static_cast<const float*>(addr(b2)), static_cast<const int32_t*>(addr(t)), f[0], f[1], f[2],
        f[3], f[4], no == 7 ? f[6] : nullptr, (int)M, (int)K1, (int)N1, (int)N2, f[5], ws, need, s);
}

struct Entry {
    const char* name;
    jh_kernel_fn fn;
};

// Names emitted by KernelRoutingPass (lib/Passes/KernelRoutingPass.cpp:144-166,
// :189-211, :261, :287, :330, :378, :409) and listed in KernelRoutingPass.h:13-23,
// then the names this library adds.
const Entry kRegistry[] = {
    {"fusedMatmulRelu", k_matmul_relu},
    {"fusedMatmulSigmoid", k_matmul_sigmoid},
    {"fusedMatmulTanh", k_matmul_tanh},
    {"fusedMatmulGelu", k_matmul_gelu},
    {"fusedMatmulBiasRelu", k_matmul_bias_relu},
    {"fusedMatmulBiasSigmoid", k_matmul_bias_sigmoid},
    {"fusedMatmulBiasTanh", k_matmul_bias_tanh},
    {"fusedGelu", k_gelu},
    {"matmulInt8", k_int8},
    {"flashAttention", k_attn},
    {"fusedSoftmax", k_softmax},
    {"fusedLayerNorm", k_layernorm},
    {"fusedCrossEntropyLoss", k_cross_entropy},
    {"fusedMLPForward", k_mlp_forward},
    {"interleavedMLPForwardBackward", k_mlp},
    {"fusedMatmul", k_matmul},
    {"fusedMatmulBias", k_matmul_bias},
    {"fusedMatmulBiasGelu", k_matmul_bias_gelu},
    {"fusedMatmulBiasSilu", k_matmul_bias_silu},
    {"flashAttentionCausal", k_attn_causal},
    {"matmulW8A16BiasSilu", k_w8a16_silu},
    {"matmulW8A8", k_w8a8},
};
constexpr int kRegistrySize = sizeof(kRegistry) / sizeof(kRegistry[0]);

}  // namespace

extern "C" {

jh_kernel_fn jules_hip_lookup(const char* name) {
    if (!name) {
        fail(JH_ERR_NULL, "lookup: null name");
        return nullptr;
    }
    for (int i = 0; i < kRegistrySize; ++i)
        if (strcmp(kRegistry[i].name, name) == 0) return kRegistry[i].fn;
    fail(JH_ERR_NOT_FOUND, "lookup: no kernel named '%s'", name);
    return nullptr;
}

int jules_hip_kernel_count(void) { return kRegistrySize; }

const char* jules_hip_kernel_name(int index) {
    if (index < 0 || index >= kRegistrySize) return nullptr;
    return kRegistry[index].name;
}

}  // extern "C"
