// launch.hpp - internal launchers of libjules_hip (not part of the C ABI).
// Arguments have been validated by capi.cpp before any of these is called.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace jh {

hipError_t launch_gemm_f32(int act, const float* A, const float* B, const float* bias,
                           float* C, int M, int N, int K, hipStream_t s);
// one fp32 GEMM kernel of the tile table (tiles.hpp: GV_F32_*); the caller
// has checked f32_variant_valid()
hipError_t launch_gemm_f32_variant(int variant, int act, const float* A, const float* B,
                                   const float* bias, float* C, int M, int N, int K,
                                   hipStream_t s);
// the fp32 GEMM entry point's validation and launch with a chosen table
// variant (-1: the table's default), for jules::kernel::tiledMatmulWithActivation
int gemm_f32_with_variant(int variant, int act, const float* A, const float* B, const float* bias,
                          float* C, int M, int N, int K, hipStream_t s);
// C = alpha op(A) op(B) + beta C, fp32 on MFMA (mlp.hip); op(X) = X^T when
// the trans flag is set; row-major with leading dimensions lda, ldb, ldc
hipError_t launch_sgemm(bool transA, bool transB, int M, int N, int K, float alpha, const float* A,
                        int lda, const float* B, int ldb, float beta, float* C, int ldc,
                        hipStream_t s);
hipError_t launch_gemm_bf16(int act, const uint16_t* A, const uint16_t* B, const float* bias,
                            uint16_t* C, int M, int N, int K, hipStream_t s);
hipError_t launch_activation(int act, float* out, const float* in, int64_t n, hipStream_t s);
hipError_t launch_flash_fwd(int dtype, int causal, float scale, const void* Q, const void* K,
                            const void* V, void* O, float* lse, int B, int H, int S, int D,
                            hipStream_t s);
// flash-attention backward (flash_bwd.hip): bf16; workspace = fp32 [B,H,S]
size_t flash_bwd_workspace_size(int B, int H, int S);
hipError_t launch_flash_bwd(int dtype, int causal, float scale, const void* Q, const void* K,
                            const void* V, const void* O, const void* dO, const float* lse,
                            void* dQ, void* dK, void* dV, int B, int H, int S, int D, void* ws,
                            hipStream_t s);
size_t w8a16_workspace_size(int M, int N, int K);
// int8 x int8 at M <= 16 with the W8A16 split-K design (w8a16.hip); K and N
// multiples of 16, A and B 16-byte aligned
size_t int8_decode_workspace_size(int M, int N, int K);
hipError_t launch_int8_decode(const int8_t* A, const int8_t* B, float* C, int M, int N, int K,
                              float scale_a, float scale_b, const float* row_scale,
                              const float* col_scale, const float* bias, void* ws, hipStream_t s);
hipError_t launch_w8a16(int act, const uint16_t* x, const int8_t* W, const float* scale,
                        const float* bias, uint16_t* y, int M, int N, int K, void* ws,
                        hipStream_t s);
// the same computation with the last workgroup of each column tile found by
// an arrival counter (counters: one uint32 per 256-column tile, zero before
// the call, left at zero); partials: w8a16_partials_size(M, N, K) bytes
size_t w8a16_partials_size(int M, int N, int K);
hipError_t launch_w8a16_counters(int act, const uint16_t* x, const int8_t* W, const float* scale,
                                 const float* bias, uint16_t* y, int M, int N, int K,
                                 float* partials, uint32_t* counters, hipStream_t s);
// dQ pass of the flash backward (flash_bwd_dq.hip); dvec = rowsum(dO * O)
hipError_t launch_flash_bwd_dq(int D, bool causal, const uint16_t* Q, const uint16_t* K,
                               const uint16_t* V, const uint16_t* dO, const float* lse,
                               const float* dvec, uint16_t* dQ, int BH, int S, float scale,
                               hipStream_t s);
// W8A16 on the packed weight layout (w8a16_packed.hip): Wp holds
// w8a16_packed_bytes(K, N) bytes, written by launch_w8a16_pack from
// row-major W [K,N]
size_t w8a16_packed_bytes(int K, int N);
hipError_t launch_w8a16_pack(const int8_t* W, int K, int N, int8_t* Wp, hipStream_t s);
hipError_t launch_w8a16_packed(int act, const uint16_t* x, const int8_t* Wp, const float* scale,
                               const float* bias, uint16_t* y, int M, int N, int K, hipStream_t s);
hipError_t launch_matmul_int8(const int8_t* A, const int8_t* B, float* C, int M, int N, int K,
                              float scale_a, float scale_b, const float* bias, hipStream_t s);
hipError_t launch_matmul_w8a8(const int8_t* A, const int8_t* B, float* C, int M, int N, int K,
                              const float* scale_a, const float* scale_b, const float* bias,
                              hipStream_t s);
hipError_t launch_softmax(float* out, const float* in, int M, int N, hipStream_t s);
hipError_t launch_layernorm(float* out, const float* in, const float* gamma, const float* beta,
                            int M, int N, float eps, hipStream_t s);
// row_loss: M floats of scratch (per-row losses before the fixed-order sum)
hipError_t launch_cross_entropy(const float* logits, const int32_t* targets, float* grad,
                                float* loss, float* row_loss, int M, int N, hipStream_t s);

// 2-layer MLP forward + softmax cross entropy + backward (mlp.hip)
size_t mlp_forward_workspace_size(int M, int K1, int N1, int N2);
hipError_t launch_mlp_forward(const float* X, const float* W1, const float* b1, const float* W2,
                              const float* b2, float* output, int M, int K1, int N1, int N2,
                              void* ws, hipStream_t s);
size_t mlp_workspace_size(int M, int K1, int N1, int N2);
hipError_t launch_mlp_forward_backward(const float* X, const float* W1, const float* b1,
                                       const float* W2, const float* b2, const int32_t* targets,
                                       float* output, float* dW1, float* db1, float* dW2, float* db2,
                                       float* dX, float* loss, int M, int K1, int N1, int N2,
                                       void* ws, hipStream_t s);

// PJRT executor ops (pjrt_ops.hip): fp32, rank <= 8
enum PjOp {
    PJ_ADD = 0, PJ_SUB, PJ_MUL, PJ_DIV, PJ_MAX, PJ_MIN,
    PJ_NEG, PJ_RELU, PJ_SIGMOID, PJ_TANH, PJ_EXP, PJ_LOG
};
struct PjIndexMap {
    int rank;
    int64_t out_stride[8];  // strides of the index space walked
    int64_t in_step[8];     // input offset per unit step of each index
};
hipError_t launch_pj_binary(int op, const float* a, int64_t na, const float* b, int64_t nb,
                            float* out, int64_t n, hipStream_t s);
hipError_t launch_pj_unary(int op, const float* a, float* out, int64_t n, hipStream_t s);
hipError_t launch_pj_transpose(const float* in, float* out, int64_t n, const PjIndexMap& map,
                               hipStream_t s);
hipError_t launch_pj_reduce(const float* in, float* out, int64_t n_out, int64_t n_red,
                            const PjIndexMap& keep, const PjIndexMap& red, hipStream_t s);

// calibration: workgroups x 4 waves x 16*iters MFMAs on random operands
hipError_t launch_mfma_ceiling(float* out, int workgroups, int iters, hipStream_t s);
// calibration: a plain streaming read of `bytes` (a multiple of 16) by
// `workgroups` x 256 lanes; out receives workgroups * 256 uint32
hipError_t launch_hbm_read(const void* buf, int64_t bytes, uint32_t* out, int workgroups,
                           hipStream_t s);


// flash attention at head dims other than 64 and 128 (1 <= D <= 128): inputs
// zero-padded to 64 or 128 in the per-stream workspace (flash_pad.hip)
int flash_padded_dim(int D);
hipError_t launch_flash_fwd_padded(int dtype, int causal, float scale, const void* Q, const void* K,
                                   const void* V, void* O, float* lse, int B, int H, int S, int D,
                                   hipStream_t s);
hipError_t launch_flash_bwd_padded(int dtype, int causal, float scale, const void* Q, const void* K,
                                   const void* V, const void* O, const void* dO, const float* lse,
                                   void* dQ, void* dK, void* dV, int B, int H, int S, int D,
                                   void* bwd_ws, hipStream_t s);
// device memory of `need` bytes for entry points without a workspace
// argument: one buffer per (device, stream), kept for the process
hipError_t stream_workspace(size_t need, hipStream_t s, void** ws);
// the library's static device scratch (scratch.hip): its size, and the
// device address of the current device's copy (looked up once per device;
// allocates nothing)
size_t static_scratch_bytes();
size_t static_scratch_partial_bytes();  // the partial-tile part; the counters follow it
hipError_t static_scratch(void** ptr);

}  // namespace jh
