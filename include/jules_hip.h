/*
 * jules_hip.h - C ABI of the MI355X (gfx950) kernel library libjules_hip.so.
 *
 * This is the drop-in boundary for the Jules kernel path.  In the reference
 * the path is a set of header-defined C++ functions in namespace
 * jules::kernel (include/jules/Kernel/FusedKernels.h, FlashAttention.h) plus
 * the kernel-name strings that KernelRoutingPass writes into
 * jules.extern_kernel / stablehlo.custom_call ops.  This header replaces both:
 *
 *   - typed entry points (device pointers, an explicit hipStream_t passed as
 *     void*, an int status) for each kernel, and
 *   - a name registry, jules_hip_lookup(), that resolves the extern_kernel /
 *     custom_call target names to a uniform descriptor-based calling
 *     convention (what a ROCm PJRT device or an ORC symbol resolver binds).
 *
 * The C++ signatures of jules::kernel themselves (host buffers, synchronous)
 * are provided by jules_hip_kernel.hpp on top of this ABI.
 *
 * Conventions
 *   - All tensors are dense row-major in device memory (hipMalloc'd or any
 *     pointer the device can access).  Shapes use int like the reference.
 *   - Every entry point validates its arguments and returns a jh_status; no
 *     entry point aborts.  A non-zero status leaves outputs unspecified
 *     (argument errors are detected before any launch and write nothing).
 *     jules_hip_last_error() returns a thread-local message for the last
 *     failure on the calling thread.
 *   - Launches are asynchronous on `stream` (NULL = the legacy default
 *     stream).  Entry points are re-entrant; calls on different streams may
 *     overlap.  Buffers passed to one call must not be written concurrently.
 *   - Activation codes keep jules::kernel::ActivationType's values
 *     (reference FusedKernels.h:61-67) and add SiLU = 5.
 *   - bf16 is IEEE bfloat16 (uint16 bit pattern), rounded to nearest even.
 */
#ifndef JULES_HIP_H
#define JULES_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define JULES_HIP_ABI_VERSION 1

typedef enum jh_status {
    JH_OK = 0,
    JH_ERR_NULL = 1,        /* a required pointer is NULL */
    JH_ERR_SHAPE = 2,       /* negative, zero-where-forbidden or too large dimension */
    JH_ERR_DTYPE = 3,       /* dtype not supported by this entry point */
    JH_ERR_ALIGN = 4,       /* pointer misaligned for the required vector width */
    JH_ERR_ACT = 5,         /* unknown activation code */
    JH_ERR_WORKSPACE = 6,   /* workspace NULL or smaller than required */
    JH_ERR_HIP = 7,         /* the HIP runtime reported an error */
    JH_ERR_UNSUPPORTED = 8, /* valid request this build does not implement */
    JH_ERR_NOT_FOUND = 9,   /* registry: unknown kernel name */
    JH_ERR_ARG = 10         /* any other invalid argument (scale, rank, ...) */
} jh_status;

typedef enum jh_dtype {
    JH_F32 = 0,
    JH_BF16 = 1,
    JH_I8 = 2,
    JH_I32 = 3
} jh_dtype;

typedef enum jh_act {
    JH_ACT_NONE = 0,
    JH_ACT_RELU = 1,
    JH_ACT_SIGMOID = 2,
    JH_ACT_TANH = 3,
    JH_ACT_GELU = 4, /* tanh approximation, reference FusedKernels.h:155-164 */
    JH_ACT_SILU = 5  /* x * sigmoid(x); no reference counterpart */
} jh_act;

/* ---- library information ------------------------------------------------ */
int jules_hip_abi_version(void);
const char* jules_hip_status_string(int status);
const char* jules_hip_last_error(void);

/* ---- fused GEMM + bias + activation --------------------------------------
 * C[M,N] = act(A[M,K] . B[K,N] + bias[N])
 *
 * Replaces (reference include/jules/Kernel/FusedKernels.h):
 *   tiledMatmulWithActivation(A,B,C,M,N,K,cfg,act)  :378   (bias = NULL)
 *   fusedMatmulBiasRelu(X,W,bias,out,M,K,N)         :265   (act = RELU)
 *   fusedMatmulRelu(X,W,out,M,K,N)                  :203   (bias = NULL, act = RELU)
 * and the routed names fusedMatmul<Act> / fusedMatmulBias<Act>
 * (lib/Passes/KernelRoutingPass.cpp:144-166, :189-211).
 *
 * dtype JH_F32: A, B, C float.  Each C[i,j] is the sequential fma chain
 *   over k = 0..K-1 starting from 0, then + bias[j], then the activation of
 *   the reference's vector path (fast_exp based, FusedKernels.h:90-164), so
 *   results equal the reference AVX-512 kernel bit for bit whenever its
 *   vector path covers the column (N and tile_n multiples of 16).
 * dtype JH_BF16: A, B, C bf16; fp32 accumulation on MFMA; bias fp32;
 *   epilogue in fp32, C rounded to bf16.  M, N, K must be multiples of 8
 *   (16-byte rows); other shapes return JH_ERR_UNSUPPORTED.
 * bias may be NULL.  K = 0 gives act(bias) (act(0) without bias).
 */
int jules_hip_gemm_bias_act(int dtype, int act, const void* A, const void* B,
                            const float* bias, void* C, int M, int N, int K,
                            void* stream);

/* ---- GEMM tile table -------------------------------------------------------
 * out[4] = {kernel variant, tile_m, tile_n, tile_k} that
 * jules_hip_gemm_bias_act launches for this dtype and shape (needs no GPU).
 * Variants: 0/1 fp32 row kernel with 1/2 rows per wave (tile 4 or 8 rows x
 * 64 columns, all of K in LDS, K <= 2048), 2/3 fp32 32x32 / 64x64 tiles with
 * 32-deep K slices, 4 bf16 256x256 tiles with 32-deep LDS-DMA stages, 5 bf16
 * 256x256 register-staged tiles with 64-deep slices.  Replaces the role of
 * TilePlanner::getTileConfig (reference TilePlanner.h:74-136), which sizes
 * tiles for the CPU caches; jules::kernel::TilePlanner returns these.
 */
int jules_hip_gemm_tile(int dtype, int M, int N, int K, int* out);

/* ---- general fp32 GEMM (BLAS sgemm) -----------------------------------------
 * C = alpha * op(A) op(B) + beta * C, row-major, op(X) = X^T when transX = 1;
 * A is [M,K] (transA = 0) or [K,M] (transA = 1) with row stride lda, B is
 * [K,N] or [N,K] with row stride ldb, C [M,N] with row stride ldc; lda, ldb,
 * ldc at least the stored row length (and 1).  beta = 0 writes C without
 * reading it; K = 0 or alpha = 0 gives beta * C without reading A or B.
 * Replaces blasMatmul(A,B,C,M,N,K,alpha,beta,transA,transB) (reference
 * FusedKernels.h:633-644) and the cblas_sgemm calls of the reference
 * (LLVMBackend.cpp:1242-1255, PJRT.cpp:692-697), which libjules_cblas.so
 * (include/jules_cblas.h) maps here.
 * The dense, untransposed alpha = 1, beta = 0 product (what LLVMBackend
 * emits) runs the fp32 fma-chain GEMM of jules_hip_gemm_bias_act, so its bits
 * equal the reference's tiledMatmulWithActivation; every other case runs an
 * fp32 MFMA GEMM (fp32 accumulation in another order; within fp32 rounding
 * of the exact product, as the reference's BLAS is).  Skinny products split
 * K through a library-held per-(device, stream) buffer.
 */
int jules_hip_sgemm(int transA, int transB, int M, int N, int K, float alpha,
                    const float* A, int lda, const float* B, int ldb,
                    float beta, float* C, int ldc, void* stream);

/* ---- elementwise activation ----------------------------------------------
 * out[i] = act(in[i]), fp32, n elements.  act = GELU replaces
 * fusedGelu(out,in,N) (reference FusedKernels.h:606) and the routed name
 * "fusedGelu" (KernelRoutingPass.cpp:287): elements below n & ~15 get the
 * vector-path gelu (bit-exact with the reference), the last n % 16 the
 * reference's scalar tail formula with tanhf (the device libm's tanhf, so
 * within a few ulp of the reference's).  In-place (out == in) is allowed.
 */
int jules_hip_activation(int act, float* out, const float* in, int64_t n,
                         void* stream);

/* ---- flash-attention forward ---------------------------------------------
 * O = softmax(scale * Q K^T [+ causal mask]) V, per (b,h); Q,K,V,O [B,H,S,D].
 *
 * Replaces flashAttention(out,Q,K,V,B,H,S,D,arena,planner) and
 * attention(...) (reference include/jules/Kernel/FlashAttention.h:130, :114),
 * which are non-causal with scale fixed at 1/sqrtf(D) (:135); causal = 1
 * excludes keys j > query i.
 * dtype JH_F32 or JH_BF16 (Q, K, V, O share it); softmax statistics are fp32.
 * 1 <= D <= 128 (the kernels are built for 64 and 128; other head dims are
 * zero-padded to the next of the two in a library-held per-stream buffer).
 * S >= 1.  scale must be finite and > 0.
 * lse (optional, fp32 [B,H,S]) receives the natural-log log-sum-exp of the
 * scaled, masked scores of each row.
 */
int jules_hip_flash_attn_fwd(int dtype, int causal, float scale,
                             const void* Q, const void* K, const void* V,
                             void* O, float* lse, int B, int H, int S, int D,
                             void* stream);

/* ---- flash-attention backward --------------------------------------------
 * Gradients of jules_hip_flash_attn_fwd: with P = exp(scale * Q K^T - lse)
 * (masked entries 0) and dvec = rowsum(dO * O),
 *   dV = P^T dO,  dS = P * (dO V^T - dvec),  dQ = scale dS K,  dK = scale dS^T Q.
 * No reference counterpart: the reference's attention is forward only
 * (FlashAttention.h:130-309); this is the training path for the forward above.
 * dtype JH_BF16 (JH_F32 returns JH_ERR_UNSUPPORTED); Q, K, V, O, dO, dQ, dK,
 * dV [B,H,S,D] of that dtype, 16-byte aligned; lse fp32 [B,H,S] as written by
 * the forward with the same causal and scale; 1 <= D <= 128 (padded as in
 * the forward).  fp32
 * accumulation; deterministic (no atomics).
 * workspace: jules_hip_flash_attn_bwd_workspace_size(B,H,S) bytes (fp32
 * dvec), 4-byte aligned, no initialisation.
 */
size_t jules_hip_flash_attn_bwd_workspace_size(int B, int H, int S);
int jules_hip_flash_attn_bwd(int dtype, int causal, float scale,
                             const void* Q, const void* K, const void* V,
                             const void* O, const void* dO, const float* lse,
                             void* dQ, void* dK, void* dV,
                             int B, int H, int S, int D,
                             void* workspace, size_t workspace_bytes,
                             void* stream);

/* ---- W8A16 decode GEMM + bias + activation --------------------------------
 * y[m,j] = act(scale[j] * sum_k x[m,k] * W[k,j] + bias[j])
 * x bf16 [M,K], W int8 [K,N] (row-major, indexed W[k*N+j] like matmulInt8,
 * reference FusedKernels.h:1053), scale fp32 [N] per output channel, bias
 * fp32 [N] or NULL, y bf16 [M,N].  fp32 accumulation; the int8 -> fp32
 * dequantisation is exact.  Deterministic: the split-K reduction sums the
 * partials in a fixed order.
 * Constraints: 1 <= M <= 16, N % 16 == 0, K % 8 == 0; W and x 16-byte
 * aligned, y 8-byte aligned.
 * workspace: device memory of at least jules_hip_w8a16_workspace_size(M,N,K)
 * bytes, 16-byte aligned (fp32 split-K partial tiles, KS x ceil(N/256) x
 * 16 KiB with KS <= 8, then one 8-byte flag per tile and split; one launch
 * does the split-K reduction); it needs no initialisation and is
 * overwritten by every call.  Calls that overlap in time need separate
 * workspaces.  The flags are tagged with a value chosen when the call is
 * made, so a launch captured in a HIP graph must not be replayed; graph
 * callers use jules_hip_w8a16_gemm_bias_act_noalloc.
 * No reference counterpart: the reference's int8 kernel (matmulInt8,
 * FusedKernels.h:867) is W8A8 with one scalar scale; routed name
 * "matmulW8A16BiasSilu" is new.
 */
size_t jules_hip_w8a16_workspace_size(int M, int N, int K);
int jules_hip_w8a16_gemm_bias_act(int act, const void* x, const int8_t* W,
                                  const float* scale, const float* bias,
                                  void* y, int M, int N, int K,
                                  void* workspace, size_t workspace_bytes,
                                  void* stream);

/* ---- W8A16 on packed weights ------------------------------------------------
 * The same y = act(scale * x W + bias) as jules_hip_w8a16_gemm_bias_act, same
 * constraints on M, N, K, x, scale, bias and y, with W first repacked once
 * (at weight-load time) into a layout in which each workgroup streams one
 * contiguous block: 32 output columns over all of K, in 1 KiB blocks per 32
 * rows ordered as the kernel's MFMA operands (layout in w8a16_packed.hip).
 * No split-K across workgroups, so no workspace and no cross-workgroup
 * reduction; each tile's 8 wave partials are summed in a fixed order
 * (deterministic; the order differs from the row-major entry point's, so
 * the two agree to fp32 rounding, not bit for bit).
 * jules_hip_w8a16_packed_size(K, N): bytes of the packed array
 *   (ceil(N/32) * ceil(K/32) * 1024; 0 for K or N <= 0).
 * jules_hip_w8a16_pack: W int8 [K,N] row-major (device) -> Wp (device,
 *   16-byte aligned, packed_size bytes; rows past K and columns past N are
 *   written as zero).  Same K, N limits as the GEMM.
 * jules_hip_w8a16_packed_gemm_bias_act: Wp as written by jules_hip_w8a16_pack
 *   with the same K and N.
 * No reference counterpart (the reference has no W8A16 kernel); it is the
 * decode configuration's fast path for callers that own their weights.
 */
size_t jules_hip_w8a16_packed_size(int K, int N);
int jules_hip_w8a16_pack(const int8_t* W, int K, int N, void* Wp, size_t Wp_bytes, void* stream);
int jules_hip_w8a16_packed_gemm_bias_act(int act, const void* x, const void* Wp,
                                         const float* scale, const float* bias,
                                         void* y, int M, int N, int K, void* stream);

/* ---- W8A16 without allocation ------------------------------------------------
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The same computation, kernels and bits as
 * jules_hip_w8a16_gemm_bias_act, with the split-K workspace taken from a
 * library-held static device array instead of an argument; the call
 * allocates nothing (no hipMalloc, hipFree or allocating library routine).
 * Limit: the workspace of the shape must fit the array,
 * jules_hip_w8a16_noalloc_max_bytes() bytes (8 MiB + 4 KiB: N <= 16384 at
 * any K); larger shapes return JH_ERR_WORKSPACE.  Each GPU holds one such
 * array for the life of the process and every call on that GPU shares it, so
 * calls that overlap in time on one GPU (different streams, or threads
 * without ordering) race and give wrong results; calls ordered on one stream
 * are safe.  The split-K reduction finds each column tile's last workgroup
 * with an arrival counter in the array that the last workgroup resets, so
 * the launch carries no per-call value: the call may be captured in a HIP
 * graph and replayed (the workspace entry point cannot: its completion flags
 * are tagged with a value chosen at launch, which capture would freeze).
 */
size_t jules_hip_w8a16_noalloc_max_bytes(void);
int jules_hip_w8a16_gemm_bias_act_noalloc(int act, const void* x, const int8_t* W,
                                          const float* scale, const float* bias,
                                          void* y, int M, int N, int K, void* stream);
/* Diagnostics for the entry point above (no reference counterpart): copies
 * the first n (0 <= n <= 1024) per-column-tile arrival counters of the
 * current GPU's static array into host memory out, after waiting for the
 * device.  Every call that has finished leaves them all 0; a counter that is
 * not 0 with no call running means a launch was aborted part-way. */
int jules_hip_w8a16_noalloc_counters(uint32_t* out, int n);

/* ---- int8 x int8 GEMM (matmulInt8 semantics) -------------------------------
 * C[i,j] = float(sum_k A[i,k]*B[k,j]) * (scale_A*scale_B) [+ bias[j]]
 * Replaces matmulInt8(A,B,C,M,N,K,scale_A,scale_B,bias,arena) with the
 * semantics of its scalar path (reference FusedKernels.h:1046-1066): exact
 * int32 accumulation, B indexed B[k*N+j]; the product scale_A*scale_B is
 * rounded to fp32 first, then one multiply, then one add of bias.
 * (The reference's AVX-512F and VNNI paths index the wrong columns; this
 * entry point follows the scalar path.)  K <= 131071 keeps the int32 sum
 * exact (every product is at most 2^14); larger K returns JH_ERR_SHAPE.
 * M <= 16 (decode) keeps its split-K partials in a device buffer the library
 * keeps per (device, stream), allocated on the first call that needs it.
 */
int jules_hip_matmul_int8(const int8_t* A, const int8_t* B, float* C, int M,
                          int N, int K, float scale_A, float scale_B,
                          const float* bias, void* stream);

/* ---- W8A8 GEMM with per-token / per-channel scales ---------------------------
 * C[i,j] = float(sum_k A[i,k]*B[k,j]) * (sA_i * sB_j) [+ bias[j]]
 * The matmulInt8 the routing pass would emit once QuantizePass carries
 * scales (the reference's matmulInt8, FusedKernels.h:867-1073, has
 * per-tensor scales only): B indexed B[k*N+j]
 * like the scalar path, exact int32 accumulation, the scale product
 * sA_i * sB_j rounded to fp32 per element, one multiply, one add of bias.
 * With constant scale vectors the result equals jules_hip_matmul_int8 bit for
 * bit.  scale_A: fp32 [M] per-token scales, or NULL for 1; scale_B: fp32 [N]
 * per-output-channel scales (required).  K <= 131071.
 */
int jules_hip_matmul_w8a8(const int8_t* A, const int8_t* B, float* C, int M,
                          int N, int K, const float* scale_A,
                          const float* scale_B, const float* bias, void* stream);

/* ---- row kernels ----------------------------------------------------------
 * fp32, row-major [M, N], device pointers, 4-byte aligned; out may alias in.
 * Each row is processed with the reference's per-element arithmetic (exp
 * split: fast_exp for j < N & ~15, expf for the tail; reciprocal multiply
 * vs divide likewise); sums are taken in a fixed tree order, so results
 * match the reference to rounding and are deterministic run to run.
 * Up to 64 rows longer than 65536 are split over workgroups (three
 * launches); their partial maxima and sums, 8*M*ceil(N/4096) bytes, go to a
 * device buffer the library keeps per (device, stream), allocated on the
 * first call that needs it (calls on one stream share it in order).
 *
 * jules_hip_softmax: out[i,:] = softmax(in[i,:]).
 *   Replaces fusedSoftmax(output, input, M, N)
 *   (reference include/jules/Kernel/FusedKernels.h:464-526); routed name
 *   "fusedSoftmax" (KernelRoutingPass.cpp:261).
 *
 * jules_hip_layernorm: out[i,j] = (in[i,j]-mean_i)*rstd_i*gamma[j] + beta[j],
 *   rstd_i = 1/sqrtf(var_i + epsilon), population variance.
 *   Replaces fusedLayerNorm(output, input, gamma, beta, M, N, epsilon)
 *   (FusedKernels.h:532-600; the reference's default epsilon is 1e-5f);
 *   routed name "fusedLayerNorm" (KernelRoutingPass.cpp:330).
 *
 * jules_hip_cross_entropy: grad[i,:] = (softmax(logits[i,:]) - onehot(t_i))/M,
 *   *loss = mean_i -logf(p_i[t_i] + 1e-10f), written to device memory.
 *   Replaces float fusedCrossEntropyLoss(logits, targets, grad, M, N)
 *   (FusedKernels.h:766-854), which returns the loss by value; routed name
 *   "fusedCrossEntropyLoss" (KernelRoutingPass.cpp:378).  targets: int32 [M]
 *   on the device; a target outside [0, N) gives a NaN loss for its row
 *   (the reference reads out of bounds).  workspace: device memory of at
 *   least jules_hip_cross_entropy_workspace_size(M) bytes (per-row losses),
 *   overwritten by every call; M = 0 writes a NaN loss (0/0, as the
 *   reference's total_loss / M).
 */
int jules_hip_softmax(float* out, const float* in, int M, int N, void* stream);
int jules_hip_layernorm(float* out, const float* in, const float* gamma,
                        const float* beta, int M, int N, float epsilon,
                        void* stream);
size_t jules_hip_cross_entropy_workspace_size(int M);
int jules_hip_cross_entropy(const float* logits, const int32_t* targets,
                            float* grad, float* loss, int M, int N,
                            void* workspace, size_t workspace_bytes,
                            void* stream);

/* ---- 2-layer MLP forward ---------------------------------------------------
 * output [M,N2] = relu(X W1 + b1) W2 + b2, fp32 row-major; X [M,K1],
 * W1 [K1,N1], b1 [N1], W2 [N1,N2], b2 [N2].
 * Replaces fusedMLPForward(output, X, MLPParams{W1,b1,W2,b2,M,K1,N1,N2},
 * arena, planner) (FusedKernels.h:650-760); routed name "fusedMLPForward"
 * (KernelRoutingPass.h:20): (X, W1, b1, W2, b2) -> output.  The products are
 * fp32 MFMA GEMMs (the reference's are BLAS calls: results agree to fp32
 * rounding).  workspace: jules_hip_mlp_forward_workspace_size(M,K1,N1,N2)
 * bytes (the hidden activations), 16-byte aligned, no initialisation.
 */
size_t jules_hip_mlp_forward_workspace_size(int M, int K1, int N1, int N2);
int jules_hip_mlp_forward(const float* X, const float* W1, const float* b1,
                          const float* W2, const float* b2, float* output,
                          int M, int K1, int N1, int N2,
                          void* workspace, size_t workspace_bytes, void* stream);

/* ---- 2-layer MLP forward + loss + backward --------------------------------
 * Replaces interleavedMLPForwardBackward (include/jules/Kernel/
 * InterleavedAutodiff.h:55-62): same operands in the same order, minus the
 * ExecutionArena/TilePlanner, plus loss/workspace/stream.  fp32 row-major:
 * X [M,K1], W1 [K1,N1], b1 [N1], W2 [N1,N2], b2 [N2], targets [M] int32.
 *   output [M,N2] = relu(X W1 + b1) W2 + b2
 *   *loss (device float) = mean_i -log(softmax(output_i)[t_i] + 1e-10)
 *   dW1 [K1,N1], db1 [N1], dW2 [N1,N2], db2 [N2]: gradients of the loss
 *   dX [M,K1] or NULL
 * Gradients are overwritten (the reference zeroes them first).  A target
 * outside [0,N2) gives a NaN row loss and no one-hot term, as in
 * jules_hip_cross_entropy.  M = 0 zeroes the gradients and writes a NaN loss
 * (the reference's 0/0).  Deterministic.
 * workspace: jules_hip_mlp_workspace_size(M,K1,N1,N2) bytes, 16-byte aligned
 * (activations, dO, dH, row losses, column-sum partials); no initialisation.
 * Routed name "interleavedMLPForwardBackward" (KernelRoutingPass.h:21):
 * (X, W1, b1, W2, b2, targets) -> (output, dW1, db1, dW2, db2, loss[, dX]).
 */
size_t jules_hip_mlp_workspace_size(int M, int K1, int N1, int N2);
int jules_hip_mlp_forward_backward(const float* X, const float* W1, const float* b1,
                                   const float* W2, const float* b2, const int32_t* targets,
                                   float* output, float* dW1, float* db1, float* dW2,
                                   float* db2, float* dX, int M, int K1, int N1, int N2,
                                   float* loss, void* workspace, size_t workspace_bytes,
                                   void* stream);

/* ---- MFMA calibration -----------------------------------------------------
 * No counterpart in the reference: a roofline calibration for callers that
 * report MFMA rates against the rate the part sustains under load (its engine
 * clock drops under the power limit when the matrix cores are busy).  Launches
 * `workgroups` x 4 waves; each wave issues 16 * iters independent
 * v_mfma_f32_32x32x16_bf16 on random bf16 operands held in registers, i.e.
 * 32768 * 16 * iters * 4 * workgroups FLOP in total.  out: device fp32
 * [workgroups * 256], 4-byte aligned; its values only keep the work live.
 * workgroups in [1, 65535], iters in [1, 1 << 20].
 */
int jules_hip_mfma_ceiling(float* out, int workgroups, int iters, void* stream);

/* ---- HBM read calibration ---------------------------------------------------
 * No counterpart in the reference: the read rate a plain streaming read
 * attains, the floor an HBM-bound kernel such as the W8A16 GEMM is compared
 * with next to the published 8 TB/s.  Reads `bytes` (a multiple of 16) of
 * `buf` once with 16-byte nontemporal loads, 8 in flight per lane, from
 * `workgroups` x 256 lanes (256 workgroups measured fastest for 64 MiB);
 * out: device uint32 [workgroups * 256], 4-byte aligned, receives values that
 * only keep the loads live.  buf 16-byte aligned.
 */
int jules_hip_hbm_read_floor(const void* buf, int64_t bytes, uint32_t* out, int workgroups,
                             void* stream);

/* ---- kernel-name registry -------------------------------------------------
 * Resolves the names KernelRoutingPass emits (fusedMatmul{Relu,Sigmoid,Tanh,
 * Gelu}, fusedMatmulBias{Relu,Sigmoid,Tanh,Gelu}, fusedGelu, matmulInt8,
 * flashAttention, fusedSoftmax, fusedLayerNorm, fusedCrossEntropyLoss) and
 * the ones this library adds (fusedMatmul,
 * fusedMatmulBias, fusedMatmulBiasSilu, flashAttentionCausal,
 * matmulW8A16BiasSilu, matmulW8A8) to a descriptor-based entry point.  The descriptor
 * extends the reference's TensorDescriptor (include/jules/LLVMBackend.h:60-66:
 * data, offset, sizes[6], strides[6], rank) with a dtype; data + offset is
 * the device address of element 0 and strides are in elements.
 * Operand order follows extern_kernel: (lhs, rhs[, bias]) for the matmuls
 * (KernelRoutingPass.cpp:154,198), (Q, K, V) for attention,
 * (x, W, scale[, bias]) for W8A16, (A, B, scale_A, scale_B[, bias]) for
 * matmulW8A8, (A, B[, bias]) plus backend_config
 * "scale_a=<f>,scale_b=<f>" for matmulInt8 (the reference emits no scales,
 * KernelRoutingPass.cpp:406-410).  Attention accepts backend_config
 * "scale=<f>"; the default is 1/sqrtf(D).  Row kernels: (x) -> y for
 * fusedSoftmax, (x, gamma, beta) -> y with backend_config "epsilon=<f>"
 * (default 1e-5) for fusedLayerNorm, (logits, targets) -> (grad, loss) for
 * fusedCrossEntropyLoss (loss: one fp32 element); rows are the last
 * dimension.  W8A16, cross entropy and the MLP entries need a workspace;
 * the registry uses a library-held buffer per (device, stream), grown on
 * demand: calls on one stream share it in stream order, calls on different
 * streams never share one.
 */
typedef struct jh_tensor {
    void* data;
    int64_t offset;
    int64_t sizes[6];
    int64_t strides[6];
    int32_t rank;
    int32_t dtype; /* jh_dtype */
} jh_tensor;

typedef int (*jh_kernel_fn)(int n_inputs, const jh_tensor* inputs,
                            int n_outputs, jh_tensor* outputs,
                            const char* backend_config, void* stream);

jh_kernel_fn jules_hip_lookup(const char* name);
int jules_hip_kernel_count(void);
const char* jules_hip_kernel_name(int index);

/* ---- ROCm PJRT executor ----------------------------------------------------
 * C access to the ROCm PJRT client of jules_hip_pjrt.hpp, whose classes
 * mirror the reference's PJRTClient / PJRTDevice / PJRTExecutable
 * (include/jules/PJRT.h:113-233).  A program is StableHLO text in generic op
 * form, read with the reference CPU executable's parse rules and op semantics
 * (lib/PJRT.cpp:169-858); stablehlo.custom_call runs the registry kernel its
 * call_target_name names instead of the reference's copy (PJRT.cpp:491-499).
 *
 * jules_hip_pjrt_compile: loads `program` onto GPU `device`; *exe receives a
 *   handle for execute/destroy.
 * jules_hip_pjrt_execute: runs the program on the inputs (contiguous device
 *   tensors, not modified) and returns after the GPU is done.  outputs[0..)
 *   receive descriptors of every value the program produced, in program
 *   order (*n_outputs of them; JH_ERR_WORKSPACE when more than max_outputs).
 *   Their memory belongs to the handle and stays valid until the next execute
 *   on it or its destruction.
 * jules_hip_pjrt_describe: the parsed op list for n_inputs inputs as text
 *   (needs no GPU); JH_ERR_WORKSPACE if buf_len is too small.
 */
typedef struct jh_pjrt_exe jh_pjrt_exe;
int jules_hip_pjrt_compile(const char* program, int device, jh_pjrt_exe** exe);
int jules_hip_pjrt_execute(jh_pjrt_exe* exe, int n_inputs, const jh_tensor* inputs,
                           int max_outputs, jh_tensor* outputs, int* n_outputs);
int jules_hip_pjrt_destroy(jh_pjrt_exe* exe);
int jules_hip_pjrt_describe(const char* program, int n_inputs, char* buf, size_t buf_len);

#ifdef __cplusplus
}
#endif
#endif /* JULES_HIP_H */
