/*
 * jules_oracle.h - CPU restatement of the Jules AVX-512 kernel path, plus an
 * fp64 oracle.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library (libjules_hip.so)
 * links, loads or calls this code.  It is used by tests/ as the checker, by
 * __graft_entry__.smoke() as the checker, and by bench.py's cpu_baseline leg
 * as the timed CPU port of the reference AVX-512 path.
 *
 * Two families of functions:
 *
 *  jo_*   fp32 restatement of the reference kernels, written from the
 *         reference's algorithm (file:line cited per function).  Where every
 *         operation of the reference is an IEEE-754 primitive (fma, mul, add,
 *         div, floor, exponent-bit construction) the restatement performs the
 *         same primitives in the same order, so it reproduces the reference's
 *         bits.  Where the reference calls a third-party BLAS (the score tiles
 *         of flashAttention) the bits are BLAS-dependent and the restatement
 *         only matches to rounding.
 *
 *  jo64_* fp64 oracle: textbook definitions evaluated in double precision.
 *         This is what every kernel's error is measured against.
 *
 * Activation codes follow jules::kernel::ActivationType
 * (reference include/jules/Kernel/FusedKernels.h:61-67) with SiLU appended:
 *   0 None, 1 Relu, 2 Sigmoid, 3 Tanh, 4 Gelu, 5 Silu.
 *
 * Pinning status (what checks each function; see tests/test_oracle.py):
 *   jo_fast_exp        fp64 exp over a dense fp32 sweep of [-88,88] + special points
 *   jo_gelu/sigmoid/
 *   jo_tanh/silu       fp64 closed forms over a sweep; known values
 *   jo_tiled_matmul_act/
 *   jo_matmul_bias_act numpy fp64 GEMM, B=I, K=1, A=0 closed forms, brute
 *                      force on ragged shapes, tile-invariance
 *   jo_flash_attention fp64 softmax attention; V=1 => O=1; Q=0 => mean of V
 *                      (prefix means when causal); causal row 0 = V[0];
 *                      key-permutation invariance (non-causal); tiling
 *                      invariance; S=1 and ragged S
 *   jo_matmul_int8     exact int64 numpy reference; one-hot KAT
 *   jo_w8a16           numpy fp64; one-hot KAT (bit-exact dequant)
 *   jo_softmax         fp64 softmax; rows sum to 1; shift invariance; uniform
 *                      rows give 1/N; N = 1; the 16-lane/tail split at N = 15,
 *                      16, 17, 31, 33
 *   jo_layernorm       fp64 layernorm; constant rows give beta; gamma = 1,
 *                      beta = 0 rows have mean 0 and variance var/(var+eps)
 *   jo_cross_entropy   fp64 loss and gradient; uniform logits give log N;
 *                      gradient rows sum to 0; grad[target] = (p - 1)/M
 *   jo64_*             independent numpy fp64 implementations at small sizes
 * The reference itself cannot be compiled in this image (its headers include
 * <cblas.h>, which the image lacks), so no function is pinned against
 * reference-produced vectors; the reference ships none either.
 */
#ifndef JULES_ORACLE_H
#define JULES_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { JO_ACT_NONE = 0, JO_ACT_RELU = 1, JO_ACT_SIGMOID = 2, JO_ACT_TANH = 3,
       JO_ACT_GELU = 4, JO_ACT_SILU = 5 };

/* ---- scalar activation helpers (reference FusedKernels.h:81-164) ---- */
float jo_fast_exp(float x);
float jo_fast_tanh(float x);
float jo_sigmoid(float x);
float jo_gelu(float x);
float jo_silu(float x);
float jo_act(int act, float x);          /* vector-path epilogue, :408-414 */
float jo_act_tail(int act, float x);     /* scalar-tail epilogue, :424-430 */
void  jo_act_array(int act, float* out, const float* in, int64_t n);
void  jo_fast_exp_array(float* out, const float* in, int64_t n);

/* fusedGelu (reference FusedKernels.h:606-627) */
void jo_fused_gelu(float* out, const float* in, int n);

/* tiledMatmulWithActivation (reference FusedKernels.h:378-458) */
void jo_tiled_matmul_act(const float* A, const float* B, float* C,
                         int M, int N, int K, int tile_m, int tile_n,
                         int tile_k, int act);

/* act(A.B + bias): the bias epilogue of fusedMatmulBiasRelu
 * (reference FusedKernels.h:265-372, epilogue :308-313) generalised to every
 * activation.  bias may be NULL (then this is tiledMatmulWithActivation).
 * Argument order (M,K,N) as in the reference. */
void jo_matmul_bias_act(const float* X, const float* W, const float* bias,
                        float* out, int M, int K, int N, int tile_m,
                        int tile_n, int tile_k, int act);

/* TilePlanner::computeAnalytical (reference TilePlanner.h:97-136) given
 * cache sizes; writes tile_m, tile_n, tile_k. */
void jo_tile_analytical(int M, int N, int K, int64_t l1d_bytes,
                        int64_t l2_bytes, int avx512, int* tm, int* tn,
                        int* tk);

/* flashAttention (reference FlashAttention.h:130-309), extended with a causal
 * mask (key j > query i excluded, fully masked key tiles skipped) and an
 * explicit scale.  tile_q/tile_k as chosen by the reference's tile shrink
 * (:137-149); pass 32/64 for the unshrunk defaults.  Layout [B,H,S,D]. */
void jo_flash_attention(float* out, const float* Q, const float* K,
                        const float* V, int B, int H, int S, int D,
                        int tile_q, int tile_k, int causal, float scale);

/* the tile shrink of flashAttention (reference FlashAttention.h:137-149) */
void jo_flash_tiles(int S, int D, int64_t l2_bytes, int* tile_q, int* tile_k);

/* matmulInt8 scalar semantics (reference FusedKernels.h:1046-1066):
 * C[i,j] = float(sum_k A[i,k]*B[k,j]) * (sA*sB) [+ bias[j]] */
void jo_matmul_int8(const int8_t* A, const int8_t* B, float* C, int M, int N,
                    int K, float scale_A, float scale_B, const float* bias);

/* W8A16 GEMM + bias + act (no reference counterpart; restated from
 * matmulInt8's indexing W[k*N+j] and the activation helpers):
 *   acc    = sum_k x[m,k] * float(W[k*N+j])   (fp32, sequential k)
 *   y[m,j] = act(acc * scale[j] + bias[j])
 * x holds bf16 values widened to fp32. bias may be NULL. */
void jo_w8a16(const float* x, const int8_t* W, const float* scale,
              const float* bias, float* y, int M, int N, int K, int act);

/* ---- fp64 oracle ---- */
double jo64_act(int act, double x);
/* C[r,:] = act(A[rows[r],:] . B + bias) in fp64 for the listed rows
 * (rows==NULL: all M rows, nrows ignored). */
void jo64_gemm_bias_act(const float* A, const float* B, const float* bias,
                        double* C, int M, int N, int K, int act,
                        const int* rows, int nrows);
/* One head: O[r,:] = softmax(scale * Q[q_r,:] K^T) V over keys j (j <= q_r if
 * causal), for the listed query rows (rows==NULL: all S rows). */
void jo64_attention_head(const float* Q, const float* K, const float* V,
                         double* O, int S, int D, int causal, double scale,
                         const int* rows, int nrows);
void jo64_w8a16(const float* x, const int8_t* W, const float* scale,
                const float* bias, double* y, int M, int N, int K, int act);

/* threads the OpenMP runtime will use (for reporting the CPU baseline) */
/* ---- row kernels (reference FusedKernels.h:464-526, :532-600, :766-854) ---- */
void  jo_softmax(float* out, const float* in, int M, int N);
void  jo_layernorm(float* out, const float* in, const float* gamma,
                   const float* beta, int M, int N, float eps);
float jo_cross_entropy(const float* logits, const int32_t* targets, float* grad,
                       int M, int N);
void   jo64_softmax(double* out, const float* in, int M, int N);
void   jo64_layernorm(double* out, const float* in, const float* gamma,
                      const float* beta, int M, int N, double eps);
double jo64_cross_entropy(const float* logits, const int32_t* targets,
                          double* grad, int M, int N);

int jo_max_threads(void);
void jo_set_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
