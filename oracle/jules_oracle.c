/*
 * jules_oracle.c - CPU restatement of the Jules AVX-512 kernel path and an
 * fp64 oracle.  TEST INFRASTRUCTURE ONLY: used by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg, never by the
 * product library.  The declarations and the pinning status of every function
 * are in jules_oracle.h.
 *
 * Build: oracle/build_oracle.py (gcc -O3 -ffp-contract=off -fopenmp).  The
 * hot loops carry target_clones so one .so built here runs on any x86-64 host
 * and still uses 512-bit FMA where the host has AVX-512F.
 *
 * -ffp-contract=off matters: the restatement spells out every fma the
 * reference's compiled code performs and nothing else.  Those fmas are more
 * than the reference's explicit _mm512_fmadd_ps calls: g++ (11.4, the image's
 * compiler, C++ at its default -ffp-contract=fast, the flags of
 * benchmarks/bench_kernel.cpp:15-19 plus -mavx512bw) expands _mm512_add_ps,
 * _mm512_sub_ps and _mm512_mul_ps into generic vector arithmetic and then
 * fuses a product into every add or subtract that consumes it, when every use
 * of the product is one.  The places where that happens on this path are
 * marked "contracted" below; tests/cpp/gxx_activation_probe.cpp compiles the
 * intrinsic sequences with those flags and tests/test_oracle.py checks the
 * restatement against its output bit for bit.
 */
#include "jules_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define HOT __attribute__((target_clones("avx512f", "avx2,fma", "default")))

static inline float bits_to_float(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline int imin(int a, int b) { return a < b ? a : b; }

/* ------------------------------------------------------------------------ */
/* Activation helpers                                                        */
/* ------------------------------------------------------------------------ */

/* fast_exp_zmm, reference FusedKernels.h:90-133, one lane, as its two
 * factors: clamp to [-88,88] (:92-95; min/max return the bound for NaN like
 * minps/maxps with the bound as second operand) -> r = x*log2(e) (:98-99) ->
 * floor split (:102-104) -> degree-6 Horner in fma (:109-123) -> 2^floor built
 * from exponent bits (:127-130).  The result is their product (:132); a caller
 * that only adds or subtracts that product gets it fused instead. */
static inline void fast_exp_parts(float x, float* scale, float* poly) {
    x = (x < 88.0f) ? x : 88.0f;   /* _mm512_min_ps(x, 88): NaN -> 88 */
    x = (x > -88.0f) ? x : -88.0f; /* _mm512_max_ps(x, -88) */
    const float r = x * 1.4426950408889634f; /* r also feeds the floor: not fused */
    const float ri = floorf(r);
    const float rf = r - ri;
    float p = fmaf(0.000154040f, rf, 0.001333356f);
    p = fmaf(p, rf, 0.009614425f);
    p = fmaf(p, rf, 0.055495506f);
    p = fmaf(p, rf, 0.240226507f);
    p = fmaf(p, rf, 0.693147180f);
    p = fmaf(p, rf, 1.0f);
    const int32_t e = ((int32_t)ri + 127) << 23; /* cvttps, add 127, shift 23 */
    *scale = bits_to_float((uint32_t)e);
    *poly = p;
}

float jo_fast_exp(float x) {
    float s, p;
    fast_exp_parts(x, &s, &p);
    return s * p;
}

/* fast_tanh_zmm, reference FusedKernels.h:137-143: (e^{2x}-1)/(e^{2x}+1).
 * e = scale*poly is used only by the subtract and the add, so both are
 * contracted: (fma(s,p,-1)) / (fma(s,p,1)). */
float jo_fast_tanh(float x) {
    float s, p;
    fast_exp_parts(2.0f * x, &s, &p);
    return fmaf(s, p, -1.0f) / fmaf(s, p, 1.0f);
}

/* sigmoid_zmm, reference FusedKernels.h:146-152: 1/(1+exp(0-x)); the add is
 * contracted: 1/fma(s,p,1). */
float jo_sigmoid(float x) {
    float s, p;
    fast_exp_parts(0.0f - x, &s, &p);
    return 1.0f / fmaf(s, p, 1.0f);
}

/* gelu_zmm, reference FusedKernels.h:155-164:
 * 0.5*(x*(1+tanh(c*(x + d*(x*(x*x)))))) with c=0.7978845608, d=0.044715;
 * x + d*x3 is contracted to fma(d, x3, x). */
float jo_gelu(float x) {
    const float x3 = x * (x * x);
    const float inner = 0.7978845608f * fmaf(0.044715f, x3, x);
    const float t = jo_fast_tanh(inner);
    return 0.5f * (x * (1.0f + t));
}

/* SiLU has no reference kernel; built from sigmoid_zmm as x*sigmoid(x). */
float jo_silu(float x) { return x * jo_sigmoid(x); }

/* Vector-path epilogue switch, reference FusedKernels.h:408-414.
 * relu_zmm (:81-83) is maxps(x, 0): NaN and -0 give +0. */
float jo_act(int act, float x) {
    switch (act) {
    case JO_ACT_RELU: return (x > 0.0f) ? x : 0.0f;
    case JO_ACT_SIGMOID: return jo_sigmoid(x);
    case JO_ACT_TANH: return jo_fast_tanh(x);
    case JO_ACT_GELU: return jo_gelu(x);
    case JO_ACT_SILU: return jo_silu(x);
    default: return x;
    }
}

/* The scalar GELU formula of the reference's tails (FusedKernels.h:426,
 * :616): 0.5f*x*(1+tanhf(c*(x + 0.044715f*x*x*x))), evaluated left to right,
 * with x + (0.044715f*x*x)*x contracted to one fma. */
static inline float gelu_tail(float x) {
    return 0.5f * x * (1.0f + tanhf(0.7978845608f * fmaf(0.044715f * x * x, x, x)));
}

/* Scalar-tail epilogue, reference FusedKernels.h:424-430 (columns past the
 * last full 16-wide vector of a tile): libm tanhf/expf and std::max. */
float jo_act_tail(int act, float s) {
    switch (act) {
    case JO_ACT_RELU: return (s < 0.0f) ? 0.0f : s; /* std::max(s, 0.0f) */
    case JO_ACT_GELU:
        return gelu_tail(s);
    case JO_ACT_SIGMOID: return 1.0f / (1.0f + expf(-s));
    case JO_ACT_TANH: return tanhf(s);
    case JO_ACT_SILU: return s / (1.0f + expf(-s));
    default: return s;
    }
}

void jo_fast_exp_array(float* out, const float* in, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) out[i] = jo_fast_exp(in[i]);
}

void jo_act_array(int act, float* out, const float* in, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) out[i] = jo_act(act, in[i]);
}

/* fusedGelu, reference FusedKernels.h:606-627: full 16-groups through
 * gelu_zmm, the last partial group through the tanhf formula. */
void jo_fused_gelu(float* out, const float* in, int n) {
#pragma omp parallel for schedule(static)
    for (int i = 0; i < n; i += 16) {
        if (i + 15 < n) {
            for (int l = 0; l < 16; l++) out[i + l] = jo_gelu(in[i + l]);
        } else {
            for (int j = i; j < n; j++) out[j] = gelu_tail(in[j]);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Tiled GEMM with activation                                                */
/* ------------------------------------------------------------------------ */

/* One (i, 16-column) register block of the tiled kernel's inner loop,
 * reference FusedKernels.h:401-406: c = C; for kk: c = fma(A[i,k], B[k,j:j+16], c). */
HOT static void gemm_tile_rows(const float* A, const float* B, float* C, int N,
                               int K, int ti, int tm_curr, int tj, int tn_curr,
                               int tkk, int tk_curr, int last, const float* bias,
                               int act) {
    for (int i = 0; i < tm_curr; i++) {
        const float* arow = A + (int64_t)(ti + i) * K + tkk;
        float* crow = C + (int64_t)(ti + i) * N + tj;
        int j = 0;
        for (; j + 15 < tn_curr; j += 16) {
            float c[16];
            for (int l = 0; l < 16; l++) c[l] = crow[j + l];
            for (int kk = 0; kk < tk_curr; kk++) {
                const float a = arow[kk];
                const float* brow = B + (int64_t)(tkk + kk) * N + tj + j;
#pragma omp simd
                for (int l = 0; l < 16; l++) c[l] = fmaf(a, brow[l], c[l]);
            }
            if (last) {
                if (bias) {
                    for (int l = 0; l < 16; l++) c[l] = c[l] + bias[tj + j + l];
                }
                for (int l = 0; l < 16; l++) c[l] = jo_act(act, c[l]);
            }
            for (int l = 0; l < 16; l++) crow[j + l] = c[l];
        }
        /* scalar tail (:418-433 / :316-326) */
        for (; j < tn_curr; j++) {
            float sum = crow[j];
            for (int kk = 0; kk < tk_curr; kk++)
                sum = fmaf(arow[kk], B[(int64_t)(tkk + kk) * N + tj + j], sum);
            if (last) {
                if (bias) sum = sum + bias[tj + j];
                sum = jo_act_tail(act, sum);
            }
            crow[j] = sum;
        }
    }
}

/* Loop nest of tiledMatmulWithActivation (reference FusedKernels.h:382-417)
 * and of fusedMatmulBiasRelu's tiled path (:283-345): zero C, OpenMP over
 * row tiles, then tj -> tkk; the epilogue fires when tkk + tile_k >= K. */
static void tiled_gemm(const float* A, const float* B, const float* bias,
                       float* C, int M, int N, int K, int tm, int tn, int tk,
                       int act) {
    memset(C, 0, (size_t)M * N * sizeof(float));
    if (tm <= 0 || tn <= 0 || tk <= 0) return;
#pragma omp parallel for schedule(dynamic)
    for (int ti = 0; ti < M; ti += tm) {
        const int tm_curr = imin(tm, M - ti);
        for (int tj = 0; tj < N; tj += tn) {
            const int tn_curr = imin(tn, N - tj);
            for (int tkk = 0; tkk < K; tkk += tk) {
                const int tk_curr = imin(tk, K - tkk);
                gemm_tile_rows(A, B, C, N, K, ti, tm_curr, tj, tn_curr, tkk,
                               tk_curr, tkk + tk >= K, bias, act);
            }
        }
    }
    /* K == 0: the reference never enters the tkk loop, so C stays zero and no
     * activation is applied. */
}

void jo_tiled_matmul_act(const float* A, const float* B, float* C, int M,
                         int N, int K, int tile_m, int tile_n, int tile_k,
                         int act) {
    tiled_gemm(A, B, NULL, C, M, N, K, tile_m, tile_n, tile_k, act);
}

void jo_matmul_bias_act(const float* X, const float* W, const float* bias,
                        float* out, int M, int K, int N, int tile_m,
                        int tile_n, int tile_k, int act) {
    tiled_gemm(X, W, bias, out, M, N, K, tile_m, tile_n, tile_k, act);
}

/* TilePlanner::computeAnalytical, reference TilePlanner.h:97-136 */
void jo_tile_analytical(int M, int N, int K, int64_t l1d_bytes,
                        int64_t l2_bytes, int avx512, int* tm, int* tn,
                        int* tk) {
    int m = avx512 ? 32 : 16, n = avx512 ? 32 : 16, k = avx512 ? 128 : 64;
    const int64_t l1_budget = l1d_bytes * 3 / 4;
#define FOOT(m_, n_, k_) (((int64_t)(m_) * (k_) + (int64_t)(k_) * (n_) + (int64_t)(m_) * (n_)) * 4)
    while (FOOT(m, n, k) > l1_budget && k > 16) k /= 2;
#undef FOOT
    const int64_t l2_budget = l2_bytes * 3 / 4;
    if ((int64_t)K * N * 4 <= l2_budget) k = K;
    m = imin(m, M);
    n = imin(n, N);
    k = imin(k, K);
    const int vw = avx512 ? 16 : 8;
    m = (m / vw) * vw;
    n = (n / vw) * vw;
    if (m == 0) m = vw;
    if (n == 0) n = vw;
    *tm = m; *tn = n; *tk = k;
}

/* ------------------------------------------------------------------------ */
/* Flash attention                                                           */
/* ------------------------------------------------------------------------ */

/* tile shrink, reference FlashAttention.h:137-149 */
void jo_flash_tiles(int S, int D, int64_t l2_bytes, int* tile_q, int* tile_k) {
    int tq = 32, tk = 64;
    const int64_t budget = l2_bytes * 3 / 4;
    int64_t per = (int64_t)tq * (D + S) * 4 + (int64_t)tk * D * 4;
    while (per > budget && tq > 4) {
        tq /= 2;
        per = (int64_t)tq * (D + S) * 4 + (int64_t)tk * D * 4;
    }
    while (per > budget && tk > 8) {
        tk /= 2;
        per = (int64_t)tq * (D + S) * 4 + (int64_t)tk * D * 4;
    }
    *tile_q = tq;
    *tile_k = tk;
}

/* _mm512_reduce_add_ps as GCC expands it: halves, quarters, then pairs. */
static inline float reduce_add16(const float* e) {
    float t3[8], t6[4];
    for (int i = 0; i < 8; i++) t3[i] = e[i + 8] + e[i];
    for (int i = 0; i < 4; i++) t6[i] = t3[i + 4] + t3[i];
    const float a = t6[0] + t6[2], b = t6[1] + t6[3];
    return a + b;
}

HOT static void flash_head(float* out, const float* q, const float* k,
                           const float* v, int S, int D, int tile_q,
                           int tile_k, int causal, float scale, float* acc,
                           float* mx, float* sm, float* scores) {
    memset(out, 0, (size_t)S * D * sizeof(float));
    for (int tq = 0; tq < S; tq += tile_q) {
        const int tq_curr = imin(tile_q, S - tq);
        for (int i = 0; i < tq_curr; i++) { mx[i] = -FLT_MAX; sm[i] = 0.0f; }
        memset(acc, 0, (size_t)tq_curr * D * sizeof(float));
        for (int tk = 0; tk < S; tk += tile_k) {
            /* causal extension: key tiles wholly above the diagonal are skipped */
            if (causal && tk > tq + tq_curr - 1) break;
            const int tk_curr = imin(tile_k, S - tk);
            /* scores = scale * Q_t K_t^T (the reference calls cblas_sgemm with
             * alpha = scale, FlashAttention.h:184-188) */
            for (int i = 0; i < tq_curr; i++) {
                const float* qi = q + (int64_t)(tq + i) * D;
                for (int j = 0; j < tk_curr; j++) {
                    const float* kj = k + (int64_t)(tk + j) * D;
                    float s = 0.0f;
                    for (int d = 0; d < D; d++) s = fmaf(qi[d], kj[d], s);
                    scores[i * tk_curr + j] = scale * s;
                }
            }
            /* online softmax update, reference :192-254 */
            for (int i = 0; i < tq_curr; i++) {
                float* row = scores + i * tk_curr;
                const int qi = tq + i;
                /* number of keys of this tile visible to query qi */
                int nvis = tk_curr;
                if (causal) nvis = (qi - tk + 1 < tk_curr) ? qi - tk + 1 : tk_curr;
                if (nvis < 0) nvis = 0;
                float new_max = -FLT_MAX;
                for (int j = 0; j < nvis; j++) new_max = (row[j] > new_max) ? row[j] : new_max;
                const float old_max = mx[i];
                new_max = (old_max > new_max) ? old_max : new_max;
                float* ai = acc + (int64_t)i * D;
                if (old_max > -FLT_MAX) {
                    const float rescale = expf(old_max - new_max);
                    for (int d = 0; d < D; d++) ai[d] = ai[d] * rescale;
                    sm[i] = sm[i] * rescale;
                }
                float row_sum = 0.0f;
                int j = 0;
                for (; j + 15 < tk_curr; j += 16) {
                    float e[16];
                    for (int l = 0; l < 16; l++)
                        e[l] = (j + l < nvis) ? jo_fast_exp(row[j + l] - new_max) : 0.0f;
                    for (int l = 0; l < 16; l++) row[j + l] = e[l];
                    row_sum += reduce_add16(e);
                }
                for (; j < tk_curr; j++) {
                    row[j] = (j < nvis) ? expf(row[j] - new_max) : 0.0f;
                    row_sum += row[j];
                }
                /* acc[i,:] += p_j * V[tk+j,:], reference :238-250 */
                for (int jj = 0; jj < nvis; jj++) {
                    const float w = row[jj];
                    const float* vj = v + (int64_t)(tk + jj) * D;
#pragma omp simd
                    for (int d = 0; d < D; d++) ai[d] = fmaf(w, vj[d], ai[d]);
                }
                mx[i] = new_max;
                sm[i] = sm[i] + row_sum;
            }
        }
        /* final normalisation, reference :288-299 */
        for (int i = 0; i < tq_curr; i++) {
            const float inv = 1.0f / sm[i];
            float* oi = out + (int64_t)(tq + i) * D;
            const float* ai = acc + (int64_t)i * D;
            int d = 0;
            for (; d + 15 < D; d += 16)
                for (int l = 0; l < 16; l++) oi[d + l] = ai[d + l] * inv;
            for (; d < D; d++) oi[d] = ai[d] / sm[i];
        }
    }
}

void jo_flash_attention(float* out, const float* Q, const float* K,
                        const float* V, int B, int H, int S, int D,
                        int tile_q, int tile_k, int causal, float scale) {
    if (S <= 0 || D <= 0 || tile_q <= 0 || tile_k <= 0) return;
    const int BH = B * H;
#pragma omp parallel
    {
        float* acc = (float*)malloc((size_t)tile_q * D * sizeof(float));
        float* mx = (float*)malloc((size_t)tile_q * sizeof(float));
        float* sm = (float*)malloc((size_t)tile_q * sizeof(float));
        float* sc = (float*)malloc((size_t)tile_q * tile_k * sizeof(float));
#pragma omp for schedule(dynamic)
        for (int bh = 0; bh < BH; bh++) {
            const int64_t off = (int64_t)bh * S * D;
            flash_head(out + off, Q + off, K + off, V + off, S, D, tile_q,
                       tile_k, causal, scale, acc, mx, sm, sc);
        }
        free(acc); free(mx); free(sm); free(sc);
    }
}

/* ------------------------------------------------------------------------ */
/* Int8                                                                      */
/* ------------------------------------------------------------------------ */

/* matmulInt8 scalar semantics: reference FusedKernels.h:1046-1057 (int32
 * accumulate, B indexed B[k*N+j]) and epilogue :1060-1066. */
void jo_matmul_int8(const int8_t* A, const int8_t* B, float* C, int M, int N,
                    int K, float scale_A, float scale_B, const float* bias) {
    const float output_scale = scale_A * scale_B;
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; i++) {
        for (int j = 0; j < N; j++) {
            int32_t sum = 0;
            for (int k = 0; k < K; k++)
                sum += (int32_t)A[(int64_t)i * K + k] * (int32_t)B[(int64_t)k * N + j];
            float c = (float)sum * output_scale;
            if (bias) c = c + bias[j];
            C[(int64_t)i * N + j] = c;
        }
    }
}

/* W8A16 + bias + act.  Row-streaming restatement in the reference's matmulInt8
 * loop order (OpenMP over rows, FusedKernels.h:1006-1033): for each k the row
 * of W is broadcast-multiplied into the accumulator row. */
HOT static void w8a16_row(const float* xr, const int8_t* W, float* acc, int N,
                          int K) {
    for (int j = 0; j < N; j++) acc[j] = 0.0f;
    for (int k = 0; k < K; k++) {
        const float a = xr[k];
        const int8_t* wr = W + (int64_t)k * N;
#pragma omp simd
        for (int j = 0; j < N; j++) acc[j] = fmaf(a, (float)wr[j], acc[j]);
    }
}

void jo_w8a16(const float* x, const int8_t* W, const float* scale,
              const float* bias, float* y, int M, int N, int K, int act) {
#pragma omp parallel
    {
        float* acc = (float*)malloc((size_t)N * sizeof(float));
        /* rows are few (decode shape), so split columns across threads too */
#pragma omp for schedule(static)
        for (int i = 0; i < M; i++) {
            w8a16_row(x + (int64_t)i * K, W, acc, N, K);
            for (int j = 0; j < N; j++) {
                float t = acc[j] * scale[j];
                if (bias) t = t + bias[j];
                y[(int64_t)i * N + j] = jo_act(act, t);
            }
        }
        free(acc);
    }
}

/* ------------------------------------------------------------------------ */
/* fp64 oracle                                                               */
/* ------------------------------------------------------------------------ */

double jo64_act(int act, double x) {
    switch (act) {
    case JO_ACT_RELU: return x > 0.0 ? x : 0.0;
    case JO_ACT_SIGMOID: return 1.0 / (1.0 + exp(-x));
    case JO_ACT_TANH: return tanh(x);
    case JO_ACT_GELU: {
        const double c = sqrt(2.0 / 3.14159265358979323846);
        return 0.5 * x * (1.0 + tanh(c * (x + 0.044715 * x * x * x)));
    }
    case JO_ACT_SILU: return x / (1.0 + exp(-x));
    default: return x;
    }
}

void jo64_gemm_bias_act(const float* A, const float* B, const float* bias,
                        double* C, int M, int N, int K, int act,
                        const int* rows, int nrows) {
    const int R = rows ? nrows : M;
#pragma omp parallel
    {
        double* acc = (double*)malloc((size_t)(N > 0 ? N : 1) * sizeof(double));
#pragma omp for schedule(dynamic)
        for (int r = 0; r < R; r++) {
            const int i = rows ? rows[r] : r;
            for (int j = 0; j < N; j++) acc[j] = 0.0;
            for (int k = 0; k < K; k++) {
                const double a = A[(int64_t)i * K + k];
                const float* br = B + (int64_t)k * N;
                for (int j = 0; j < N; j++) acc[j] += a * (double)br[j];
            }
            for (int j = 0; j < N; j++)
                C[(int64_t)r * N + j] = jo64_act(act, acc[j] + (bias ? (double)bias[j] : 0.0));
        }
        free(acc);
    }
}

void jo64_attention_head(const float* Q, const float* K, const float* V,
                         double* O, int S, int D, int causal, double scale,
                         const int* rows, int nrows) {
    const int R = rows ? nrows : S;
#pragma omp parallel
    {
        double* p = (double*)malloc((size_t)(S > 0 ? S : 1) * sizeof(double));
#pragma omp for schedule(dynamic)
        for (int r = 0; r < R; r++) {
            const int i = rows ? rows[r] : r;
            const int nk = causal ? i + 1 : S;
            double m = -INFINITY;
            for (int j = 0; j < nk; j++) {
                double s = 0.0;
                for (int d = 0; d < D; d++)
                    s += (double)Q[(int64_t)i * D + d] * (double)K[(int64_t)j * D + d];
                p[j] = s * scale;
                if (p[j] > m) m = p[j];
            }
            double l = 0.0;
            for (int j = 0; j < nk; j++) { p[j] = exp(p[j] - m); l += p[j]; }
            for (int d = 0; d < D; d++) {
                double o = 0.0;
                for (int j = 0; j < nk; j++) o += p[j] * (double)V[(int64_t)j * D + d];
                O[(int64_t)r * D + d] = o / l;
            }
        }
        free(p);
    }
}

void jo64_w8a16(const float* x, const int8_t* W, const float* scale,
                const float* bias, double* y, int M, int N, int K, int act) {
#pragma omp parallel
    {
        double* acc = (double*)malloc((size_t)(N > 0 ? N : 1) * sizeof(double));
#pragma omp for schedule(static)
        for (int i = 0; i < M; i++) {
            for (int j = 0; j < N; j++) acc[j] = 0.0;
            for (int k = 0; k < K; k++) {
                const double a = x[(int64_t)i * K + k];
                const int8_t* wr = W + (int64_t)k * N;
                for (int j = 0; j < N; j++) acc[j] += a * (double)wr[j];
            }
            for (int j = 0; j < N; j++)
                y[(int64_t)i * N + j] = jo64_act(
                    act, acc[j] * (double)scale[j] + (bias ? (double)bias[j] : 0.0));
        }
        free(acc);
    }
}

int jo_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void jo_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* ======================================================================
 * Row kernels.  The reference's AVX-512 path keeps 16 lane partials for
 * the part of a row that fills whole 16-float vectors (j < N & ~15), folds
 * them with _mm512_reduce_* and finishes the < 16 tail with scalar code
 * (libm expf, sequential adds).  reduce16 folds the lanes by halves
 * (8+8, 4+4, 2+2, 1+1), the order of the GCC reduce intrinsics; the tail
 * is the reference's scalar loop.
 * ====================================================================== */
static float reduce16_add(const float* v) {
    float a[8], b[4], c[2];
    for (int i = 0; i < 8; ++i) a[i] = v[i + 8] + v[i];
    for (int i = 0; i < 4; ++i) b[i] = a[i + 4] + a[i];
    c[0] = b[0] + b[2];
    c[1] = b[1] + b[3];
    return c[0] + c[1];
}
static float reduce16_max(const float* v) {
    float m = v[0];
    for (int i = 1; i < 16; ++i) m = (v[i] > m) ? v[i] : m;
    return m;
}

/* One softmax row into out (reference FusedKernels.h:467-509): returns the
 * row sum.  The vector part uses fast_exp and out = e * (1/sum); the tail
 * uses expf and out = e / sum. */
static float softmax_row(float* out, const float* in, int N) {
    const int nv = N & ~15;
    float lane[16];
    for (int l = 0; l < 16; ++l) lane[l] = -FLT_MAX;
    /* _mm512_max_ps(acc, x) = acc > x ? acc : x (MAXPS returns its second
     * operand on NaN); std::max(m, x) = m < x ? x : m */
    for (int j = 0; j < nv; j += 16)
        for (int l = 0; l < 16; ++l) lane[l] = (lane[l] > in[j + l]) ? lane[l] : in[j + l];
    float mx = reduce16_max(lane); /* _mm512_reduce_max_ps */
    for (int j = nv; j < N; ++j) mx = (mx < in[j]) ? in[j] : mx;
    for (int l = 0; l < 16; ++l) lane[l] = 0.0f;
    for (int j = 0; j < nv; j += 16)
        for (int l = 0; l < 16; ++l) {
            const float e = jo_fast_exp(in[j + l] - mx);
            out[j + l] = e;
            lane[l] = lane[l] + e;
        }
    float sum = reduce16_add(lane);
    for (int j = nv; j < N; ++j) {
        const float e = expf(in[j] - mx);
        out[j] = e;
        sum += e;
    }
    const float inv = 1.0f / sum;
    for (int j = 0; j < nv; ++j) out[j] = out[j] * inv;
    for (int j = nv; j < N; ++j) out[j] = out[j] / sum;
    return sum;
}

/* fusedSoftmax, reference FusedKernels.h:464-526 (AVX-512 branch) */
void jo_softmax(float* out, const float* in, int M, int N) {
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; ++i) softmax_row(out + (int64_t)i * N, in + (int64_t)i * N, N);
}

/* fusedLayerNorm, reference FusedKernels.h:532-600 (AVX-512 branch).
 * Mean and variance: 16 lane partials over the vector part (the variance
 * with _mm512_fmadd_ps), reduce, scalar tail, then / N.  The tail's
 * `var += diff * diff` and `(x - mean) * inv_std * gamma + beta` are taken
 * as contracted to fma, as GCC does for C++ when FMA is available (the
 * vector path uses _mm512_fmadd_ps for both). */
void jo_layernorm(float* out, const float* in, const float* gamma, const float* beta,
                  int M, int N, float eps) {
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; ++i) {
        const float* x = in + (int64_t)i * N;
        float* y = out + (int64_t)i * N;
        const int nv = N & ~15;
        float lane[16];
        for (int l = 0; l < 16; ++l) lane[l] = 0.0f;
        for (int j = 0; j < nv; j += 16)
            for (int l = 0; l < 16; ++l) lane[l] = lane[l] + x[j + l];
        float mean = reduce16_add(lane);
        for (int j = nv; j < N; ++j) mean += x[j];
        mean /= (float)N;
        for (int l = 0; l < 16; ++l) lane[l] = 0.0f;
        for (int j = 0; j < nv; j += 16)
            for (int l = 0; l < 16; ++l) {
                const float d = x[j + l] - mean;
                lane[l] = fmaf(d, d, lane[l]);
            }
        float var = reduce16_add(lane);
        for (int j = nv; j < N; ++j) {
            const float d = x[j] - mean;
            var = fmaf(d, d, var);
        }
        var /= (float)N;
        const float inv_std = 1.0f / sqrtf(var + eps);
        for (int j = 0; j < N; ++j) y[j] = fmaf((x[j] - mean) * inv_std, gamma[j], beta[j]);
    }
}

/* fusedCrossEntropyLoss, reference FusedKernels.h:766-854 (AVX-512 branch):
 * grad = softmax(logits) - onehot(target), divided by M; returns the mean of
 * -log(p[target] + 1e-10).  The reference sums the row losses with an
 * OpenMP reduction (thread-dependent order); here they are summed in row
 * order. */
float jo_cross_entropy(const float* logits, const int32_t* targets, float* grad, int M, int N) {
    float* row_loss = (float*)malloc(sizeof(float) * (size_t)(M > 0 ? M : 1));
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; ++i) {
        float* g = grad + (int64_t)i * N;
        softmax_row(g, logits + (int64_t)i * N, N);
        const int t = targets[i];
        row_loss[i] = -logf(g[t] + 1e-10f);
        g[t] -= 1.0f;
        for (int j = 0; j < N; ++j) g[j] /= (float)M;
    }
    float total = 0.0f;
    for (int i = 0; i < M; ++i) total += row_loss[i];
    free(row_loss);
    return total / (float)M;
}

/* ---- fp64: textbook definitions ---- */
void jo64_softmax(double* out, const float* in, int M, int N) {
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; ++i) {
        const float* x = in + (int64_t)i * N;
        double* y = out + (int64_t)i * N;
        double mx = -INFINITY, s = 0.0;
        for (int j = 0; j < N; ++j) mx = x[j] > mx ? x[j] : mx;
        for (int j = 0; j < N; ++j) s += (y[j] = exp((double)x[j] - mx));
        for (int j = 0; j < N; ++j) y[j] /= s;
    }
}

void jo64_layernorm(double* out, const float* in, const float* gamma, const float* beta,
                    int M, int N, double eps) {
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; ++i) {
        const float* x = in + (int64_t)i * N;
        double* y = out + (int64_t)i * N;
        double mean = 0.0, var = 0.0;
        for (int j = 0; j < N; ++j) mean += x[j];
        mean /= N;
        for (int j = 0; j < N; ++j) var += ((double)x[j] - mean) * ((double)x[j] - mean);
        var /= N;
        const double r = 1.0 / sqrt(var + eps);
        for (int j = 0; j < N; ++j) y[j] = ((double)x[j] - mean) * r * gamma[j] + beta[j];
    }
}

double jo64_cross_entropy(const float* logits, const int32_t* targets, double* grad, int M,
                          int N) {
    double total = 0.0;
    jo64_softmax(grad, logits, M, N);
    for (int i = 0; i < M; ++i) {
        double* g = grad + (int64_t)i * N;
        total += -log(g[targets[i]] + 1e-10);
        g[targets[i]] -= 1.0;
        for (int j = 0; j < N; ++j) g[j] /= M;
    }
    return total / M;
}
