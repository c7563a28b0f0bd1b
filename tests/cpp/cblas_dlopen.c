/* cblas_dlopen.c - binds cblas_sgemm the way a JIT's process-symbol lookup
 * does: no link-time dependency, dlopen(RTLD_NOW | RTLD_GLOBAL) of
 * libjules_cblas.so, then dlsym of the CBLAS name (the reference's ORC JIT
 * resolves it from the process, lib/LLVMBackend.cpp:1338-1356).
 *
 * Usage: cblas_dlopen LIB [--gpu]
 *   always: the symbols resolve, and invalid calls (bad order or transpose
 *     code, negative sizes, short leading dimensions, NULL operands) record
 *     their status without touching C or the GPU;
 *   --gpu: also the call LLVMBackend emits (LLVMBackend.cpp:1242-1255),
 *     cblas_sgemm(101, 111, 111, M, N, K, 1, A, K, B, N, 0, C, N), on host
 *     buffers, checked against a double-precision loop.
 * Prints "cblas dlopen ok" and exits 0 when every check holds. */
#define _GNU_SOURCE /* RTLD_DEFAULT */
#include <dlfcn.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef void (*sgemm_fn)(int, int, int, int, int, int, float, const float*, int, const float*,
                         int, float, float*, int);
typedef int (*status_fn)(void);

static int fails = 0;
#define CHECK(c)                                                    \
    do {                                                            \
        if (!(c)) {                                                 \
            printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #c);      \
            ++fails;                                                \
        }                                                           \
    } while (0)

int main(int argc, char** argv) {
    if (argc < 2) {
        printf("usage: cblas_dlopen LIB [--gpu]\n");
        return 2;
    }
    void* h = dlopen(argv[1], RTLD_NOW | RTLD_GLOBAL);
    if (!h) {
        printf("FAIL dlopen: %s\n", dlerror());
        return 1;
    }
    sgemm_fn sgemm = (sgemm_fn)dlsym(RTLD_DEFAULT, "cblas_sgemm");  /* process-wide lookup */
    status_fn status = (status_fn)dlsym(h, "jules_cblas_last_status");
    CHECK(sgemm != NULL && status != NULL);
    if (!sgemm || !status) return 1;

    float c[4] = {7, 7, 7, 7};
    const float a[4] = {1, 2, 3, 4}, b[4] = {5, 6, 7, 8};
    /* argument errors: status recorded, C untouched, no device work */
    sgemm(103, 111, 111, 2, 2, 2, 1.0f, a, 2, b, 2, 0.0f, c, 2);
    CHECK(status() == 10);                      /* JH_ERR_ARG: order */
    sgemm(101, 114, 111, 2, 2, 2, 1.0f, a, 2, b, 2, 0.0f, c, 2);
    CHECK(status() == 10);                      /* transpose code */
    sgemm(101, 111, 111, -1, 2, 2, 1.0f, a, 2, b, 2, 0.0f, c, 2);
    CHECK(status() == 2);                       /* JH_ERR_SHAPE: M < 0 */
    sgemm(101, 111, 111, 2, 2, 3, 1.0f, a, 2, b, 2, 0.0f, c, 2);
    CHECK(status() == 2);                       /* lda = 2 < K = 3 */
    sgemm(101, 112, 111, 3, 2, 2, 1.0f, a, 2, b, 2, 0.0f, c, 2);
    CHECK(status() == 2);                       /* transposed A: lda = 2 < M = 3 */
    sgemm(102, 111, 111, 2, 2, 2, 1.0f, a, 1, b, 2, 0.0f, c, 2);
    CHECK(status() == 2);                       /* column-major: lda = 1 < M = 2 */
    sgemm(101, 111, 111, 2, 2, 2, 1.0f, NULL, 2, b, 2, 0.0f, c, 2);
    CHECK(status() == 1);                       /* JH_ERR_NULL */
    sgemm(101, 111, 111, 2, 2, 2, 1.0f, a, 2, b, 2, 0.0f, NULL, 2);
    CHECK(status() == 1);
    sgemm(101, 111, 111, 0, 2, 2, 1.0f, NULL, 2, NULL, 2, 0.0f, NULL, 2);
    CHECK(status() == 0);                       /* M = 0: nothing to do */
    for (int i = 0; i < 4; ++i) CHECK(c[i] == 7.0f);

    if (argc > 2 && strcmp(argv[2], "--gpu") == 0) {
        const int M = 33, N = 48, K = 70;
        float* A = malloc(sizeof(float) * M * K);
        float* B = malloc(sizeof(float) * K * N);
        float* C = malloc(sizeof(float) * M * N);
        unsigned s = 1u;
        for (int i = 0; i < M * K; ++i) A[i] = (float)((s = s * 1664525u + 1013904223u) >> 8) / 16777216.0f - 0.5f;
        for (int i = 0; i < K * N; ++i) B[i] = (float)((s = s * 1664525u + 1013904223u) >> 8) / 16777216.0f - 0.5f;
        sgemm(101, 111, 111, M, N, K, 1.0f, A, K, B, N, 0.0f, C, N);
        CHECK(status() == 0);
        double err = 0, mx = 0;
        for (int i = 0; i < M; ++i)
            for (int j = 0; j < N; ++j) {
                double r = 0;
                for (int k = 0; k < K; ++k) r += (double)A[i * K + k] * B[k * N + j];
                err = fmax(err, fabs(r - C[i * N + j]));
                mx = fmax(mx, fabs(r));
            }
        CHECK(err <= 1e-5 * mx);
        free(A);
        free(B);
        free(C);
    }
    if (fails) {
        printf("%d failures\n", fails);
        return 1;
    }
    printf("cblas dlopen ok\n");
    return 0;
}
