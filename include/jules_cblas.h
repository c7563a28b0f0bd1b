/*
 * jules_cblas.h - cblas_sgemm on MI355X, for code that resolves that symbol
 * at run time (libjules_cblas.so).
 *
 * The reference's LLVMBackend lowers a matmul to a call of
 *   cblas_sgemm(101, 111, 111, M, N, K, 1.0f, A, K, B, N, 0.0f, C, N)
 * on the host buffers held in its TensorDescriptors (lib/LLVMBackend.cpp:
 * 1216-1255), and its ORC JIT resolves cblas_sgemm from the symbols of the
 * host process (EPCDynamicLibrarySearchGenerator::GetForTargetProcess,
 * lib/LLVMBackend.cpp:1338-1356).  Loading libjules_cblas.so into the
 * process with global symbol visibility before the JIT links (dlopen with
 * RTLD_NOW | RTLD_GLOBAL, or linking the program against it) makes that call
 * run on the GPU, without changing the lowering.  libjules_hip.so itself
 * exports no cblas symbol, so loading it never interposes a BLAS for other
 * callers.
 *
 * Semantics: the CBLAS sgemm interface, C = alpha op(A) op(B) + beta C, with
 * row-major (101) or column-major (102) storage and NoTrans (111), Trans
 * (112) or ConjTrans (113, the same as Trans for real data).  Pointers may be
 * host memory (staged through the GPU, only the M x N elements of C are
 * written back) or device memory (used in place); the call returns when C
 * holds the result.  The dense row-major NoTrans/NoTrans alpha = 1,
 * beta = 0 call above computes every element as one fp32 fma chain over k in
 * order, the bits of the reference's tiledMatmulWithActivation
 * (include/jules/Kernel/FusedKernels.h:378-458); all other calls run an fp32
 * MFMA GEMM (jules_hip_sgemm, include/jules_hip.h).
 *
 * Errors: CBLAS returns nothing.  An invalid argument (the checks of the
 * reference BLAS: order and transpose codes JH_ERR_ARG, M/N/K >= 0 and the
 * leading dimensions JH_ERR_SHAPE, a NULL operand that is needed
 * JH_ERR_NULL) leaves C untouched and, like a HIP failure (JH_ERR_HIP), is
 * recorded as a jh_status readable with jules_cblas_last_status() on the
 * calling thread; nothing prints or aborts.
 */
#ifndef JULES_CBLAS_H
#define JULES_CBLAS_H

#ifdef __cplusplus
extern "C" {
#endif

enum JULES_CBLAS_ORDER { JulesCblasRowMajor = 101, JulesCblasColMajor = 102 };
enum JULES_CBLAS_TRANSPOSE {
    JulesCblasNoTrans = 111,
    JulesCblasTrans = 112,
    JulesCblasConjTrans = 113
};

/* The standard CBLAS signature (enums passed as int, as LLVMBackend.cpp:
 * 1219-1223 declares them). */
void cblas_sgemm(int Order, int TransA, int TransB, int M, int N, int K, float alpha,
                 const float* A, int lda, const float* B, int ldb, float beta, float* C,
                 int ldc);

/* jh_status of the last cblas_sgemm on this thread (0 = JH_OK). */
int jules_cblas_last_status(void);

#ifdef __cplusplus
}
#endif
#endif /* JULES_CBLAS_H */
