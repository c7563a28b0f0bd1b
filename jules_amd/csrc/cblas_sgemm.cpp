// cblas_sgemm.cpp - libjules_cblas.so: the CBLAS sgemm symbol on MI355X
// (include/jules_cblas.h), for callers that resolve cblas_sgemm at run time,
// such as the reference's ORC JIT (lib/LLVMBackend.cpp:1216-1255, resolved
// from the process's symbols at :1338-1356).  A thin host layer: argument
// checks, column-major to row-major, host buffers staged through dense device
// copies, then jules_hip_sgemm and a synchronisation, as a CPU BLAS call
// returns with C written.
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <utility>

#include "jules_cblas.h"
#include "jules_hip.h"

namespace {

thread_local int g_status = JH_OK;

bool is_device(const void* p) {
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeDevice;
}

// A row-major matrix of rows x cols floats with row stride ld as the GPU
// sees it: the caller's memory when it is device memory, else a dense device
// copy (row stride cols), copied in when `in`.
class Staged {
public:
    Staged(const float* p, int rows, int cols, int ld, bool in)
        : host_(const_cast<float*>(p)), rows_(rows), cols_(cols), host_ld_(ld) {
        if (!p || rows == 0 || cols == 0) return;
        if (is_device(p)) {
            dev_ = host_;
            ld_ = ld;
            return;
        }
        ld_ = cols;
        owned_ = true;
        const size_t row_bytes = sizeof(float) * (size_t)cols;
        void* d = nullptr;
        ok_ = hipMalloc(&d, row_bytes * rows) == hipSuccess;
        dev_ = static_cast<float*>(d);
        if (ok_ && in)
            ok_ = hipMemcpy2D(dev_, row_bytes, p, sizeof(float) * (size_t)ld, row_bytes, rows,
                              hipMemcpyHostToDevice) == hipSuccess;
    }
    ~Staged() {
        if (owned_ && dev_) (void)hipFree(dev_);
    }
    Staged(const Staged&) = delete;
    Staged& operator=(const Staged&) = delete;
    // write the rows x cols elements back to host memory (the rest of each
    // host row is left as it was)
    bool copy_out() {
        if (!owned_ || !ok_) return ok_;
        const size_t row_bytes = sizeof(float) * (size_t)cols_;
        return hipMemcpy2D(host_, sizeof(float) * (size_t)host_ld_, dev_, row_bytes, row_bytes, rows_,
                           hipMemcpyDeviceToHost) == hipSuccess;
    }
    bool ok() const { return ok_; }
    float* get() const { return dev_; }
    int ld() const { return ld_; }

private:
    float* host_;
    int rows_, cols_, host_ld_;
    float* dev_ = nullptr;
    int ld_ = 1;
    bool owned_ = false;
    bool ok_ = true;
};

int trans_code(int t) {
    if (t == JulesCblasNoTrans) return 0;
    if (t == JulesCblasTrans || t == JulesCblasConjTrans) return 1;
    return -1;
}

int imax1(int a) { return a > 1 ? a : 1; }

constexpr int64_t kMaxElems = int64_t(1) << 40;  // the element limit of libjules_hip

}  // namespace

extern "C" {

int jules_cblas_last_status(void) { return g_status; }

void cblas_sgemm(int Order, int TransA, int TransB, int M, int N, int K, float alpha,
                 const float* A, int lda, const float* B, int ldb, float beta, float* C, int ldc) {
    int ta = trans_code(TransA), tb = trans_code(TransB);
    if ((Order != JulesCblasRowMajor && Order != JulesCblasColMajor) || ta < 0 || tb < 0) {
        g_status = JH_ERR_ARG;
        return;
    }
    // column-major C = op(A) op(B) is row-major C^T = op(B)^T op(A)^T
    if (Order == JulesCblasColMajor) {
        std::swap(ta, tb);
        std::swap(M, N);
        std::swap(A, B);
        std::swap(lda, ldb);
    }
    // the reference BLAS's checks, before any staging
    const int a_rows = ta ? K : M, a_cols = ta ? M : K;
    const int b_rows = tb ? N : K, b_cols = tb ? K : N;
    if (M < 0 || N < 0 || K < 0 || lda < imax1(a_cols) || ldb < imax1(b_cols) || ldc < imax1(N) ||
        (int64_t)a_rows * lda > kMaxElems || (int64_t)b_rows * ldb > kMaxElems ||
        (int64_t)M * ldc > kMaxElems) {
        g_status = JH_ERR_SHAPE;
        return;
    }
    if (M == 0 || N == 0) {  // nothing to compute
        g_status = JH_OK;
        return;
    }
    if (!C || (K > 0 && alpha != 0.0f && (!A || !B))) {
        g_status = JH_ERR_NULL;
        return;
    }
    const bool product = K > 0 && alpha != 0.0f;
    Staged a(product ? A : nullptr, a_rows, a_cols, lda, true);
    Staged b(product ? B : nullptr, b_rows, b_cols, ldb, true);
    Staged c(C, M, N, ldc, beta != 0.0f);
    if (!a.ok() || !b.ok() || !c.ok()) {
        g_status = JH_ERR_HIP;
        return;
    }
    // without a product (K = 0 or alpha = 0) A and B are not read: no copies,
    // the caller's (already checked) leading dimensions
    int st = jules_hip_sgemm(ta, tb, M, N, K, alpha, a.get(), product ? a.ld() : lda, b.get(),
                             product ? b.ld() : ldb, beta, c.get(), c.ld(), nullptr);
    if (st == JH_OK && hipStreamSynchronize(nullptr) != hipSuccess) st = JH_ERR_HIP;
    if (st == JH_OK && !c.copy_out()) st = JH_ERR_HIP;
    g_status = st;
}

}  // extern "C"
