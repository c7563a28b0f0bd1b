// kernel_selftest.cpp - exercises the jules::kernel C++ entry points of
// include/jules_hip_kernel.hpp with host buffers (staged to and from the GPU
// by the library) on GPU 0: interleavedMLPForwardBackward and
// fusedMLPForward against a double-precision loop restatement of the same
// formulas.  Prints
// "kernel selftest ok" and exits 0 when every check holds.  Built by
// jules_amd/build.py, run by tests/test_gpu_mlp.py.
#include <cmath>
#include <cstdio>
#include <vector>

#include "jules_hip_kernel.hpp"

using namespace jules::kernel;

#define CHECK(c)                                                          \
    do {                                                                  \
        if (!(c)) {                                                       \
            std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #c);       \
            return 1;                                                     \
        }                                                                 \
    } while (0)

static double max_rel(const std::vector<float>& y, const std::vector<double>& r) {
    double num = 0, den = 0;
    for (size_t i = 0; i < y.size(); ++i) {
        num = std::fmax(num, std::fabs((double)y[i] - r[i]));
        den = std::fmax(den, std::fabs(r[i]));
    }
    return den > 0 ? num / den : num;
}

int main() {
    const int M = 19, K1 = 23, N1 = 17, N2 = 5;
    unsigned s = 12345u;
    auto rnd = [&]() {
        s = s * 1664525u + 1013904223u;
        return ((int)(s >> 9) % 2001 - 1000) / 1000.0f;
    };
    std::vector<float> X(M * K1), W1(K1 * N1), b1(N1), W2(N1 * N2), b2(N2);
    for (auto* v : {&X, &W1, &b1, &W2, &b2})
        for (auto& e : *v) e = rnd();
    std::vector<int32_t> t(M);
    for (int i = 0; i < M; ++i) t[i] = (i * 7 + 3) % N2;

    // double-precision restatement (InterleavedAutodiff.h:144-267)
    std::vector<double> h(M * N1), a(M * N1), o(M * N2), dO(M * N2), dH(M * N1);
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N1; ++j) {
            double acc = b1[j];
            for (int k = 0; k < K1; ++k) acc += (double)X[i * K1 + k] * W1[k * N1 + j];
            h[i * N1 + j] = acc;
            a[i * N1 + j] = acc > 0 ? acc : 0;
        }
    double loss = 0;
    for (int i = 0; i < M; ++i) {
        double mx = -1e300, sum = 0;
        for (int j = 0; j < N2; ++j) {
            double acc = b2[j];
            for (int k = 0; k < N1; ++k) acc += a[i * N1 + k] * W2[k * N2 + j];
            o[i * N2 + j] = acc;
            mx = std::fmax(mx, acc);
        }
        for (int j = 0; j < N2; ++j) sum += std::exp(o[i * N2 + j] - mx);
        for (int j = 0; j < N2; ++j) dO[i * N2 + j] = std::exp(o[i * N2 + j] - mx) / sum;
        loss -= std::log(dO[i * N2 + t[i]] + 1e-10);
        dO[i * N2 + t[i]] -= 1;
        for (int j = 0; j < N2; ++j) dO[i * N2 + j] /= M;
    }
    loss /= M;
    std::vector<double> rdW2(N1 * N2, 0), rdb2(N2, 0), rdW1(K1 * N1, 0), rdb1(N1, 0), rdX(M * K1, 0);
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N1; ++j) {
            double acc = 0;
            for (int k = 0; k < N2; ++k) acc += dO[i * N2 + k] * W2[j * N2 + k];
            dH[i * N1 + j] = h[i * N1 + j] > 0 ? acc : 0;
        }
    for (int i = 0; i < M; ++i) {
        for (int k = 0; k < N1; ++k)
            for (int j = 0; j < N2; ++j) rdW2[k * N2 + j] += a[i * N1 + k] * dO[i * N2 + j];
        for (int j = 0; j < N2; ++j) rdb2[j] += dO[i * N2 + j];
        for (int k = 0; k < K1; ++k)
            for (int j = 0; j < N1; ++j) rdW1[k * N1 + j] += (double)X[i * K1 + k] * dH[i * N1 + j];
        for (int j = 0; j < N1; ++j) rdb1[j] += dH[i * N1 + j];
        for (int k = 0; k < K1; ++k)
            for (int j = 0; j < N1; ++j) rdX[i * K1 + k] += dH[i * N1 + j] * W1[k * N1 + j];
    }

    std::vector<float> out(M * N2), dW1(K1 * N1), db1(N1), dW2(N1 * N2), db2(N2), dX(M * K1);
    ExecutionArena arena;
    TilePlanner planner;
    InterleavedMLPResult r = interleavedMLPForwardBackward(
        X.data(), W1.data(), b1.data(), W2.data(), b2.data(), t.data(), out.data(), dW1.data(),
        db1.data(), dW2.data(), db2.data(), dX.data(), M, K1, N1, N2, arena, planner);
    CHECK(lastStatus() == JH_OK);
    CHECK(r.grads.dW1 == dW1.data() && r.grads.dX == dX.data());
    CHECK(std::fabs(r.loss - loss) <= 1e-5 * std::fabs(loss));
    CHECK(max_rel(out, o) < 1e-5);
    CHECK(max_rel(dW1, rdW1) < 1e-5);
    CHECK(max_rel(db1, rdb1) < 1e-5);
    CHECK(max_rel(dW2, rdW2) < 1e-5);
    CHECK(max_rel(db2, rdb2) < 1e-5);
    CHECK(max_rel(dX, rdX) < 1e-5);

    // without dX, and a shape error
    r = interleavedMLPForwardBackward(X.data(), W1.data(), b1.data(), W2.data(), b2.data(), t.data(),
                                      out.data(), dW1.data(), db1.data(), dW2.data(), db2.data(),
                                      nullptr, M, K1, N1, N2, arena, planner);
    CHECK(lastStatus() == JH_OK && std::fabs(r.loss - loss) <= 1e-5 * std::fabs(loss));
    r = interleavedMLPForwardBackward(X.data(), W1.data(), b1.data(), W2.data(), b2.data(), t.data(),
                                      out.data(), dW1.data(), db1.data(), dW2.data(), db2.data(),
                                      nullptr, M, K1, 0, N2, arena, planner);
    CHECK(lastStatus() == JH_ERR_SHAPE && std::isnan(r.loss));

    // fusedMLPForward (FusedKernels.h:659): the same forward, no loss
    std::vector<float> fwd(M * N2, -7.0f);
    const MLPParams p{W1.data(), b1.data(), W2.data(), b2.data(), M, K1, N1, N2};
    fusedMLPForward(fwd.data(), X.data(), p, arena, planner);
    CHECK(lastStatus() == JH_OK);
    CHECK(max_rel(fwd, o) < 1e-5);
    const MLPParams bad{W1.data(), b1.data(), W2.data(), b2.data(), M, 0, N1, N2};
    fusedMLPForward(fwd.data(), X.data(), bad, arena, planner);
    CHECK(lastStatus() == JH_ERR_SHAPE);
    std::printf("kernel selftest ok\n");
    return 0;
}
