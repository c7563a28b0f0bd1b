// pjrt_selftest.cpp - exercises the C++ PJRT API of include/jules_hip_pjrt.hpp
// (client, device, buffers, executeAsync/events, executePipeline, custom_call,
// errors) on GPU 0; prints "pjrt selftest ok" and exits 0 when every check
// holds.  Built by jules_amd/build.py, run by tests/test_gpu_pjrt.py.
#include <cmath>
#include <cstdio>
#include <vector>

#include "jules_hip_pjrt.hpp"

using jules_hip::PJRTClient;
using jules_hip::PJRTError;

#define CHECK(c)                                                          \
    do {                                                                  \
        if (!(c)) {                                                       \
            std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #c);       \
            return 1;                                                     \
        }                                                                 \
    } while (0)

int main() {
    try {
        auto client = PJRTClient::create("rocm");
        CHECK(client->platform() == "rocm");
        CHECK(client->deviceCount() >= 1);
        auto* dev = client->getDefaultDevice();
        CHECK(dev == client->getDevice(0) && client->getDevice(client->deviceCount()) == nullptr);
        CHECK(dev->kind() == "ROCM_GPU" && dev->vendor() == "AMD" && dev->availableMemory() > 0);

        // buffer round trip
        std::vector<float> x(1000);
        for (int i = 0; i < 1000; ++i) x[i] = 0.25f * (float)i - 7.0f;
        auto b = client->allocateBuffer({10, 100}, JH_F32);
        CHECK(b->size() == 4000 && !b->isHostBuffer() && b->deviceId() == dev->id());
        CHECK((b->shape() == std::vector<int64_t>{10, 100}) && b->elementType() == JH_F32);
        b->copyFromHost(x.data(), 4000);
        std::vector<float> back(1000);
        b->copyToHost(back.data(), 4000);
        CHECK(back == x);

        // executeAsync + event
        auto twice = client->compileAndLoad("%0 = \"stablehlo.add\"(%arg0, %arg0) : () -> ()");
        CHECK(twice->name() == "rocm_executable");
        auto r = twice->executeAsync({b});
        r.second->await();
        CHECK(r.second->isReady() && r.first.size() == 1);
        std::vector<float> y(1000);
        r.first[0]->copyToHost(y.data(), 4000);
        for (int i = 0; i < 1000; ++i) CHECK(y[i] == x[i] + x[i]);

        // pipeline: stage 2 consumes stage 1's outputs
        auto square = client->compileAndLoad("%0 = \"stablehlo.multiply\"(%arg0, %arg0) : () -> ()");
        auto out = client->executePipeline({twice.get(), square.get(), twice.get()}, {b});
        CHECK(out.size() == 1);
        std::vector<float> z(1000);
        out[0]->copyToHost(z.data(), 4000);
        for (int i = 0; i < 1000; ++i) {
            const float t = x[i] + x[i];
            const float sq = t * t;
            CHECK(z[i] == sq + sq);
        }
        client->synchronizeAll();

        // custom_call through the registry: fusedSoftmax rows sum to 1
        auto sm = dev->loadExecutable(
            "%0 = \"stablehlo.custom_call\"(%arg0) {call_target_name = \"fusedSoftmax\"} : "
            "(tensor<10x100xf32>) -> tensor<10x100xf32>");
        auto so = sm->execute({b});
        CHECK(so.size() == 1 && (so[0]->shape() == std::vector<int64_t>{10, 100}));
        std::vector<float> p(1000);
        so[0]->copyToHost(p.data(), 4000);
        for (int row = 0; row < 10; ++row) {
            double s = 0.0;
            for (int j = 0; j < 100; ++j) s += p[row * 100 + j];
            CHECK(std::fabs(s - 1.0) < 1e-5);
        }

        // a non-owning view of caller memory as an input
        auto view = jules_hip::wrapDeviceMemory(b->rawPointer(), {1000}, JH_F32, dev->id());
        auto vo = twice->execute({view});
        std::vector<float> w(1000);
        vo[0]->copyToHost(w.data(), 4000);
        CHECK(w == y);

        // errors
        try {
            PJRTClient::create("tpu");
            CHECK(false);
        } catch (const PJRTError& e) {
            CHECK(e.status() == JH_ERR_UNSUPPORTED);
        }
        auto bad = client->compileAndLoad(
            "%0 = \"stablehlo.custom_call\"(%arg0) {call_target_name = \"nope\"} : (tensor<1000xf32>) -> tensor<1000xf32>");
        try {
            bad->execute({view});
            CHECK(false);
        } catch (const PJRTError& e) {
            CHECK(e.status() == JH_ERR_NOT_FOUND);
        }
        try {
            b->copyToHost(back.data(), 4004);
            CHECK(false);
        } catch (const PJRTError& e) {
            CHECK(e.status() == JH_ERR_SHAPE);
        }
        std::printf("pjrt selftest ok\n");
        return 0;
    } catch (const std::exception& e) {
        std::printf("FAIL exception: %s\n", e.what());
        return 1;
    }
}
