// test_backend_hip.cpp — C++ test of the "hip" backend through the plugin
// interface, in the shape of the reference's tests/test_backend_cuda.cpp:12-76
// (registry, H2D/D2H round trip, RMSNorm against a scalar reference) plus the
// quantized MATMUL path and the error behaviour of the registry
// (tests/test_backend_x86.cpp:25-29).  Exit code 0 = all checks passed.
//
// Built twice: against this tree's restatement of the interface
// (axf_backend.hpp), and with AXF_AXONFORGE_HEADERS against the reference's
// own headers, registry and Tensor (tests/cpp/build_dropin.py), linked with the
// plugin compiled in its drop-in mode.  `--no-device` checks what holds on a
// host without a GPU: the backend is registered, initialize() reports no
// device, and device work throws std::runtime_error.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#if defined(AXF_AXONFORGE_HEADERS)
#include "axonforge/backend.hpp"
using namespace axonforge;
#else
#include "axf_backend.hpp"
using namespace axf;
#endif
#include "axf_hip.h"

static int g_fail = 0;
#define REQUIRE(cond)                                                        \
    do {                                                                     \
        if (!(cond)) {                                                       \
            std::printf("FAILED %s:%d: %s\n", __FILE__, __LINE__, #cond);    \
            g_fail++;                                                        \
        }                                                                    \
    } while (0)

static bool within_rel(float a, float b, float rel) {
    return std::fabs(a - b) <= rel * std::fmax(std::fabs(a), std::fabs(b));
}

static void test_registry_and_transfer() {
    auto& reg = BackendRegistry::instance();
    REQUIRE(reg.has_backend("hip"));
    bool threw = false;
    try {
        (void)reg.create("no_such_backend");
    } catch (const std::runtime_error&) {
        threw = true;
    }
    REQUIRE(threw);

    auto b = reg.create("hip");
    REQUIRE(b->initialize());
    REQUIRE(b->device_id().type == DeviceType::HIP);
    auto h = Tensor::zeros({4}, DType::F32);
    auto hd = h.data_as<float>();
    for (int i = 0; i < 4; ++i) hd[i] = static_cast<float>(i + 1);
    auto d = Tensor::from_storage(b->allocate(h.nbytes(), 256), {4}, DType::F32);
    b->transfer(h, d);
    auto out = Tensor::zeros({4}, DType::F32);
    b->transfer(d, out);
    auto od = out.data_as<float>();
    for (int i = 0; i < 4; ++i) REQUIRE(od[i] == hd[i]);
    b->finalize();
    std::printf("registry/transfer: done\n");
}

static void test_rmsnorm() {
    auto b = BackendRegistry::instance().create("hip");
    REQUIRE(b->initialize());
    constexpr int N = 64;
    auto xh = Tensor::zeros({N}, DType::F32), wh = Tensor::zeros({N}, DType::F32);
    auto yh = Tensor::zeros({N}, DType::F32);
    auto xd = xh.data_as<float>();
    auto wd = wh.data_as<float>();
    for (int i = 0; i < N; ++i) {
        xd[i] = static_cast<float>(i % 8 + 1);
        wd[i] = 1.0f + 0.1f * static_cast<float>(i % 8);
    }
    auto x = Tensor::from_storage(b->allocate(xh.nbytes(), 256), {N}, DType::F32);
    auto w = Tensor::from_storage(b->allocate(wh.nbytes(), 256), {N}, DType::F32);
    auto y = Tensor::from_storage(b->allocate(yh.nbytes(), 256), {N}, DType::F32);
    b->transfer(xh, x);
    b->transfer(wh, w);
    std::vector<DType> dtypes = {DType::F32, DType::F32};
    AttributeMap attrs;
    attrs.set("eps", 1e-5f);
    auto k = b->get_kernel(OpType::RMS_NORM, dtypes, attrs);
    std::vector<Tensor> inputs = {x, w};
    std::vector<Tensor> outputs = {y};
    k->execute(inputs, outputs, attrs);
    b->synchronize();
    b->transfer(y, yh);
    // x cycles 1..8: mean(x^2) = 204/8 (tests/test_backend_x86.cpp:84-116 closed form)
    const float inv = 1.0f / std::sqrt(204.f / 8.f + 1e-5f);
    auto yd = yh.data_as<float>();
    for (int i = 0; i < N; ++i) REQUIRE(within_rel(yd[i], xd[i] * inv * wd[i], 1e-5f));
    b->finalize();
    std::printf("rmsnorm: done\n");
}

static void test_matmul_q4k() {
    auto b = BackendRegistry::instance().create("hip");
    REQUIRE(b->initialize());
    const int rows = 64, cols = 512;
    const size_t rb = axf_row_bytes(AXF_TYPE_Q4_K, cols);
    std::vector<uint8_t> wq(rows * rb);
    REQUIRE(axf_synth_weight(AXF_TYPE_Q4_K, wq.data(), rows, cols, 7, 0.02f) == AXF_OK);
    std::vector<float> xv(cols), wf((size_t)rows * cols);
    REQUIRE(axf_synth_normal(xv.data(), cols, 8, 0.f, 1.f) == AXF_OK);
    // scalar reference from the device dequant of the same bytes
    // block-quantized host data carries its real size (from_raw_blob, as the
    // reference's GGUF tensors)
    auto wh = Tensor::from_raw_blob(wq.data(), wq.size(), {rows, cols}, DType::Q4_K_M);
    auto xh = Tensor::from_blob(xv.data(), {cols}, DType::F32);
    auto W = Tensor::from_storage(b->allocate(wq.size(), 256), {rows, cols}, DType::Q4_K_M);
    auto X = Tensor::from_storage(b->allocate(xh.nbytes(), 256), {cols}, DType::F32);
    auto Y = Tensor::from_storage(b->allocate((size_t)rows * 4, 256), {rows}, DType::F32);
    auto WF = Tensor::from_storage(b->allocate(wf.size() * 4, 256), {rows * cols}, DType::F32);
    b->transfer(wh, W);
    b->transfer(xh, X);
    std::vector<DType> dt = {DType::Q4_K_M, DType::F32};
    AttributeMap attrs;
    auto k = b->get_kernel(OpType::MATMUL, dt, attrs);
    std::vector<Tensor> in = {W, X};
    std::vector<Tensor> out = {Y};
    k->execute(in, out, attrs);
    b->synchronize();
    auto yh = Tensor::zeros({rows}, DType::F32);
    b->transfer(Y, yh);
    // dequantised weights through the C-ABI, then a double-precision dot
    axf_ctx* ctx = nullptr;
    REQUIRE(axf_hip_create(0, &ctx) == AXF_OK);
    void* dW = nullptr;
    void* dF = nullptr;
    REQUIRE(axf_hip_alloc(ctx, wq.size(), &dW) == AXF_OK);
    REQUIRE(axf_hip_alloc(ctx, wf.size() * 4, &dF) == AXF_OK);
    REQUIRE(axf_hip_memcpy_h2d(ctx, dW, wq.data(), wq.size()) == AXF_OK);
    REQUIRE(axf_hip_dequant_q4k(ctx, (float*)dF, dW, (int64_t)rows * cols / 256) == AXF_OK);
    REQUIRE(axf_hip_memcpy_d2h(ctx, wf.data(), dF, wf.size() * 4) == AXF_OK);
    axf_hip_free(ctx, dW);
    axf_hip_free(ctx, dF);
    axf_hip_destroy(ctx);
    auto yd = yh.data_as<float>();
    for (int r = 0; r < rows; r++) {
        double acc = 0;
        for (int c = 0; c < cols; c++) acc += (double)wf[(size_t)r * cols + c] * xv[c];
        REQUIRE(std::fabs(yd[r] - acc) <= 1e-4 + 1e-3 * std::fabs(acc));
    }
    // unsupported combination throws
    bool threw = false;
    try {
        std::vector<DType> bad = {DType::F16, DType::F32};
        (void)b->get_kernel(OpType::MATMUL, bad, attrs);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    REQUIRE(threw);
    b->finalize();
    std::printf("matmul q4k: done\n");
}

static void test_no_device() {
    auto& reg = BackendRegistry::instance();
    REQUIRE(reg.has_backend("hip"));
    bool listed = false;
    for (const auto& id : reg.available_backends()) listed = listed || id == "hip";
    REQUIRE(listed);
    bool threw = false;
    try {
        (void)reg.create("no_such_backend");
    } catch (const std::runtime_error&) {
        threw = true;
    }
    REQUIRE(threw);
    auto b = reg.create("hip");
    REQUIRE(b->name() == "hip");
    REQUIRE(b->device_id().type == DeviceType::HIP);
    bool init = true;
    try {
        init = b->initialize();
    } catch (const std::runtime_error&) {
        init = false;
    }
    REQUIRE(!init);
    threw = false;
    try {
        (void)b->allocate(256, 256);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    REQUIRE(threw);
    threw = false;
    try {
        std::vector<DType> dt = {DType::Q4_K_M, DType::F32};
        (void)b->get_kernel(OpType::MATMUL, dt, AttributeMap{});
    } catch (const std::runtime_error&) {
        threw = true;
    }
    REQUIRE(threw);
    std::printf("no device: done\n");
}

int main(int argc, char** argv) {
    if (argc > 1 && std::strcmp(argv[1], "--no-device") == 0) {
        try {
            test_no_device();
        } catch (const std::exception& e) {
            std::printf("EXCEPTION: %s\n", e.what());
            return 2;
        }
        std::printf("%s (%d failures)\n", g_fail ? "FAILED" : "PASSED", g_fail);
        return g_fail ? 1 : 0;
    }
    try {
        test_registry_and_transfer();
        test_rmsnorm();
        test_matmul_q4k();
    } catch (const std::exception& e) {
        std::printf("EXCEPTION: %s\n", e.what());
        return 2;
    }
    std::printf("%s (%d failures)\n", g_fail ? "FAILED" : "PASSED", g_fail);
    return g_fail ? 1 : 0;
}
