// hip_backend.cpp — the "hip" IBackend: device storage, synchronous transfer,
// and IKernel::execute for the ops of the quantized decode path, registered
// before main like the reference's backends (x86_backend.cpp:135-146,
// cuda_backend.cu:219-225).  Kernel launches go through the C-ABI
// (include/axf_hip.h); a non-zero status becomes std::runtime_error, as
// check_cuda does in the reference (cuda_backend.cu:15-25).
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <stdexcept>
#include <utility>

#include "../capi_internal.hpp"

// Interface switch.  In this tree the plugin interface comes from
// axf_backend.hpp (namespace axf).  Built inside the reference tree, define
// AXF_AXONFORGE_HEADERS: the interface then comes from its own
// include/axonforge/backend.hpp (namespace axonforge, DeviceType::HIP added
// to its common.hpp), and the core types below (Tensor, storage,
// BackendRegistry) are the reference's own definitions.
#if defined(AXF_AXONFORGE_HEADERS)
#include "axonforge/backend.hpp"
namespace axf_api = axonforge;
#else
#include "axf_backend.hpp"
namespace axf_api = axf;
#endif

namespace axf {

using namespace axf_api;

#if !defined(AXF_AXONFORGE_HEADERS)
// ---- core types ----------------------------------------------------------

CpuTensorStorage::CpuTensorStorage(size_t bytes) : bytes_(bytes) {
    if (bytes_) {
        ptr_ = std::aligned_alloc(64, (bytes_ + 63) / 64 * 64);
        if (!ptr_) throw std::bad_alloc();
        std::memset(ptr_, 0, bytes_);
    }
}
CpuTensorStorage::CpuTensorStorage(void* external, size_t bytes)
    : ptr_(external), bytes_(bytes), owns_(false) {}
CpuTensorStorage::~CpuTensorStorage() {
    if (owns_) std::free(ptr_);
}

int64_t Tensor::numel() const noexcept {
    if (shape_.empty()) return storage_ ? 1 : 0;
    int64_t n = 1;
    for (auto d : shape_) n *= d;
    return n;
}

Tensor Tensor::zeros(Shape shape, DType dtype) {
    Tensor t;
    t.shape_ = std::move(shape);
    t.dtype_ = dtype;
    t.storage_ = std::make_shared<CpuTensorStorage>(t.nbytes());
    return t;
}

Tensor Tensor::from_blob(void* data, Shape shape, DType dtype) {
    Tensor t;
    t.shape_ = std::move(shape);
    t.dtype_ = dtype;
    t.storage_ = std::make_shared<CpuTensorStorage>(data, t.nbytes());
    return t;
}

Tensor Tensor::from_raw_blob(void* data, size_t nbytes, Shape shape, DType dtype) {
    Tensor t;
    t.shape_ = std::move(shape);
    t.dtype_ = dtype;
    t.storage_ = std::make_shared<CpuTensorStorage>(data, nbytes);
    return t;
}

Tensor Tensor::from_storage(std::shared_ptr<TensorStorage> storage, Shape shape, DType dtype) {
    Tensor t;
    t.storage_ = std::move(storage);
    t.shape_ = std::move(shape);
    t.dtype_ = dtype;
    return t;
}

BackendRegistry& BackendRegistry::instance() {
    static BackendRegistry registry;
    return registry;
}

void BackendRegistry::register_backend(std::string_view id, FactoryFn factory) {
    factories_.insert_or_assign(std::string(id), std::move(factory));
}

std::unique_ptr<IBackend> BackendRegistry::create(std::string_view id) const {
    auto it = factories_.find(std::string(id));
    if (it == factories_.end())
        throw std::runtime_error("BackendRegistry: no backend registered with id '" +
                                 std::string(id) + "'");
    return it->second();
}

bool BackendRegistry::has_backend(std::string_view id) const noexcept {
    return factories_.count(std::string(id)) > 0;
}

std::vector<std::string> BackendRegistry::available_backends() const {
    std::vector<std::string> ids;
    for (const auto& kv : factories_) ids.push_back(kv.first);
    return ids;
}
#endif  // !AXF_AXONFORGE_HEADERS

// ---- HIP backend ---------------------------------------------------------

namespace {

void check(int rc, const char* where) {
    if (rc != AXF_OK)
        throw std::runtime_error(std::string(where) + ": " + axf_hip_last_error());
}

class HipTensorStorage final : public TensorStorage {
public:
    HipTensorStorage(axf_ctx* ctx, size_t bytes) : ctx_(ctx), bytes_(bytes) {
        check(axf_hip_alloc(ctx_, bytes_, &ptr_), "HipTensorStorage");
    }
    ~HipTensorStorage() override {
        if (ptr_) axf_hip_free(ctx_, ptr_);
    }
    HipTensorStorage(const HipTensorStorage&) = delete;
    HipTensorStorage& operator=(const HipTensorStorage&) = delete;
    void* data() noexcept override { return ptr_; }
    const void* data() const noexcept override { return ptr_; }
    size_t byte_size() const noexcept override { return bytes_; }
    DeviceId device() const noexcept override { return DeviceId{DeviceType::HIP, ctx_->device}; }

private:
    axf_ctx* ctx_;
    void* ptr_{nullptr};
    size_t bytes_{0};
};

struct RopeTable {
    float* cos_t = nullptr;
    float* sin_t = nullptr;
    int max_pos = 0;
};

class HipKernel final : public IKernel {
public:
    HipKernel(OpType op, axf_ctx* ctx, std::map<std::pair<int, float>, RopeTable>* ropes)
        : op_(op), ctx_(ctx), ropes_(ropes) {}

    void execute(std::span<const Tensor> inputs, std::span<Tensor> outputs,
                 const AttributeMap& attrs) override {
        if (outputs.empty()) throw std::runtime_error("HipKernel::execute: no output tensor");
        float* out = static_cast<float*>(outputs[0].raw_data());
        switch (op_) {
            case OpType::RMS_NORM: {
                if (inputs.size() < 2) throw std::runtime_error("HIP RMS_NORM requires x and weight");
                const int n = static_cast<int>(inputs[0].numel());
                const float eps = attrs.get_or<float>("eps", 1e-5f);
                void* q8 = outputs.size() > 1 ? outputs[1].raw_data() : nullptr;
                check(axf_hip_rmsnorm(ctx_, out, q8, f32(inputs[0]), f32(inputs[1]), n, eps),
                      "HIP RMS_NORM");
                break;
            }
            case OpType::SILU: {
                if (inputs.empty()) throw std::runtime_error("HIP SILU requires input");
                const int n = static_cast<int>(inputs[0].numel());
                check(launch_or_fail(launch_silu(out, f32(inputs[0]), n, ctx_->stream)), "HIP SILU");
                break;
            }
            case OpType::MUL:
            case OpType::ADD: {
                if (inputs.size() < 2) throw std::runtime_error("HIP MUL/ADD requires two inputs");
                const int n = static_cast<int>(outputs[0].numel());
                if (op_ == OpType::MUL)
                    check(launch_or_fail(launch_mul(out, f32(inputs[0]), f32(inputs[1]), n,
                                                    ctx_->stream)),
                          "HIP MUL");
                else
                    check(axf_hip_add(ctx_, out, f32(inputs[0]), f32(inputs[1]), n), "HIP ADD");
                break;
            }
            case OpType::ROPE: {
                if (inputs.empty()) throw std::runtime_error("HIP ROPE requires input/output alias tensor");
                const int n_heads = static_cast<int>(attrs.get_or<int64_t>("n_heads", 0));
                const int head_dim = static_cast<int>(attrs.get_or<int64_t>("head_dim", 0));
                const int pos = static_cast<int>(attrs.get_or<int64_t>("pos", 0));
                const float theta = attrs.get_or<float>("theta", 10000.0f);
                if (n_heads <= 0 || head_dim <= 0 || head_dim % 2 || pos < 0)
                    throw std::runtime_error("HIP ROPE: bad n_heads/head_dim/pos");
                const RopeTable& t = table(head_dim, theta, pos + 1);
                check(axf_hip_rope(ctx_, out, f32(inputs[0]), pos, n_heads, head_dim, t.cos_t,
                                   t.sin_t),
                      "HIP ROPE");
                break;
            }
            case OpType::MATMUL: {
                if (inputs.size() < 2) throw std::runtime_error("HIP MATMUL requires weight and x");
                matmul(inputs[0], inputs[1], outputs[0], attrs);
                break;
            }
            case OpType::EMBEDDING_LOOKUP: {
                if (inputs.empty()) throw std::runtime_error("HIP EMBEDDING_LOOKUP requires weight");
                const int token = static_cast<int>(attrs.get_or<int64_t>("token", 0));
                const int cols = static_cast<int>(outputs[0].numel());
                const int rows = inputs[0].shape().empty()
                                     ? 0
                                     : static_cast<int>(inputs[0].numel() / cols);
                check(axf_hip_embed(ctx_, out, qtype(inputs[0].dtype()), inputs[0].raw_data(),
                                    token, rows, cols),
                      "HIP EMBEDDING_LOOKUP");
                break;
            }
            default:
                throw std::runtime_error("HipKernel::execute: unsupported op");
        }
    }

private:
    static const float* f32(const Tensor& t) { return static_cast<const float*>(t.raw_data()); }

    static int qtype(DType d) {
        if (d == DType::Q4_K_M) return AXF_TYPE_Q4_K;
        if (d == DType::Q6_K) return AXF_TYPE_Q6_K;
        throw std::runtime_error("HIP: weight dtype must be Q4_K_M or Q6_K");
    }

    static int launch_or_fail(hipError_t e) {
        return e == hipSuccess ? AXF_OK : hip_fail(e, "launch");
    }

    // MATMUL conventions of the reference CUDA backend (cuda_backend.cu:98-111):
    // inputs[0] weight, inputs[1] activation, outputs[0] y, rows = y.numel(),
    // cols = x.numel(), attribute "row_bytes".  Extensions: Q6_K weights, Q8_0
    // activations, "accumulate" (y += W x), and 2-D activations [T, cols] with
    // y [T, rows] for the batched Q4_K / Q6_K x Q8_0 paths.
    void matmul(const Tensor& w, const Tensor& x, Tensor& y, const AttributeMap& attrs) {
        const int qt = qtype(w.dtype());
        const bool batched = x.shape().size() == 2 && x.shape()[0] > 1;
        const int T = batched ? static_cast<int>(x.shape()[0]) : 1;
        const int cols = static_cast<int>(x.numel() / T);
        const int rows = static_cast<int>(y.numel() / T);
        const size_t row_bytes =
            (size_t)attrs.get_or<int64_t>("row_bytes", (int64_t)axf_row_bytes(qt, cols));
        const int acc = attrs.get_or<int64_t>("accumulate", 0) ? 1 : 0;
        float* yp = static_cast<float*>(y.raw_data());
        if (x.dtype() == DType::F32) {
            if (batched || acc) throw std::runtime_error("HIP MATMUL: F32 activations support M=1 only");
            if (qt == AXF_TYPE_Q4_K)
                check(axf_hip_gemv_q4k_f32(ctx_, yp, w.raw_data(), f32(x), rows, cols, row_bytes),
                      "HIP MATMUL");
            else
                check(axf_hip_gemv_q6k_f32(ctx_, yp, w.raw_data(), f32(x), rows, cols, row_bytes),
                      "HIP MATMUL");
        } else if (x.dtype() == DType::Q8_0) {
            if (batched) {
                if (acc) throw std::runtime_error("HIP MATMUL: batched path does not accumulate");
                if (qt == AXF_TYPE_Q4_K)
                    check(axf_hip_gemm_q4k_q8(ctx_, yp, w.raw_data(), x.raw_data(), rows, T, cols,
                                              row_bytes),
                          "HIP MATMUL");
                else
                    check(axf_hip_gemm_q6k_q8(ctx_, yp, w.raw_data(), x.raw_data(), rows, T, cols,
                                              row_bytes),
                          "HIP MATMUL");
            } else if (qt == AXF_TYPE_Q4_K) {
                check(axf_hip_gemv_q4k_q8(ctx_, yp, w.raw_data(), x.raw_data(), rows, cols,
                                          row_bytes, acc),
                      "HIP MATMUL");
            } else {
                check(axf_hip_gemv_q6k_q8(ctx_, yp, w.raw_data(), x.raw_data(), rows, cols,
                                          row_bytes, acc),
                      "HIP MATMUL");
            }
        } else {
            throw std::runtime_error("HIP MATMUL: activation must be F32 or Q8_0");
        }
    }

    const RopeTable& table(int hd, float theta, int need_pos) {
        RopeTable& t = (*ropes_)[{hd, theta}];
        if (t.max_pos < need_pos) {
            int mp = t.max_pos ? t.max_pos : 256;
            while (mp < need_pos) mp *= 2;
            std::vector<float> c((size_t)mp * hd / 2), s(c.size());
            check(axf_rope_table(c.data(), s.data(), hd, theta, mp), "HIP ROPE table");
            void *dc = nullptr, *ds = nullptr;
            check(axf_hip_alloc(ctx_, c.size() * 4, &dc), "HIP ROPE table");
            check(axf_hip_alloc(ctx_, s.size() * 4, &ds), "HIP ROPE table");
            check(axf_hip_memcpy_h2d(ctx_, dc, c.data(), c.size() * 4), "HIP ROPE table");
            check(axf_hip_memcpy_h2d(ctx_, ds, s.data(), s.size() * 4), "HIP ROPE table");
            if (t.cos_t) {
                axf_hip_sync(ctx_);
                axf_hip_free(ctx_, t.cos_t);
                axf_hip_free(ctx_, t.sin_t);
            }
            t = RopeTable{static_cast<float*>(dc), static_cast<float*>(ds), mp};
        }
        return t;
    }

    OpType op_;
    axf_ctx* ctx_;
    std::map<std::pair<int, float>, RopeTable>* ropes_;
};

class HipBackend final : public IBackend {
public:
    HipBackend() = default;
    ~HipBackend() override { finalize(); }

    std::string_view name() const noexcept override { return "hip"; }
    DeviceId device_id() const noexcept override { return DeviceId{DeviceType::HIP, 0}; }

    bool initialize() override {
        if (ctx_) return true;
        int n = 0;
        check(axf_hip_device_count(&n), "axf_hip_device_count");
        if (n <= 0) return false;
        check(axf_hip_create(0, &ctx_), "axf_hip_create");
        char name[256];
        if (axf_hip_device_name(ctx_, name, sizeof(name)) == AXF_OK)
            std::printf("[AxonForge] HIP backend: %s\n", name);
        return true;
    }

    void finalize() override {
        if (!ctx_) return;
        axf_hip_sync(ctx_);
        for (auto& kv : ropes_) {
            axf_hip_free(ctx_, kv.second.cos_t);
            axf_hip_free(ctx_, kv.second.sin_t);
        }
        ropes_.clear();
        axf_hip_destroy(ctx_);
        ctx_ = nullptr;
    }

    std::shared_ptr<TensorStorage> allocate(size_t bytes, size_t) override {
        require_init();
        return std::make_shared<HipTensorStorage>(ctx_, bytes);
    }

    // Bytes a contiguous tensor's data spans.  The reference's Tensor::nbytes()
    // counts block-quantized elements as 1 byte (Q6_K as 0), so block types take
    // their block sizes here: Q4_K 144 and Q6_K 210 bytes per 256 weights, Q5_0
    // 22 per 32, and Q8_0 the 36-byte activation block of q8_block.hpp:8-15.
    static size_t span_bytes(const Tensor& t) {
        const auto n = static_cast<size_t>(t.numel());
        switch (t.dtype()) {
            case DType::Q4_K_M: return n / 256 * 144;
            case DType::Q6_K: return n / 256 * 210;
            case DType::Q5_0: return n / 32 * 22;
            case DType::Q8_0: return n / 32 * 36;
            default: return t.nbytes();
        }
    }

    // Synchronous copy, as CudaBackend::transfer (cuda_backend.cu:170-178);
    // both storages must hold the span.
    void transfer(const Tensor& src, Tensor& dst) override {
        require_init();
        const size_t n = span_bytes(src);
        if (src.dtype() != dst.dtype() || src.numel() != dst.numel() || n != span_bytes(dst))
            throw std::runtime_error("HipBackend::transfer: size mismatch");
        if (!src.storage() || !dst.storage() || src.storage()->byte_size() < n ||
            dst.storage()->byte_size() < n)
            throw std::runtime_error("HipBackend::transfer: storage smaller than the tensor");
        void* d = dst.raw_data();
        const void* s = src.raw_data();
        const bool sh = src.device().type == DeviceType::HIP,
                   dh = dst.device().type == DeviceType::HIP;
        if (sh && dh)
            check(axf_hip_memcpy_d2d(ctx_, d, s, n), "HipBackend::transfer");
        else if (dh)
            check(axf_hip_memcpy_h2d(ctx_, d, s, n), "HipBackend::transfer");
        else if (sh)
            check(axf_hip_memcpy_d2h(ctx_, d, s, n), "HipBackend::transfer");
        else
            std::memcpy(d, s, n);
        synchronize();
    }

    void synchronize() override {
        if (ctx_) check(axf_hip_sync(ctx_), "HipBackend::synchronize");
    }

    bool can_handle(OpType op, std::span<const DType> dt) const override {
        switch (op) {
            case OpType::RMS_NORM:
            case OpType::SILU:
            case OpType::MUL:
            case OpType::ADD:
            case OpType::ROPE:
                return dt.empty() || dt[0] == DType::F32;
            case OpType::MATMUL:
                return dt.size() >= 2 && (dt[0] == DType::Q4_K_M || dt[0] == DType::Q6_K) &&
                       (dt[1] == DType::F32 || dt[1] == DType::Q8_0);
            case OpType::EMBEDDING_LOOKUP:
                return !dt.empty() && (dt[0] == DType::Q4_K_M || dt[0] == DType::Q6_K);
            default:
                return false;
        }
    }

    std::unique_ptr<IKernel> get_kernel(OpType op, std::span<const DType> dt,
                                        const AttributeMap&) override {
        require_init();
        if (!can_handle(op, dt))
            throw std::runtime_error("HipBackend::get_kernel: unsupported op/dtype combination");
        return std::make_unique<HipKernel>(op, ctx_, &ropes_);
    }

private:
    void require_init() const {
        if (!ctx_) throw std::runtime_error("HipBackend: initialize() has not succeeded");
    }

    axf_ctx* ctx_ = nullptr;
    std::map<std::pair<int, float>, RopeTable> ropes_;
};

}  // namespace
}  // namespace axf

[[gnu::constructor]] static void axf_register_hip_backend() {
    axf_api::BackendRegistry::instance().register_backend(
        "hip", []() -> std::unique_ptr<axf_api::IBackend> { return std::make_unique<axf::HipBackend>(); });
}
