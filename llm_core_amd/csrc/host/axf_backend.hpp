// axf_backend.hpp — host-side plugin interface of this library, mirroring the
// reference engine's backend API so a `-b hip` backend drops into the same
// registry slot:
//   IKernel / IBackend / BackendRegistry : include/axonforge/backend.hpp:18-104
//   DType values (GGUF-compatible)        : include/axonforge/dtype.hpp:8-31
//   dtype_element_size                    : dtype.hpp:34-51
//   DeviceId / TensorStorage / Tensor     : common.hpp:9-33, memory.hpp:12-24, tensor.hpp
//   OpType subset, AttributeMap           : graph.hpp:17-80
// Only what the quantized decode path needs is declared here; names, argument
// meaning and error behaviour (std::runtime_error) follow the reference.
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <memory>
#include <span>
#include <string>
#include <string_view>
#include <unordered_map>
#include <variant>
#include <vector>

namespace axf {

enum class DType : uint8_t {
    F32 = 0,
    F16 = 1,
    BF16 = 2,
    Q8_0 = 8,
    Q4_0 = 9,
    Q4_K_M = 10,
    Q3_K_M = 11,
    Q2_K = 12,
    Q6_K = 13,
    Q5_0 = 14,
    I32 = 16,
    I16 = 17,
    I8 = 18,
    BOOL = 24,
    UNKNOWN = 255,
};

// Bytes per element as the reference counts them (dtype_element_size,
// dtype.hpp:34-51): exact for the plain types, 1 ("approx") for the
// block-quantized Q8_0 / Q4_0 / Q5_0 / Q4_K_M / Q3_K_M / Q2_K and 0 for the
// others (Q6_K included).  Tensor::nbytes() is numel times this; block
// tensors carry their real size in their storage (Tensor::from_raw_blob).
constexpr size_t dtype_element_size(DType dtype) noexcept {
    switch (dtype) {
        case DType::F32: return 4;
        case DType::F16: return 2;
        case DType::BF16: return 2;
        case DType::Q8_0: return 1;
        case DType::Q4_0: return 1;
        case DType::Q5_0: return 1;
        case DType::Q4_K_M: return 1;
        case DType::Q3_K_M: return 1;
        case DType::Q2_K: return 1;
        case DType::I32: return 4;
        case DType::I16: return 2;
        case DType::I8: return 1;
        case DType::BOOL: return 1;
        default: return 0;
    }
}

enum class DeviceType : uint8_t { CPU = 0, CUDA = 1, Vulkan = 2, Metal = 3, NPU = 4, HIP = 5 };

struct DeviceId {
    DeviceType type{DeviceType::CPU};
    int32_t index{0};
    constexpr bool operator==(const DeviceId&) const noexcept = default;
    constexpr bool is_cpu() const noexcept { return type == DeviceType::CPU; }
    static constexpr DeviceId cpu(int i = 0) { return {DeviceType::CPU, i}; }
};

class TensorStorage {
public:
    virtual ~TensorStorage() = default;
    virtual void* data() noexcept = 0;
    virtual const void* data() const noexcept = 0;
    virtual size_t byte_size() const noexcept = 0;
    virtual DeviceId device() const noexcept = 0;
};

class CpuTensorStorage final : public TensorStorage {
public:
    explicit CpuTensorStorage(size_t bytes);
    CpuTensorStorage(void* external, size_t bytes);  // non-owning view
    ~CpuTensorStorage() override;
    void* data() noexcept override { return ptr_; }
    const void* data() const noexcept override { return ptr_; }
    size_t byte_size() const noexcept override { return bytes_; }
    DeviceId device() const noexcept override { return DeviceId::cpu(); }

private:
    void* ptr_{nullptr};
    size_t bytes_{0};
    bool owns_{true};
};

using Shape = std::vector<int64_t>;

// Contiguous tensor view (the reference's Tensor has strides and view ops;
// the backend only consumes contiguous tensors).
class Tensor {
public:
    Tensor() = default;
    static Tensor zeros(Shape shape, DType dtype);
    static Tensor from_blob(void* data, Shape shape, DType dtype);
    // block-quantized data whose size is not numel * dtype_element_size
    static Tensor from_raw_blob(void* data, size_t nbytes, Shape shape, DType dtype);
    static Tensor from_storage(std::shared_ptr<TensorStorage> storage, Shape shape, DType dtype);

    const Shape& shape() const noexcept { return shape_; }
    DType dtype() const noexcept { return dtype_; }
    DeviceId device() const noexcept { return storage_ ? storage_->device() : DeviceId::cpu(); }
    int64_t numel() const noexcept;
    size_t nbytes() const noexcept { return (size_t)numel() * dtype_element_size(dtype_); }
    void* raw_data() noexcept { return storage_ ? storage_->data() : nullptr; }
    const void* raw_data() const noexcept { return storage_ ? storage_->data() : nullptr; }
    template <class T>
    std::span<T> data_as() noexcept {
        return {static_cast<T*>(raw_data()), static_cast<size_t>(numel())};
    }
    std::shared_ptr<TensorStorage> storage() const noexcept { return storage_; }

private:
    std::shared_ptr<TensorStorage> storage_;
    Shape shape_;
    DType dtype_{DType::UNKNOWN};
};

// Same enumerator values as the reference's OpType (graph.hpp:17-55).
enum class OpType : uint16_t {
    SILU = 6,
    ADD = 11,
    MUL = 13,
    MATMUL = 28,
    RMS_NORM = 31,
    SOFTMAX = 32,
    ROPE = 33,
    EMBEDDING_LOOKUP = 34,
    CUSTOM = 0xFFFF,
};

using AttrValue = std::variant<int64_t, float, bool, std::string, std::vector<int64_t>>;

class AttributeMap {
public:
    void set(std::string_view key, AttrValue value) { data_[std::string(key)] = std::move(value); }
    const AttrValue* get(std::string_view key) const noexcept {
        auto it = data_.find(std::string(key));
        return it == data_.end() ? nullptr : &it->second;
    }
    template <typename T>
    T get_or(std::string_view key, T default_val) const {
        if (auto* v = get(key); v)
            if (auto* p = std::get_if<T>(v)) return *p;
        return default_val;
    }

private:
    std::unordered_map<std::string, AttrValue> data_;
};

class IKernel {
public:
    virtual ~IKernel() = default;
    virtual void execute(std::span<const Tensor> inputs, std::span<Tensor> outputs,
                         const AttributeMap& attrs) = 0;
};

class IBackend {
public:
    virtual ~IBackend() = default;
    virtual std::string_view name() const noexcept = 0;
    virtual DeviceId device_id() const noexcept = 0;
    virtual bool initialize() = 0;
    virtual void finalize() = 0;
    virtual std::shared_ptr<TensorStorage> allocate(size_t bytes, size_t alignment = 64) = 0;
    virtual void transfer(const Tensor& src, Tensor& dst) = 0;
    virtual void synchronize() = 0;
    virtual bool can_handle(OpType op, std::span<const DType> input_dtypes) const = 0;
    virtual std::unique_ptr<IKernel> get_kernel(OpType op, std::span<const DType> input_dtypes,
                                                const AttributeMap& attrs) = 0;
};

class BackendRegistry {
public:
    using FactoryFn = std::function<std::unique_ptr<IBackend>()>;
    static BackendRegistry& instance();
    void register_backend(std::string_view id, FactoryFn factory);
    std::unique_ptr<IBackend> create(std::string_view id) const;
    bool has_backend(std::string_view id) const noexcept;
    std::vector<std::string> available_backends() const;

private:
    BackendRegistry() = default;
    std::unordered_map<std::string, FactoryFn> factories_;
};

}  // namespace axf
