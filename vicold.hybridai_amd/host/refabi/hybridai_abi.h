// hybridai_abi.h -- the reference's backend plug-in ABI, declared here so the
// MI355X backend builds and is tested without the reference tree.
//
// A backend is a subclass of hybridai::Backend that the reference's
// BackendRegistry creates by name.  For the subclass to drop into a
// reference build, everything that crosses that boundary must have the
// reference's exact shape, so this header keeps, from the files cited:
//   * enum values and underlying types: StatusCode (src/core/status.h:9-21),
//     DeviceType (src/core/device.h:9-14), DType (src/core/dtype.h:8-19),
//     MemoryType (src/backends/interface/backend.h:20-26);
//   * the data members of Status and Device in order (status.h:23-39,
//     device.h:16-53), which are passed and returned by value;
//   * the virtual functions of Allocator, Stream, Event, Buffer and Backend
//     in vtable order with identical signatures (backend.h:28-263);
//   * the BackendRegistry / KernelRegistry entry points and the
//     HYBRIDAI_REGISTER_BACKEND macro (src/backends/backend_registry.h:12-49,
//     src/ops/registry.h:18-81).
// Compiling with HAI_WITH_REFERENCE_TREE (and the reference's src/ on the
// include path) uses the reference's own headers instead; the
// `override`-checked MI355X backend compiles either way.
#pragma once

#ifdef HAI_WITH_REFERENCE_TREE
#include "backends/backend_registry.h"
#include "core/tensor.h"
#include "ops/registry.h"
#else

#include <cstddef>
#include <cstdint>
#include <functional>
#include <memory>
#include <mutex>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

namespace hybridai {

enum class StatusCode : int32_t {
    OK = 0,
    InvalidArgument = 1,
    OutOfMemory = 2,
    NotImplemented = 3,
    InternalError = 4,
    InvalidDevice = 5,
    UnsupportedDType = 6,
    FileNotFound = 7,
    InvalidModel = 8,
    BackendError = 9,
    Unknown = 99,
};

class Status {
public:
    Status() noexcept : code_(StatusCode::OK) {}
    explicit Status(StatusCode code) noexcept : code_(code) {}
    Status(StatusCode code, std::string_view message) : code_(code), message_(message) {}
    bool ok() const noexcept { return code_ == StatusCode::OK; }
    StatusCode code() const noexcept { return code_; }
    const std::string& message() const noexcept { return message_; }
    static Status OK() noexcept { return Status(); }

private:
    StatusCode code_;
    std::string message_;
};

enum class DeviceType : uint8_t { CPU, IntegratedGPU, DiscreteGPU, Unknown };

class Device {
public:
    Device() noexcept : id_(0), type_(DeviceType::CPU) {}
    Device(int32_t id, DeviceType type, std::string_view backend, bool unified_memory = false)
        : id_(id), type_(type), backend_(backend), unified_memory_supported_(unified_memory) {}
    int32_t id() const noexcept { return id_; }
    DeviceType type() const noexcept { return type_; }
    const std::string& backend() const noexcept { return backend_; }
    bool unified_memory_supported() const noexcept { return unified_memory_supported_; }
    bool is_cpu() const noexcept { return type_ == DeviceType::CPU; }
    bool is_gpu() const noexcept { return type_ == DeviceType::IntegratedGPU || type_ == DeviceType::DiscreteGPU; }
    static Device Cpu() noexcept { return Device(0, DeviceType::CPU, "cpu", false); }
    bool operator==(const Device& o) const noexcept {
        return id_ == o.id_ && type_ == o.type_ && backend_ == o.backend_;
    }
    bool operator!=(const Device& o) const noexcept { return !(*this == o); }

private:
    int32_t id_;
    DeviceType type_;
    std::string backend_;
    bool unified_memory_supported_ = false;
};

enum class DType : uint8_t { FP32, FP16, BF16, FP8_E4M3, FP8_E5M2, INT8, INT32, INT64, UINT8, BOOL };

constexpr size_t SizeOfDType(DType t) {
    switch (t) {
        case DType::FP32: case DType::INT32: return 4;
        case DType::FP16: case DType::BF16: return 2;
        case DType::INT64: return 8;
        case DType::FP8_E4M3: case DType::FP8_E5M2: case DType::INT8: case DType::UINT8: case DType::BOOL: return 1;
    }
    return 0;
}

class Buffer;
class Stream;
class Event;
class Tensor;  // only named by kernel signatures here

enum class MemoryType : uint8_t { Device, Unified, HostPinned, Host };

class Allocator {
public:
    virtual ~Allocator() = default;
    virtual Status allocate(size_t size, void** ptr) = 0;
    virtual Status deallocate(void* ptr) = 0;
    virtual MemoryType memory_type() const noexcept = 0;
};

class Stream {
public:
    virtual ~Stream() = default;
    virtual Status synchronize() = 0;
};

class Event {
public:
    virtual ~Event() = default;
    virtual Status record(Stream* stream) = 0;
    virtual Status wait(Stream* stream) = 0;
    virtual Status synchronize() = 0;
    virtual Status elapsed_time_since(const Event& start, double* milliseconds) const = 0;
};

class Buffer {
public:
    virtual ~Buffer() = default;
    virtual void* data() noexcept = 0;
    virtual const void* data() const noexcept = 0;
    virtual size_t size() const noexcept = 0;
    virtual Device device() const noexcept = 0;
    virtual MemoryType memory_type() const noexcept = 0;
};

// Optional kernels return NotImplemented by default so callers keep their
// CPU fallback (the reference's contract); the order of declaration is the
// vtable order and must not change.
#define HAI_ABI_NOT_IMPL(what) return Status(StatusCode::NotImplemented, what)

class Backend {
public:
    virtual ~Backend() = default;
    virtual const char* name() const noexcept = 0;
    virtual Device device() const noexcept = 0;
    virtual bool is_available() const noexcept = 0;
    virtual std::vector<Device> enumerate_devices() const { return {}; }
    virtual std::unique_ptr<Allocator> create_allocator(MemoryType type) = 0;
    virtual std::unique_ptr<Stream> create_stream() = 0;
    virtual std::unique_ptr<Event> create_event() = 0;
    virtual std::shared_ptr<Buffer> create_buffer(size_t size, MemoryType type) = 0;
    virtual Status memcpy_h2d(Buffer* dst, const void* src, size_t size, Stream* stream = nullptr) = 0;
    virtual Status memcpy_d2h(void* dst, const Buffer* src, size_t size, Stream* stream = nullptr) = 0;
    virtual Status memcpy_d2d(Buffer* dst, const Buffer* src, size_t size, Stream* stream = nullptr) = 0;
    virtual Status copy(Buffer* dst, const Buffer* src, size_t size, Stream* stream = nullptr) = 0;
    virtual Status memset(Buffer* dst, int value, size_t size, Stream* stream = nullptr) = 0;
    virtual Status synchronize() = 0;
    virtual Status gemm(Buffer* c, const Buffer* a, const Buffer* b, DType c_type, DType a_type, DType b_type,
                        DType compute_type, bool trans_a, bool trans_b, int64_t m, int64_t n, int64_t k,
                        float alpha, float beta, Stream* stream = nullptr) = 0;
    virtual Status cast(Buffer*, const Buffer*, DType, DType, int64_t, Stream* = nullptr) {
        HAI_ABI_NOT_IMPL("cast");
    }
    virtual Status add(Buffer*, const Buffer*, const Buffer*, DType, int64_t, Stream* = nullptr) {
        HAI_ABI_NOT_IMPL("add");
    }
    virtual Status embedding_gather(Buffer*, const Buffer*, const Buffer*, DType, int64_t, int64_t, int64_t,
                                    Stream* = nullptr) {
        HAI_ABI_NOT_IMPL("embedding_gather");
    }
    virtual Status rmsnorm(Buffer*, const Buffer*, const Buffer*, DType, int64_t, int64_t, float, bool,
                           Stream* = nullptr) {
        HAI_ABI_NOT_IMPL("rmsnorm");
    }
    virtual Status unary(Buffer*, const Buffer*, DType, int64_t, int, float, Stream* = nullptr) {
        HAI_ABI_NOT_IMPL("unary");
    }
    virtual Status silu_mul(Buffer*, const Buffer*, const Buffer*, DType, int64_t, Stream* = nullptr) {
        HAI_ABI_NOT_IMPL("silu_mul");
    }
    virtual Status split_q_gate(Buffer*, Buffer*, const Buffer*, DType, int64_t, int64_t, int64_t,
                                Stream* = nullptr) {
        HAI_ABI_NOT_IMPL("split_q_gate");
    }
    virtual Status partial_rope(Buffer*, const Buffer*, DType, int64_t, int64_t, int64_t, int64_t, int64_t, float,
                                Stream* = nullptr) {
        HAI_ABI_NOT_IMPL("partial_rope");
    }
    virtual Status qk_rmsnorm_rope(Buffer*, const Buffer*, const Buffer*, Buffer*, const Buffer*, const Buffer*,
                                   DType, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, float, float, bool,
                                   Stream* = nullptr) {
        HAI_ABI_NOT_IMPL("qk_rmsnorm_rope");
    }
    virtual Status causal_gqa(Buffer*, const Buffer*, const Buffer*, const Buffer*, const Buffer*, DType, int64_t,
                              int64_t, int64_t, int64_t, Stream* = nullptr) {
        HAI_ABI_NOT_IMPL("causal_gqa");
    }
    virtual Status append_kv_cache(Buffer*, Buffer*, const Buffer*, const Buffer*, DType, int64_t, int64_t, int64_t,
                                   int64_t, int64_t, Stream* = nullptr) {
        HAI_ABI_NOT_IMPL("append_kv_cache");
    }
    virtual Status cached_gqa(Buffer*, const Buffer*, const Buffer*, const Buffer*, const Buffer*, DType, int64_t,
                              int64_t, int64_t, int64_t, int64_t, Stream* = nullptr) {
        HAI_ABI_NOT_IMPL("cached_gqa");
    }
    virtual Status cached_gqa_with_current_token(Buffer*, const Buffer*, const Buffer*, const Buffer*,
                                                 const Buffer*, const Buffer*, const Buffer*, DType, int64_t,
                                                 int64_t, int64_t, int64_t, Stream* = nullptr) {
        HAI_ABI_NOT_IMPL("cached_gqa_with_current_token");
    }
    virtual Status causal_conv1d_silu(Buffer*, Buffer*, const Buffer*, const Buffer*, DType, int64_t, int64_t,
                                      int64_t, Stream* = nullptr) {
        HAI_ABI_NOT_IMPL("causal_conv1d_silu");
    }
    virtual Status deltanet_grouped_conv(Buffer*, Buffer*, Buffer*, Buffer*, const Buffer*, const Buffer*, DType,
                                         int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, Stream* = nullptr) {
        HAI_ABI_NOT_IMPL("deltanet_grouped_conv");
    }
    virtual Status deltanet_recurrent(Buffer*, Buffer*, const Buffer*, const Buffer*, const Buffer*, const Buffer*,
                                      const Buffer*, const Buffer*, const Buffer*, const Buffer*, const Buffer*,
                                      DType, int64_t, int64_t, int64_t, int64_t, int64_t, float,
                                      Stream* = nullptr) {
        HAI_ABI_NOT_IMPL("deltanet_recurrent");
    }
    virtual Status argmax_last_row(Buffer*, const Buffer*, DType, int64_t, int64_t, Stream* = nullptr) {
        HAI_ABI_NOT_IMPL("argmax_last_row");
    }
    virtual Status argmax_rows(Buffer*, const Buffer*, DType, int64_t, int64_t, Stream* = nullptr) {
        HAI_ABI_NOT_IMPL("argmax_rows");
    }
    virtual void register_kernels() {}
    virtual Status add_row_bias(Buffer*, const Buffer*, DType, int64_t, int64_t, Stream* = nullptr) {
        HAI_ABI_NOT_IMPL("add_row_bias");
    }
    virtual Status strided_copy(Buffer*, const Buffer*, DType, int64_t, const int64_t*, const int64_t*, int64_t,
                                Stream* = nullptr) {
        HAI_ABI_NOT_IMPL("strided_copy");
    }
    virtual Status copy_to_offset(Buffer*, size_t, const Buffer*, size_t, size_t, Stream* = nullptr) {
        HAI_ABI_NOT_IMPL("copy_to_offset");
    }
    virtual Status q_gate_rmsnorm_rope(Buffer*, Buffer*, const Buffer*, const Buffer*, DType, int64_t, int64_t,
                                       int64_t, int64_t, int64_t, float, float, bool, Stream* = nullptr) {
        HAI_ABI_NOT_IMPL("q_gate_rmsnorm_rope");
    }
};

#undef HAI_ABI_NOT_IMPL

using BackendFactory = std::function<std::unique_ptr<Backend>(const Device&)>;

// Name -> factory, plus one shared instance per (name, device id, type).
class BackendRegistry {
public:
    static BackendRegistry& instance();
    void register_backend(std::string_view name, BackendFactory factory);
    std::unique_ptr<Backend> create_backend(const Device& device);
    std::shared_ptr<Backend> get_backend(const Device& device);
    bool has_backend(std::string_view name) const;
    std::vector<std::string> backend_names() const;

private:
    BackendRegistry() = default;
    mutable std::mutex mutex_;
    std::unordered_map<std::string, BackendFactory> factories_;
    std::unordered_map<std::string, std::shared_ptr<Backend>> backends_;
};

class BackendRegistrar {
public:
    BackendRegistrar(std::string_view name, BackendFactory factory) {
        BackendRegistry::instance().register_backend(name, std::move(factory));
    }
};

#define HYBRIDAI_REGISTER_BACKEND(name, factory) \
    static ::hybridai::BackendRegistrar g_hybridai_backend_##name(#name, factory)

namespace ops {

using KernelFn = std::function<Status(const std::vector<Tensor*>& inputs, std::vector<Tensor*>& outputs)>;

struct KernelKey {
    std::string op_name;
    DeviceType device_type;
    DType dtype;
    bool operator==(const KernelKey& o) const noexcept {
        return op_name == o.op_name && device_type == o.device_type && dtype == o.dtype;
    }
};

struct KernelKeyHash {
    size_t operator()(const KernelKey& k) const noexcept {
        return std::hash<std::string>{}(k.op_name) ^ (static_cast<size_t>(k.device_type) << 8) ^
               (static_cast<size_t>(k.dtype) << 16);
    }
};

class KernelRegistry {
public:
    static KernelRegistry& instance();
    bool register_kernel(const KernelKey& key, KernelFn kernel, bool overwrite = false);
    KernelFn find_kernel(const KernelKey& key) const;
    bool has_kernel(const KernelKey& key) const;
    bool unregister_kernel(const KernelKey& key);
    size_t kernel_count() const;

private:
    KernelRegistry() = default;
    mutable std::mutex mutex_;
    std::unordered_map<KernelKey, KernelFn, KernelKeyHash> kernels_;
};

}  // namespace ops
}  // namespace hybridai

#endif  // HAI_WITH_REFERENCE_TREE
