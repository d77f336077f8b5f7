// mi355x_backend.cc -- the MI355X hybridai::Backend on top of the hai_* ABI.
#include "mi355x_backend.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <map>
#include <memory>
#include <mutex>
#include <string>

#include "hai_kernels.h"

namespace hybridai {

namespace {

Status from_hai(int rc, const char* what) {
    if (rc == HAI_OK) return Status::OK();
    StatusCode code = StatusCode::BackendError;
    if (rc == HAI_ERR_INVALID_ARGUMENT) code = StatusCode::InvalidArgument;
    else if (rc == HAI_ERR_OUT_OF_MEMORY) code = StatusCode::OutOfMemory;
    else if (rc == HAI_ERR_NOT_IMPLEMENTED) code = StatusCode::NotImplemented;
    else if (rc == HAI_ERR_INVALID_DEVICE) code = StatusCode::InvalidDevice;
    return Status(code, std::string(what) + ": " + hai_last_error());
}

#define HAI_STATUS(expr, what)                                  \
    do {                                                        \
        const int _rc = (expr);                                 \
        if (_rc != HAI_OK) return from_hai(_rc, what);          \
    } while (0)

#define RETURN_IF_ERROR(expr)                                   \
    do {                                                        \
        Status _st = (expr);                                    \
        if (!_st.ok()) return _st;                              \
    } while (0)

Status invalid(const std::string& what) { return Status(StatusCode::InvalidArgument, "MI355XBackend: " + what); }
Status not_impl(const std::string& what) { return Status(StatusCode::NotImplemented, "MI355XBackend: " + what); }

// ---- resources ---------------------------------------------------------------

class HaiStream final : public Stream {
public:
    explicit HaiStream(void* s) : s_(s) {}
    ~HaiStream() override {
        if (s_) hai_stream_destroy(s_);
    }
    Status synchronize() override {
        HAI_STATUS(hai_stream_synchronize(s_), "stream synchronize");
        return Status::OK();
    }
    void* handle() const { return s_; }

private:
    void* s_;
};

// The native stream of a Backend call: null means the null stream; any
// other Stream type is not ours.
Status native(Stream* stream, void** out) {
    *out = nullptr;
    if (stream == nullptr) return Status::OK();
    auto* hs = dynamic_cast<HaiStream*>(stream);
    if (hs == nullptr) return invalid("stream was not created by this backend");
    *out = hs->handle();
    return Status::OK();
}

class HaiEvent final : public Event {
public:
    explicit HaiEvent(void* e) : e_(e) {}
    ~HaiEvent() override {
        if (e_) hai_event_destroy(e_);
    }
    Status record(Stream* stream) override {
        void* s = nullptr;
        RETURN_IF_ERROR(native(stream, &s));
        HAI_STATUS(hai_event_record(e_, s), "event record");
        return Status::OK();
    }
    Status wait(Stream* stream) override {
        void* s = nullptr;
        RETURN_IF_ERROR(native(stream, &s));
        HAI_STATUS(hai_stream_wait_event(s, e_), "event wait");
        return Status::OK();
    }
    Status synchronize() override {
        HAI_STATUS(hai_event_synchronize(e_), "event synchronize");
        return Status::OK();
    }
    Status elapsed_time_since(const Event& start, double* milliseconds) const override {
        const auto* st = dynamic_cast<const HaiEvent*>(&start);
        if (st == nullptr || milliseconds == nullptr) return invalid("elapsed_time_since arguments");
        float ms = 0.0f;
        HAI_STATUS(hai_event_elapsed_ms(st->e_, e_, &ms), "event elapsed time");
        *milliseconds = ms;
        return Status::OK();
    }

private:
    void* e_;
};

Status raw_alloc(MemoryType type, size_t size, void** ptr) {
    *ptr = nullptr;
    switch (type) {
        case MemoryType::Device:
            HAI_STATUS(hai_malloc(ptr, size), "device allocation");
            return Status::OK();
        case MemoryType::HostPinned:
            HAI_STATUS(hai_host_malloc(ptr, size), "pinned host allocation");
            return Status::OK();
        case MemoryType::Host:
            *ptr = std::malloc(size == 0 ? 1 : size);
            return *ptr ? Status::OK() : Status(StatusCode::OutOfMemory, "MI355XBackend: host allocation");
        case MemoryType::Unified:
            break;
    }
    return not_impl("unified memory buffers");
}

void raw_free(MemoryType type, void* ptr) {
    if (ptr == nullptr) return;
    if (type == MemoryType::Device) hai_free(ptr);
    else if (type == MemoryType::HostPinned) hai_host_free(ptr);
    else std::free(ptr);
}

class HaiAllocator final : public Allocator {
public:
    explicit HaiAllocator(MemoryType t) : t_(t) {}
    Status allocate(size_t size, void** ptr) override {
        if (ptr == nullptr) return invalid("allocate: null output");
        return raw_alloc(t_, size, ptr);
    }
    Status deallocate(void* ptr) override {
        raw_free(t_, ptr);
        return Status::OK();
    }
    MemoryType memory_type() const noexcept override { return t_; }

private:
    MemoryType t_;
};

// Recycles the transient buffers of the reference's ops, which allocate
// every output through create_buffer: the same bounds as the reference's
// pool (hip_backend.cc:380-408: blocks up to 8 MiB pooled, at most 256 MiB
// cached per device and memory type; larger blocks go straight to the
// allocator), with size classes of at most 1.25x the request (256-byte
// steps up to 4 KiB, then four classes per power of two).  A block returns
// to its class's free list when its Buffer dies, without a device
// synchronisation: like the reference's, the pool relies on the ops running
// in stream order on one stream.
class BlockPool {
public:
    static constexpr size_t kMaxBlock = size_t{8} << 20;
    static constexpr size_t kMaxCached = size_t{256} << 20;

    explicit BlockPool(MemoryType t) : t_(t) {}

    static size_t size_class(size_t n) {
        if (n <= 4096) return std::max<size_t>(256, (n + 255) & ~size_t{255});
        size_t base = 4096;
        while (base * 2 < n) base *= 2;
        const size_t step = base / 4;
        return base + (n - base + step - 1) / step * step;
    }

    Status take(size_t n, void** p, size_t* cls) {
        *cls = n <= kMaxBlock ? size_class(n) : 0;
        if (*cls != 0) {
            std::lock_guard<std::mutex> lock(mu_);
            auto& fl = free_[*cls];
            if (!fl.empty()) {
                *p = fl.back();
                fl.pop_back();
                cached_ -= *cls;
                return Status::OK();
            }
        }
        return raw_alloc(t_, *cls != 0 ? *cls : n, p);
    }

    void give(void* p, size_t cls) {
        if (p == nullptr) return;
        if (cls != 0) {
            std::lock_guard<std::mutex> lock(mu_);
            if (cached_ + cls <= kMaxCached) {
                free_[cls].push_back(p);
                cached_ += cls;
                return;
            }
        }
        raw_free(t_, p);
    }

    size_t cached_bytes() {
        std::lock_guard<std::mutex> lock(mu_);
        return cached_;
    }

private:
    MemoryType t_;
    std::mutex mu_;
    std::map<size_t, std::vector<void*>> free_;
    size_t cached_ = 0;
};

// One pool per (device, memory type), shared by every backend instance of
// the process and kept until it ends (the cached blocks go with it).
std::shared_ptr<BlockPool> pool_for(int device, MemoryType type) {
    static std::mutex mu;
    static auto* pools = new std::map<std::pair<int, int>, std::shared_ptr<BlockPool>>();
    std::lock_guard<std::mutex> lock(mu);
    auto& p = (*pools)[{device, static_cast<int>(type)}];
    if (!p) p = std::make_shared<BlockPool>(type);
    return p;
}

class HaiBuffer final : public Buffer {
public:
    HaiBuffer(void* p, size_t n, Device d, MemoryType t, std::shared_ptr<BlockPool> pool, size_t cls)
        : p_(p), n_(n), d_(std::move(d)), t_(t), pool_(std::move(pool)), cls_(cls) {}
    ~HaiBuffer() override {
        if (pool_) pool_->give(p_, cls_);
        else raw_free(t_, p_);
    }
    void* data() noexcept override { return p_; }
    const void* data() const noexcept override { return p_; }
    size_t size() const noexcept override { return n_; }
    Device device() const noexcept override { return d_; }
    MemoryType memory_type() const noexcept override { return t_; }

private:
    void* p_;
    size_t n_;
    Device d_;
    MemoryType t_;
    std::shared_ptr<BlockPool> pool_;
    size_t cls_;
};

// Kernel operands must be device buffers of this backend's device holding
// at least `bytes` (the reference's validate_kernel_buffer contract).
Status need(const Buffer* b, const Device& dev, size_t bytes, const char* what) {
    if (b == nullptr || b->data() == nullptr || b->size() < bytes || b->device() != dev)
        return invalid(std::string("kernel buffer ") + what);
    return Status::OK();
}

Status need_bf16(DType t, const char* op) {
    if (t != DType::BF16) return not_impl(std::string(op) + " supports BF16 only");
    return Status::OK();
}

template <typename T>
T* at(Buffer* b, size_t byte_off = 0) {
    return reinterpret_cast<T*>(static_cast<char*>(b->data()) + byte_off);
}
template <typename T>
const T* at(const Buffer* b, size_t byte_off = 0) {
    return reinterpret_cast<const T*>(static_cast<const char*>(b->data()) + byte_off);
}

}  // namespace

// ---- lifetime, devices ----------------------------------------------------------

MI355XBackend::MI355XBackend(const Device& device) : device_(device) {}

MI355XBackend::~MI355XBackend() {
    if (is_available()) hai_set_device(device_.id());
    for (Scratch* s : {&gqa_, &argmax_})
        if (s->ptr) hai_free(s->ptr);
    for (auto& kv : rope_) {
        hai_free(kv.second.cos);
        hai_free(kv.second.sin);
    }
}

bool MI355XBackend::is_available() const noexcept {
    int n = 0;
    return hai_device_count(&n) == HAI_OK && device_.id() >= 0 && device_.id() < n;
}

std::vector<Device> MI355XBackend::enumerate_devices() const {
    std::vector<Device> out;
    int n = 0;
    if (hai_device_count(&n) != HAI_OK) return out;
    for (int i = 0; i < n; ++i) out.emplace_back(i, DeviceType::DiscreteGPU, "hip", false);
    return out;
}

Status MI355XBackend::select() const {
    if (!is_available()) return Status(StatusCode::InvalidDevice, "MI355XBackend: no such HIP device");
    HAI_STATUS(hai_set_device(device_.id()), "select device");
    return Status::OK();
}

Status MI355XBackend::scratch(Scratch& s, size_t bytes, void** out) {
    if (bytes > s.bytes) {
        if (s.ptr) {
            HAI_STATUS(hai_device_synchronize(), "scratch resize");  // no kernel may still use the old block
            hai_free(s.ptr);
            s = Scratch{};
        }
        HAI_STATUS(hai_malloc(&s.ptr, bytes), "scratch allocation");
        s.bytes = bytes;
    }
    *out = s.ptr;
    return Status::OK();
}

Status MI355XBackend::rope_table(int64_t rope_dims, float base, int64_t positions, const RopeTable** out) {
    RopeTable& t = rope_[{rope_dims, base}];
    if (positions > t.positions) {
        // grow geometrically; theta = pos / base^(2p/R) in double, as the oracle
        const int64_t n = std::max<int64_t>(positions, std::max<int64_t>(4096, 2 * t.positions));
        const int64_t half = std::max<int64_t>(1, rope_dims / 2);
        std::vector<float> c(static_cast<size_t>(n * half), 0.0f), s(c.size(), 0.0f);
        for (int64_t pos = 0; pos < n; ++pos)
            for (int64_t p = 0; p < rope_dims / 2; ++p) {
                const double theta = static_cast<double>(pos) /
                                     std::pow(static_cast<double>(base),
                                              static_cast<double>(2 * p) / static_cast<double>(rope_dims));
                c[pos * half + p] = static_cast<float>(std::cos(theta));
                s[pos * half + p] = static_cast<float>(std::sin(theta));
            }
        float *dc = nullptr, *ds = nullptr;
        HAI_STATUS(hai_malloc(reinterpret_cast<void**>(&dc), c.size() * 4), "rope table");
        const int rc = hai_malloc(reinterpret_cast<void**>(&ds), s.size() * 4);
        if (rc != HAI_OK) {
            hai_free(dc);
            return from_hai(rc, "rope table");
        }
        if (hai_memcpy_h2d(dc, c.data(), c.size() * 4, nullptr) != HAI_OK ||
            hai_memcpy_h2d(ds, s.data(), s.size() * 4, nullptr) != HAI_OK || hai_device_synchronize() != HAI_OK) {
            hai_free(dc);
            hai_free(ds);
            return from_hai(HAI_ERR_BACKEND, "rope table upload");
        }
        if (t.cos) {
            hai_free(t.cos);
            hai_free(t.sin);
        }
        t.cos = dc;
        t.sin = ds;
        t.positions = n;
    }
    *out = &t;
    return Status::OK();
}

std::unique_ptr<Allocator> MI355XBackend::create_allocator(MemoryType type) {
    return std::make_unique<HaiAllocator>(type);
}

std::unique_ptr<Stream> MI355XBackend::create_stream() {
    if (!select().ok()) return nullptr;
    void* s = nullptr;
    if (hai_stream_create(&s) != HAI_OK) return nullptr;
    return std::make_unique<HaiStream>(s);
}

std::unique_ptr<Event> MI355XBackend::create_event() {
    if (!select().ok()) return nullptr;
    void* e = nullptr;
    if (hai_event_create(&e) != HAI_OK) return nullptr;
    return std::make_unique<HaiEvent>(e);
}

std::shared_ptr<Buffer> MI355XBackend::create_buffer(size_t size, MemoryType type) {
    if (type == MemoryType::Host) {
        void* p = nullptr;
        if (!raw_alloc(type, size, &p).ok()) return nullptr;
        return std::make_shared<HaiBuffer>(p, size, device_, type, nullptr, 0);
    }
    if (!select().ok()) return nullptr;
    auto pool = pool_for(device_.id(), type);
    void* p = nullptr;
    size_t cls = 0;
    if (!pool->take(size, &p, &cls).ok()) return nullptr;
    return std::make_shared<HaiBuffer>(p, size, device_, type, std::move(pool), cls);
}

size_t MI355XBackend::pooled_bytes(MemoryType type) const { return pool_for(device_.id(), type)->cached_bytes(); }

// ---- copies -----------------------------------------------------------------------

Status MI355XBackend::memcpy_h2d(Buffer* dst, const void* src, size_t size, Stream* stream) {
    if (dst == nullptr || src == nullptr || dst->size() < size) return invalid("memcpy_h2d range");
    void* s = nullptr;
    RETURN_IF_ERROR(native(stream, &s));
    RETURN_IF_ERROR(select());
    HAI_STATUS(hai_memcpy(dst->data(), src, size, s), "memcpy_h2d");
    return Status::OK();
}

Status MI355XBackend::memcpy_d2h(void* dst, const Buffer* src, size_t size, Stream* stream) {
    if (dst == nullptr || src == nullptr || src->size() < size) return invalid("memcpy_d2h range");
    void* s = nullptr;
    RETURN_IF_ERROR(native(stream, &s));
    RETURN_IF_ERROR(select());
    HAI_STATUS(hai_memcpy(dst, src->data(), size, s), "memcpy_d2h");
    // The reference's D2H on the null stream returns with the data in place.
    if (s == nullptr) HAI_STATUS(hai_stream_synchronize(nullptr), "memcpy_d2h synchronize");
    return Status::OK();
}

Status MI355XBackend::memcpy_d2d(Buffer* dst, const Buffer* src, size_t size, Stream* stream) {
    return copy(dst, src, size, stream);
}

Status MI355XBackend::copy(Buffer* dst, const Buffer* src, size_t size, Stream* stream) {
    return copy_to_offset(dst, 0, src, 0, size, stream);
}

Status MI355XBackend::copy_to_offset(Buffer* dst, size_t dst_offset, const Buffer* src, size_t src_offset,
                                     size_t size, Stream* stream) {
    if (dst == nullptr || src == nullptr || dst_offset + size > dst->size() || src_offset + size > src->size())
        return invalid("offset copy range");
    void* s = nullptr;
    RETURN_IF_ERROR(native(stream, &s));
    RETURN_IF_ERROR(select());
    HAI_STATUS(hai_memcpy(at<char>(dst, dst_offset), at<char>(src, src_offset), size, s), "copy");
    return Status::OK();
}

Status MI355XBackend::memset(Buffer* dst, int value, size_t size, Stream* stream) {
    if (dst == nullptr || dst->size() < size) return invalid("memset range");
    if (dst->memory_type() == MemoryType::Host) {
        std::memset(dst->data(), value, size);
        return Status::OK();
    }
    void* s = nullptr;
    RETURN_IF_ERROR(native(stream, &s));
    RETURN_IF_ERROR(select());
    HAI_STATUS(hai_memset(dst->data(), value, size, s), "memset");
    return Status::OK();
}

Status MI355XBackend::synchronize() {
    RETURN_IF_ERROR(select());
    HAI_STATUS(hai_device_synchronize(), "synchronize");
    return Status::OK();
}

// ---- compute -----------------------------------------------------------------------

Status MI355XBackend::gemm(Buffer* c, const Buffer* a, const Buffer* b, DType c_type, DType a_type, DType b_type,
                           DType compute_type, bool trans_a, bool trans_b, int64_t m, int64_t n, int64_t k,
                           float alpha, float beta, Stream* stream) {
    if (m <= 0 || n <= 0 || k <= 0) return invalid("gemm dimensions");
    // The path's Linear: C[m,n] = A[m,k] * B[n,k]^T in bf16 with fp32
    // accumulation (linear.cc:149-155).  Other forms keep their fallback.
    if (c_type != DType::BF16 || a_type != DType::BF16 || b_type != DType::BF16 || compute_type != DType::FP32 ||
        trans_a || !trans_b || alpha != 1.0f || beta != 0.0f || k % 8 != 0)
        return not_impl("gemm supports bf16 C = A * B^T (alpha 1, beta 0, K % 8 == 0) only");
    RETURN_IF_ERROR(need(a, device_, static_cast<size_t>(m * k) * 2, "a"));
    RETURN_IF_ERROR(need(b, device_, static_cast<size_t>(n * k) * 2, "b"));
    RETURN_IF_ERROR(need(c, device_, static_cast<size_t>(m * n) * 2, "c"));
    void* s = nullptr;
    RETURN_IF_ERROR(native(stream, &s));
    RETURN_IF_ERROR(select());
    // One launch for any m: prompt-sized m runs in 16-row batches that read
    // each weight from HBM about once, every row in the canonical order
    // (bit-identical to the one-row result).
    HAI_STATUS(hai_gemm_bf16(c->data(), n, a->data(), k, b->data(), m, n, k, HAI_EPI_STORE, nullptr, 0, s), "gemm");
    return Status::OK();
}

Status MI355XBackend::add(Buffer* dst, const Buffer* lhs, const Buffer* rhs, DType dtype, int64_t count,
                          Stream* stream) {
    RETURN_IF_ERROR(need_bf16(dtype, "add"));
    const size_t bytes = static_cast<size_t>(count) * 2;
    RETURN_IF_ERROR(need(dst, device_, bytes, "dst"));
    RETURN_IF_ERROR(need(lhs, device_, bytes, "lhs"));
    RETURN_IF_ERROR(need(rhs, device_, bytes, "rhs"));
    void* s = nullptr;
    RETURN_IF_ERROR(native(stream, &s));
    RETURN_IF_ERROR(select());
    HAI_STATUS(hai_add_bf16(dst->data(), lhs->data(), rhs->data(), count, s), "add");
    return Status::OK();
}

Status MI355XBackend::embedding_gather(Buffer* dst, const Buffer* embedding, const Buffer* ids, DType dtype,
                                       int64_t num_ids, int64_t vocab_size, int64_t hidden_size, Stream* stream) {
    RETURN_IF_ERROR(need_bf16(dtype, "embedding_gather"));
    RETURN_IF_ERROR(need(dst, device_, static_cast<size_t>(num_ids * hidden_size) * 2, "dst"));
    RETURN_IF_ERROR(need(embedding, device_, static_cast<size_t>(vocab_size * hidden_size) * 2, "embedding"));
    RETURN_IF_ERROR(need(ids, device_, static_cast<size_t>(num_ids) * 8, "ids"));
    void* s = nullptr;
    RETURN_IF_ERROR(native(stream, &s));
    RETURN_IF_ERROR(select());
    HAI_STATUS(hai_embedding_gather_bf16(dst->data(), embedding->data(), at<int64_t>(ids), num_ids, vocab_size,
                                         hidden_size, s),
               "embedding_gather");
    return Status::OK();
}

Status MI355XBackend::rmsnorm(Buffer* dst, const Buffer* src, const Buffer* weight, DType dtype, int64_t rows,
                              int64_t hidden_size, float eps, bool add_unit_offset, Stream* stream) {
    RETURN_IF_ERROR(need_bf16(dtype, "rmsnorm"));
    const size_t bytes = static_cast<size_t>(rows * hidden_size) * 2;
    RETURN_IF_ERROR(need(dst, device_, bytes, "dst"));
    RETURN_IF_ERROR(need(src, device_, bytes, "src"));
    RETURN_IF_ERROR(need(weight, device_, static_cast<size_t>(hidden_size) * 2, "weight"));
    void* s = nullptr;
    RETURN_IF_ERROR(native(stream, &s));
    RETURN_IF_ERROR(select());
    HAI_STATUS(hai_rmsnorm_bf16(dst->data(), hidden_size, src->data(), hidden_size, weight->data(), rows,
                                hidden_size, eps, add_unit_offset ? 1 : 0, s),
               "rmsnorm");
    return Status::OK();
}

Status MI355XBackend::silu_mul(Buffer* dst, const Buffer* gate, const Buffer* up, DType dtype, int64_t count,
                               Stream* stream) {
    RETURN_IF_ERROR(need_bf16(dtype, "silu_mul"));
    const size_t bytes = static_cast<size_t>(count) * 2;
    RETURN_IF_ERROR(need(dst, device_, bytes, "dst"));
    RETURN_IF_ERROR(need(gate, device_, bytes, "gate"));
    RETURN_IF_ERROR(need(up, device_, bytes, "up"));
    void* s = nullptr;
    RETURN_IF_ERROR(native(stream, &s));
    RETURN_IF_ERROR(select());
    HAI_STATUS(hai_silu_mul_bf16(dst->data(), gate->data(), up->data(), count, s), "silu_mul");
    return Status::OK();
}

Status MI355XBackend::partial_rope(Buffer* dst, const Buffer* src, DType dtype, int64_t seq_len, int64_t num_heads,
                                   int64_t head_dim, int64_t rope_head_dim, int64_t position_offset, float base,
                                   Stream* stream) {
    RETURN_IF_ERROR(need_bf16(dtype, "partial_rope"));
    const size_t bytes = static_cast<size_t>(seq_len * num_heads * head_dim) * 2;
    RETURN_IF_ERROR(need(dst, device_, bytes, "dst"));
    RETURN_IF_ERROR(need(src, device_, bytes, "src"));
    if (position_offset < 0 || rope_head_dim < 0 || rope_head_dim > head_dim || rope_head_dim % 2 != 0)
        return invalid("partial_rope arguments");
    void* s = nullptr;
    RETURN_IF_ERROR(native(stream, &s));
    RETURN_IF_ERROR(select());
    std::lock_guard<std::mutex> lock(mu_);
    const RopeTable* t = nullptr;
    RETURN_IF_ERROR(rope_table(rope_head_dim, base, position_offset + seq_len, &t));
    HAI_STATUS(hai_partial_rope_bf16(dst->data(), src->data(), seq_len, num_heads, head_dim, rope_head_dim, t->cos,
                                     t->sin, t->positions, position_offset, s),
               "partial_rope");
    return Status::OK();
}

Status MI355XBackend::q_gate_rmsnorm_rope(Buffer* query_dst, Buffer* gate_dst, const Buffer* source,
                                          const Buffer* query_weight, DType dtype, int64_t seq_len,
                                          int64_t num_query_heads, int64_t head_dim, int64_t rope_head_dim,
                                          int64_t position_offset, float rope_base, float eps,
                                          bool add_unit_offset, Stream* stream) {
    RETURN_IF_ERROR(need_bf16(dtype, "q_gate_rmsnorm_rope"));
    if (!add_unit_offset) return not_impl("q_gate_rmsnorm_rope without the (w + 1) offset");
    const size_t out_bytes = static_cast<size_t>(seq_len * num_query_heads * head_dim) * 2;
    RETURN_IF_ERROR(need(query_dst, device_, out_bytes, "query_dst"));
    RETURN_IF_ERROR(need(gate_dst, device_, out_bytes, "gate_dst"));
    RETURN_IF_ERROR(need(source, device_, 2 * out_bytes, "source"));
    RETURN_IF_ERROR(need(query_weight, device_, static_cast<size_t>(head_dim) * 2, "query_weight"));
    if (position_offset < 0 || position_offset > std::numeric_limits<int32_t>::max() - seq_len)
        return invalid("q_gate_rmsnorm_rope position");
    void* s = nullptr;
    RETURN_IF_ERROR(native(stream, &s));
    RETURN_IF_ERROR(select());
    std::lock_guard<std::mutex> lock(mu_);
    const RopeTable* t = nullptr;
    RETURN_IF_ERROR(rope_table(rope_head_dim, rope_base, position_offset + seq_len, &t));
    HAI_STATUS(hai_q_gate_rmsnorm_rope_bf16(query_dst->data(), gate_dst->data(), source->data(),
                                            num_query_heads * 2 * head_dim, query_weight->data(), t->cos, t->sin,
                                            t->positions, 1, seq_len, num_query_heads, head_dim, rope_head_dim,
                                            nullptr, static_cast<int32_t>(position_offset), eps, s),
               "q_gate_rmsnorm_rope");
    return Status::OK();
}

Status MI355XBackend::append_kv_cache(Buffer* key_cache, Buffer* value_cache, const Buffer* key,
                                      const Buffer* value, DType dtype, int64_t token_count, int64_t num_kv_heads,
                                      int64_t head_dim, int64_t cache_offset, int64_t cache_capacity,
                                      Stream* stream) {
    RETURN_IF_ERROR(need_bf16(dtype, "append_kv_cache"));
    const int64_t row = num_kv_heads * head_dim;
    RETURN_IF_ERROR(need(key_cache, device_, static_cast<size_t>(cache_capacity * row) * 2, "key_cache"));
    RETURN_IF_ERROR(need(value_cache, device_, static_cast<size_t>(cache_capacity * row) * 2, "value_cache"));
    RETURN_IF_ERROR(need(key, device_, static_cast<size_t>(token_count * row) * 2, "key"));
    RETURN_IF_ERROR(need(value, device_, static_cast<size_t>(token_count * row) * 2, "value"));
    if (token_count < 0 || cache_offset < 0 || cache_offset + token_count > cache_capacity ||
        cache_offset > std::numeric_limits<int32_t>::max())
        return invalid("KV cache append overflows the cache capacity");
    void* s = nullptr;
    RETURN_IF_ERROR(native(stream, &s));
    RETURN_IF_ERROR(select());
    HAI_STATUS(hai_append_kv_bf16(key_cache->data(), value_cache->data(), cache_capacity, key->data(),
                                  value->data(), 1, token_count, row, nullptr, static_cast<int32_t>(cache_offset),
                                  s),
               "append_kv_cache");
    return Status::OK();
}

// causal_gqa_kernel (hip_kernels.hip:223-293, launcher :1379-1415): query s of
// [seq_len, nq, D] attends key / value rows 0..s of [seq_len, nkv, D], the
// output gated by sigmoid(gate).  The key / value tensors are a cache of
// seq_len rows, so this is the verify attention over it with every row a
// query; queries run in chunks of kCausalChunk rows (chunk [t0, t0 + n) over
// cache length t0 + n), which bounds the split-KV scratch and leaves each
// query's keys, and so every bit, as one call would.
Status MI355XBackend::causal_gqa(Buffer* dst, const Buffer* query, const Buffer* key, const Buffer* value,
                                 const Buffer* gate, DType dtype, int64_t seq_len, int64_t num_query_heads,
                                 int64_t num_kv_heads, int64_t head_dim, Stream* stream) {
    RETURN_IF_ERROR(need_bf16(dtype, "causal_gqa"));
    if (seq_len <= 0 || seq_len > std::numeric_limits<int32_t>::max()) return invalid("causal_gqa length");
    const int64_t qrow = num_query_heads * head_dim;
    const size_t q_bytes = static_cast<size_t>(seq_len * qrow) * 2;
    const size_t kv_bytes = static_cast<size_t>(seq_len * num_kv_heads * head_dim) * 2;
    RETURN_IF_ERROR(need(dst, device_, q_bytes, "dst"));
    RETURN_IF_ERROR(need(query, device_, q_bytes, "query"));
    RETURN_IF_ERROR(need(key, device_, kv_bytes, "key"));
    RETURN_IF_ERROR(need(value, device_, kv_bytes, "value"));
    if (gate != nullptr) RETURN_IF_ERROR(need(gate, device_, q_bytes, "gate"));
    void* s = nullptr;
    RETURN_IF_ERROR(native(stream, &s));
    RETURN_IF_ERROR(select());
    std::lock_guard<std::mutex> lock(mu_);
    constexpr int64_t kCausalChunk = 64;
    void* ws = nullptr;
    RETURN_IF_ERROR(scratch(gqa_, hai_gqa_scratch_bytes(1, std::min(kCausalChunk, seq_len), num_query_heads,
                                                        head_dim, seq_len),
                            &ws));
    auto* out = static_cast<uint16_t*>(dst->data());
    const auto* q = static_cast<const uint16_t*>(query->data());
    const auto* g = gate ? static_cast<const uint16_t*>(gate->data()) : nullptr;
    for (int64_t t0 = 0; t0 < seq_len; t0 += kCausalChunk) {
        const int64_t n = std::min(kCausalChunk, seq_len - t0);
        const int64_t len = t0 + n;
        HAI_STATUS(hai_gqa_verify_bf16(out + t0 * qrow, q + t0 * qrow, g ? g + t0 * qrow : nullptr, key->data(),
                                       value->data(), seq_len, ws, 1, n, num_query_heads, num_kv_heads, head_dim,
                                       nullptr, static_cast<int32_t>(len), len, s),
                   "causal_gqa");
    }
    return Status::OK();
}

Status MI355XBackend::cached_gqa(Buffer* dst, const Buffer* query, const Buffer* key_cache,
                                 const Buffer* value_cache, const Buffer* gate, DType dtype, int64_t query_len,
                                 int64_t cache_len, int64_t num_query_heads, int64_t num_kv_heads, int64_t head_dim,
                                 Stream* stream) {
    RETURN_IF_ERROR(need_bf16(dtype, "cached_gqa"));
    const size_t q_bytes = static_cast<size_t>(query_len * num_query_heads * head_dim) * 2;
    const size_t c_bytes = static_cast<size_t>(cache_len * num_kv_heads * head_dim) * 2;
    RETURN_IF_ERROR(need(dst, device_, q_bytes, "dst"));
    RETURN_IF_ERROR(need(query, device_, q_bytes, "query"));
    RETURN_IF_ERROR(need(key_cache, device_, c_bytes, "key_cache"));
    RETURN_IF_ERROR(need(value_cache, device_, c_bytes, "value_cache"));
    if (gate != nullptr) RETURN_IF_ERROR(need(gate, device_, q_bytes, "gate"));
    if (query_len <= 0 || cache_len < query_len || cache_len > std::numeric_limits<int32_t>::max())
        return invalid("cached_gqa lengths");
    void* s = nullptr;
    RETURN_IF_ERROR(native(stream, &s));
    RETURN_IF_ERROR(select());
    std::lock_guard<std::mutex> lock(mu_);
    void* ws = nullptr;
    RETURN_IF_ERROR(scratch(gqa_, hai_gqa_scratch_bytes(1, query_len, num_query_heads, head_dim, cache_len), &ws));
    HAI_STATUS(hai_gqa_verify_bf16(dst->data(), query->data(), gate ? gate->data() : nullptr, key_cache->data(),
                                   value_cache->data(), cache_len, ws, 1, query_len, num_query_heads, num_kv_heads,
                                   head_dim, nullptr, static_cast<int32_t>(cache_len), cache_len, s),
               "cached_gqa");
    return Status::OK();
}

// cached_gqa_current_token_kernel (hip_kernels.hip:396-478): attend one query row
// to cache rows 0..cache_len-2 plus the current K/V row, and store the
// current row into the caches at cache_len-1 (the reference kernel's store,
// :466-476, which attention.cc:561-571 relies on: it only advances the
// cache length afterwards).  The row is stored first and the attention
// runs over the cache in place; the result is the same because row
// cache_len-1 then is the current row.  The caches are declared const by
// the Backend virtual, as in the reference, and written all the same.
Status MI355XBackend::cached_gqa_with_current_token(Buffer* dst, const Buffer* query, const Buffer* key_cache,
                                                    const Buffer* value_cache, const Buffer* current_key,
                                                    const Buffer* current_value, const Buffer* gate, DType dtype,
                                                    int64_t cache_len, int64_t num_query_heads,
                                                    int64_t num_kv_heads, int64_t head_dim, Stream* stream) {
    RETURN_IF_ERROR(need_bf16(dtype, "cached_gqa_with_current_token"));
    if (cache_len < 1 || cache_len > std::numeric_limits<int32_t>::max()) return invalid("cache length");
    const int64_t row = num_kv_heads * head_dim;
    const size_t q_bytes = static_cast<size_t>(num_query_heads * head_dim) * 2;
    const size_t cache_bytes = static_cast<size_t>(cache_len * row) * 2;
    RETURN_IF_ERROR(need(dst, device_, q_bytes, "dst"));
    RETURN_IF_ERROR(need(query, device_, q_bytes, "query"));
    RETURN_IF_ERROR(need(key_cache, device_, cache_bytes, "key_cache"));
    RETURN_IF_ERROR(need(value_cache, device_, cache_bytes, "value_cache"));
    RETURN_IF_ERROR(need(current_key, device_, static_cast<size_t>(row) * 2, "current_key"));
    RETURN_IF_ERROR(need(current_value, device_, static_cast<size_t>(row) * 2, "current_value"));
    if (gate != nullptr) RETURN_IF_ERROR(need(gate, device_, q_bytes, "gate"));
    void* s = nullptr;
    RETURN_IF_ERROR(native(stream, &s));
    RETURN_IF_ERROR(select());
    std::lock_guard<std::mutex> lock(mu_);
    void* kc = const_cast<void*>(key_cache->data());
    void* vc = const_cast<void*>(value_cache->data());
    HAI_STATUS(hai_append_kv_bf16(kc, vc, cache_len, current_key->data(), current_value->data(), 1, 1, row, nullptr,
                                  static_cast<int32_t>(cache_len - 1), s),
               "current K/V row store");
    void* ws = nullptr;
    RETURN_IF_ERROR(scratch(gqa_, hai_gqa_scratch_bytes(1, 1, num_query_heads, head_dim, cache_len), &ws));
    HAI_STATUS(hai_gqa_verify_bf16(dst->data(), query->data(), gate ? gate->data() : nullptr, kc, vc, cache_len, ws,
                                   1, 1, num_query_heads, num_kv_heads, head_dim, nullptr,
                                   static_cast<int32_t>(cache_len), cache_len, s),
               "cached_gqa_with_current_token");
    return Status::OK();
}

Status MI355XBackend::deltanet_grouped_conv(Buffer* query, Buffer* key, Buffer* value, Buffer* conv_state,
                                            const Buffer* grouped_qkv, const Buffer* weight, DType dtype,
                                            int64_t token_count, int64_t num_qk_heads, int64_t num_value_heads,
                                            int64_t key_head_dim, int64_t value_head_dim, int64_t kernel_size,
                                            Stream* stream) {
    RETURN_IF_ERROR(need_bf16(dtype, "deltanet_grouped_conv"));
    const int64_t kw = num_qk_heads * key_head_dim, vw = num_value_heads * value_head_dim, C = 2 * kw + vw;
    RETURN_IF_ERROR(need(query, device_, static_cast<size_t>(token_count * kw) * 2, "query"));
    RETURN_IF_ERROR(need(key, device_, static_cast<size_t>(token_count * kw) * 2, "key"));
    RETURN_IF_ERROR(need(value, device_, static_cast<size_t>(token_count * vw) * 2, "value"));
    RETURN_IF_ERROR(need(conv_state, device_, static_cast<size_t>(C * (kernel_size - 1)) * 2, "conv_state"));
    RETURN_IF_ERROR(need(grouped_qkv, device_, static_cast<size_t>(token_count * C) * 2, "grouped_qkv"));
    RETURN_IF_ERROR(need(weight, device_, static_cast<size_t>(C * kernel_size) * 2, "weight"));
    void* s = nullptr;
    RETURN_IF_ERROR(native(stream, &s));
    RETURN_IF_ERROR(select());
    HAI_STATUS(hai_deltanet_conv_bf16(query->data(), key->data(), value->data(), conv_state->data(),
                                      grouped_qkv->data(), weight->data(), token_count, num_qk_heads,
                                      num_value_heads, key_head_dim, value_head_dim, kernel_size, s),
               "deltanet_grouped_conv");
    return Status::OK();
}

Status MI355XBackend::deltanet_recurrent(Buffer* dst, Buffer* recurrent_state, const Buffer* query,
                                         const Buffer* key, const Buffer* value, const Buffer* a, const Buffer* beta,
                                         const Buffer* a_log, const Buffer* dt_bias, const Buffer* norm_weight,
                                         const Buffer* z, DType dtype, int64_t token_count, int64_t num_qk_heads,
                                         int64_t num_value_heads, int64_t key_head_dim, int64_t value_head_dim,
                                         float eps, Stream* stream) {
    RETURN_IF_ERROR(need_bf16(dtype, "deltanet_recurrent"));
    const int64_t kw = num_qk_heads * key_head_dim, vw = num_value_heads * value_head_dim;
    const size_t vb = static_cast<size_t>(token_count * vw) * 2;
    const size_t sb = static_cast<size_t>(token_count * num_value_heads) * 2;
    RETURN_IF_ERROR(need(dst, device_, vb, "dst"));
    RETURN_IF_ERROR(need(recurrent_state, device_,
                         static_cast<size_t>(num_value_heads * key_head_dim * value_head_dim) * 4, "state"));
    RETURN_IF_ERROR(need(query, device_, static_cast<size_t>(token_count * kw) * 2, "query"));
    RETURN_IF_ERROR(need(key, device_, static_cast<size_t>(token_count * kw) * 2, "key"));
    RETURN_IF_ERROR(need(value, device_, vb, "value"));
    RETURN_IF_ERROR(need(a, device_, sb, "a"));
    RETURN_IF_ERROR(need(beta, device_, sb, "beta"));
    RETURN_IF_ERROR(need(a_log, device_, static_cast<size_t>(num_value_heads) * 2, "a_log"));
    RETURN_IF_ERROR(need(dt_bias, device_, static_cast<size_t>(num_value_heads) * 2, "dt_bias"));
    RETURN_IF_ERROR(need(norm_weight, device_, static_cast<size_t>(value_head_dim) * 2, "norm_weight"));
    RETURN_IF_ERROR(need(z, device_, vb, "z"));
    void* s = nullptr;
    RETURN_IF_ERROR(native(stream, &s));
    RETURN_IF_ERROR(select());
    HAI_STATUS(hai_deltanet_recurrent_bf16(dst->data(), at<float>(recurrent_state), query->data(), key->data(),
                                           value->data(), a->data(), beta->data(), a_log->data(), dt_bias->data(),
                                           norm_weight->data(), z->data(), token_count, num_qk_heads,
                                           num_value_heads, key_head_dim, value_head_dim, eps, s),
               "deltanet_recurrent");
    return Status::OK();
}

Status MI355XBackend::argmax_rows(Buffer* dst, const Buffer* src, DType dtype, int64_t rows, int64_t columns,
                                  Stream* stream) {
    RETURN_IF_ERROR(need_bf16(dtype, "argmax_rows"));
    if (rows <= 0 || columns <= 0) return invalid("argmax dimensions");
    RETURN_IF_ERROR(need(dst, device_, static_cast<size_t>(rows) * 8, "dst"));
    RETURN_IF_ERROR(need(src, device_, static_cast<size_t>(rows * columns) * 2, "src"));
    void* s = nullptr;
    RETURN_IF_ERROR(native(stream, &s));
    RETURN_IF_ERROR(select());
    std::lock_guard<std::mutex> lock(mu_);
    void* ws = nullptr;
    RETURN_IF_ERROR(scratch(argmax_, hai_argmax_scratch_bytes(rows, columns), &ws));
    HAI_STATUS(hai_argmax_rows_bf16(at<int64_t>(dst), src->data(), columns, rows, columns, ws, s), "argmax_rows");
    return Status::OK();
}

Status MI355XBackend::argmax_last_row(Buffer* dst, const Buffer* src, DType dtype, int64_t rows, int64_t columns,
                                      Stream* stream) {
    RETURN_IF_ERROR(need_bf16(dtype, "argmax_last_row"));
    if (rows <= 0 || columns <= 0) return invalid("argmax dimensions");
    RETURN_IF_ERROR(need(dst, device_, 8, "dst"));
    RETURN_IF_ERROR(need(src, device_, static_cast<size_t>(rows * columns) * 2, "src"));
    void* s = nullptr;
    RETURN_IF_ERROR(native(stream, &s));
    RETURN_IF_ERROR(select());
    std::lock_guard<std::mutex> lock(mu_);
    void* ws = nullptr;
    RETURN_IF_ERROR(scratch(argmax_, hai_argmax_scratch_bytes(1, columns), &ws));
    HAI_STATUS(hai_argmax_rows_bf16(at<int64_t>(dst), at<uint16_t>(src) + (rows - 1) * columns, columns, 1,
                                    columns, ws, s),
               "argmax_last_row");
    return Status::OK();
}

void MI355XBackend::register_kernels() {
    if (kernels_registered_) return;
    kernels_registered_ = true;
    // The keys the reference's HIP backend provides (hip_backend.cc:1517-1531).
    auto noop = [](const std::vector<Tensor*>&, std::vector<Tensor*>&) { return Status::OK(); };
    for (DeviceType t : {DeviceType::DiscreteGPU, DeviceType::IntegratedGPU})
        ops::KernelRegistry::instance().register_kernel(ops::KernelKey{"noop", t, DType::FP32}, noop);
}

// ---- registration ------------------------------------------------------------------

namespace {

std::unique_ptr<Backend> create_mi355x_backend(const Device& device) {
    auto b = std::make_unique<MI355XBackend>(device);
    b->register_kernels();
    return b;
}

HYBRIDAI_REGISTER_BACKEND(hip, create_mi355x_backend);

}  // namespace

void InitializeHipBackend() { (void)BackendRegistry::instance().has_backend("hip"); }

}  // namespace hybridai
