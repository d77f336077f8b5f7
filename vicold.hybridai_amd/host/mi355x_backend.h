// mi355x_backend.h -- hybridai::Backend for AMD Instinct MI355X (gfx950),
// registered under the name "hip" so that the reference's BackendRegistry
// hands it to every op that asks for a HIP device
// (src/backends/hip/hip_backend_factory.cc:12-19 is the slot it takes).
//
// Every device action goes through the hai_* C ABI (include/hai_kernels.h).
// Implemented natively: memory, streams, events, copies, and the virtuals of
// the speculative verify path -- gemm (bf16 X * W^T, fp32 accumulation),
// add, embedding_gather, rmsnorm, silu_mul, q_gate_rmsnorm_rope,
// partial_rope, append_kv_cache, causal_gqa, cached_gqa, cached_gqa_with_current_token,
// deltanet_grouped_conv, deltanet_recurrent, argmax_last_row, argmax_rows,
// copy_to_offset.  Everything else (other dtypes, FP32 GEMM, the prefill-only
// kernels) returns NotImplemented, which the reference's ops treat as "use
// the CPU reference path" (src/backends/interface/backend.h:116-119).
#pragma once

#include <map>
#include <memory>
#include <mutex>
#include <utility>
#include <vector>

#include "refabi/hybridai_abi.h"

namespace hybridai {

class MI355XBackend final : public Backend {
public:
    explicit MI355XBackend(const Device& device);
    ~MI355XBackend() override;

    const char* name() const noexcept override { return "hip"; }
    Device device() const noexcept override { return device_; }
    bool is_available() const noexcept override;
    std::vector<Device> enumerate_devices() const override;

    std::unique_ptr<Allocator> create_allocator(MemoryType type) override;
    std::unique_ptr<Stream> create_stream() override;
    std::unique_ptr<Event> create_event() override;
    std::shared_ptr<Buffer> create_buffer(size_t size, MemoryType type) override;
    // Bytes the buffer pool of this device and memory type holds for reuse.
    size_t pooled_bytes(MemoryType type) const;

    Status memcpy_h2d(Buffer* dst, const void* src, size_t size, Stream* stream = nullptr) override;
    Status memcpy_d2h(void* dst, const Buffer* src, size_t size, Stream* stream = nullptr) override;
    Status memcpy_d2d(Buffer* dst, const Buffer* src, size_t size, Stream* stream = nullptr) override;
    Status copy(Buffer* dst, const Buffer* src, size_t size, Stream* stream = nullptr) override;
    Status memset(Buffer* dst, int value, size_t size, Stream* stream = nullptr) override;
    Status synchronize() override;

    Status gemm(Buffer* c, const Buffer* a, const Buffer* b, DType c_type, DType a_type, DType b_type,
                DType compute_type, bool trans_a, bool trans_b, int64_t m, int64_t n, int64_t k, float alpha,
                float beta, Stream* stream = nullptr) override;
    Status add(Buffer* dst, const Buffer* lhs, const Buffer* rhs, DType dtype, int64_t count,
               Stream* stream = nullptr) override;
    Status embedding_gather(Buffer* dst, const Buffer* embedding, const Buffer* ids, DType dtype, int64_t num_ids,
                            int64_t vocab_size, int64_t hidden_size, Stream* stream = nullptr) override;
    Status rmsnorm(Buffer* dst, const Buffer* src, const Buffer* weight, DType dtype, int64_t rows,
                   int64_t hidden_size, float eps, bool add_unit_offset, Stream* stream = nullptr) override;
    Status silu_mul(Buffer* dst, const Buffer* gate, const Buffer* up, DType dtype, int64_t count,
                    Stream* stream = nullptr) override;
    Status partial_rope(Buffer* dst, const Buffer* src, DType dtype, int64_t seq_len, int64_t num_heads,
                        int64_t head_dim, int64_t rope_head_dim, int64_t position_offset, float base,
                        Stream* stream = nullptr) override;
    Status append_kv_cache(Buffer* key_cache, Buffer* value_cache, const Buffer* key, const Buffer* value,
                           DType dtype, int64_t token_count, int64_t num_kv_heads, int64_t head_dim,
                           int64_t cache_offset, int64_t cache_capacity, Stream* stream = nullptr) override;
    Status causal_gqa(Buffer* dst, const Buffer* query, const Buffer* key, const Buffer* value, const Buffer* gate,
                      DType dtype, int64_t seq_len, int64_t num_query_heads, int64_t num_kv_heads, int64_t head_dim,
                      Stream* stream = nullptr) override;
    Status cached_gqa(Buffer* dst, const Buffer* query, const Buffer* key_cache, const Buffer* value_cache,
                      const Buffer* gate, DType dtype, int64_t query_len, int64_t cache_len,
                      int64_t num_query_heads, int64_t num_kv_heads, int64_t head_dim,
                      Stream* stream = nullptr) override;
    Status cached_gqa_with_current_token(Buffer* dst, const Buffer* query, const Buffer* key_cache,
                                         const Buffer* value_cache, const Buffer* current_key,
                                         const Buffer* current_value, const Buffer* gate, DType dtype,
                                         int64_t cache_len, int64_t num_query_heads, int64_t num_kv_heads,
                                         int64_t head_dim, Stream* stream = nullptr) override;
    Status deltanet_grouped_conv(Buffer* query, Buffer* key, Buffer* value, Buffer* conv_state,
                                 const Buffer* grouped_qkv, const Buffer* weight, DType dtype, int64_t token_count,
                                 int64_t num_qk_heads, int64_t num_value_heads, int64_t key_head_dim,
                                 int64_t value_head_dim, int64_t kernel_size, Stream* stream = nullptr) override;
    Status deltanet_recurrent(Buffer* dst, Buffer* recurrent_state, const Buffer* query, const Buffer* key,
                              const Buffer* value, const Buffer* a, const Buffer* beta, const Buffer* a_log,
                              const Buffer* dt_bias, const Buffer* norm_weight, const Buffer* z, DType dtype,
                              int64_t token_count, int64_t num_qk_heads, int64_t num_value_heads,
                              int64_t key_head_dim, int64_t value_head_dim, float eps,
                              Stream* stream = nullptr) override;
    Status argmax_last_row(Buffer* dst, const Buffer* src, DType dtype, int64_t rows, int64_t columns,
                           Stream* stream = nullptr) override;
    Status argmax_rows(Buffer* dst, const Buffer* src, DType dtype, int64_t rows, int64_t columns,
                       Stream* stream = nullptr) override;
    void register_kernels() override;
    Status copy_to_offset(Buffer* dst, size_t dst_offset, const Buffer* src, size_t src_offset, size_t size,
                          Stream* stream = nullptr) override;
    Status q_gate_rmsnorm_rope(Buffer* query_dst, Buffer* gate_dst, const Buffer* source,
                               const Buffer* query_weight, DType dtype, int64_t seq_len, int64_t num_query_heads,
                               int64_t head_dim, int64_t rope_head_dim, int64_t position_offset, float rope_base,
                               float eps, bool add_unit_offset, Stream* stream = nullptr) override;

private:
    // Device scratch that grows on demand (guarded by mu_): attention
    // partials, argmax partials, a contiguous K/V copy for the current-token
    // attention, and RoPE tables per (rotary dims, base).
    struct Scratch {
        void* ptr = nullptr;
        size_t bytes = 0;
    };
    struct RopeTable {
        float* cos = nullptr;
        float* sin = nullptr;
        int64_t positions = 0;
    };
    Status select() const;
    Status scratch(Scratch& s, size_t bytes, void** out);
    Status rope_table(int64_t rope_dims, float base, int64_t positions, const RopeTable** out);

    Device device_;
    bool kernels_registered_ = false;
    std::mutex mu_;
    Scratch gqa_, argmax_;
    std::map<std::pair<int64_t, float>, RopeTable> rope_;
};

// Linker anchor: referencing it keeps the registration unit in static links
// (the reference's InitializeBuiltinBackends calls it).
void InitializeHipBackend();

}  // namespace hybridai
