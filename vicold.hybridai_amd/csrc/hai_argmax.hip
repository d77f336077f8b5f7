// hai_argmax.hip -- per-row argmax of bf16 logits and the fused greedy
// acceptance of the verify step (argmax_rows_kernel, hip_kernels.hip:
// 1243-1274; acceptance generator.cc:909-1021).
//
// Ties: the reference's CPU scan keeps the first maximum, NaN never wins and
// -inf never wins (generator.cc:343-360); the reference GPU kernel's result
// depends on thread striding.  Here each candidate is a 64-bit key
// (ordered value << 32 | ~index) reduced with max, which yields the CPU
// answer for any launch shape; invalid values map to key 0 (index 0).
#include "hai_common.h"
#include "hai_device.h"

namespace {

using namespace hai;

constexpr int kSlices = 64;  // partial blocks per row
constexpr int kMaxAcceptRows = 64;  // verify rows (k + 1) per sequence

__device__ __forceinline__ uint64_t make_key(float v, int64_t idx) {
    if (!(v > __uint_as_float(0xff800000u))) return 0ull;  // NaN or -inf
    uint32_t u = __float_as_uint(v);
    if ((u & 0x7fffffffu) == 0u) u = 0u;  // -0 ties with +0
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (static_cast<uint64_t>(ord) << 32) | static_cast<uint64_t>(0xffffffffu - static_cast<uint32_t>(idx));
}
__device__ __forceinline__ int64_t key_index(uint64_t key) {
    if (key == 0ull) return 0;
    return static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(key & 0xffffffffull));
}
__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int s) {
    const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), s, 64);
    const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), s, 64);
    return (static_cast<uint64_t>(hi) << 32) | lo;
}
__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, uint64_t* sh) {
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) {
        const uint64_t o = shfl_xor_u64(v, s);
        v = o > v ? o : v;
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) sh[wave] = v;
    __syncthreads();
    uint64_t best = 0ull;
    for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) best = sh[w] > best ? sh[w] : best;
    __syncthreads();
    return best;
}

// Elements per slice of a row: a multiple of 8, so that with VEC (rows
// 16-byte aligned) every slice starts on a 16-byte boundary.
__host__ __device__ constexpr int64_t slice_len(int64_t V) { return ((V + kSlices - 1) / kSlices + 7) / 8 * 8; }
constexpr int kArgmaxUnroll = 2;  // 16-byte pieces per thread requested together

// The largest key of the row's slices (64 lanes, one key each): the row's
// argmax, independent of the slice order.
__device__ __forceinline__ uint64_t wave_max_slices(const uint64_t* __restrict__ part, int64_t r, int lane) {
    uint64_t v = lane < kSlices ? part[r * kSlices + lane] : 0ull;
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) {
        const uint64_t o = shfl_xor_u64(v, s);
        v = o > v ? o : v;
    }
    return v;
}

// One block per (slice, row).  VEC: 16-byte pieces of 8 logits, the
// thread's pieces requested before the first compare (one round trip to
// the just-written logits instead of one per element).
template <bool VEC>
__global__ __launch_bounds__(256) void argmax_partial_kernel(uint64_t* __restrict__ part,
                                                             const uint16_t* __restrict__ logits,
                                                             int64_t ld, int64_t V) {
    __shared__ uint64_t sh[4];
    const int64_t row = blockIdx.y;
    const int slice = blockIdx.x;
    const int64_t per = slice_len(V);
    const int64_t start = static_cast<int64_t>(slice) * per;
    const int64_t end = min(V, start + per);
    const uint16_t* lr = logits + row * ld;
    uint64_t best = 0ull;
    if constexpr (VEC) {
        const int64_t npc = start < end ? (end - start + 7) / 8 : 0;  // pieces, the last one possibly ragged
        for (int64_t p0 = threadIdx.x; p0 < npc; p0 += kArgmaxUnroll * blockDim.x) {
            uint4 v[kArgmaxUnroll];
#pragma unroll
            for (int u = 0; u < kArgmaxUnroll; ++u) {
                const int64_t p = p0 + u * static_cast<int64_t>(blockDim.x);
                const int64_t i0 = start + 8 * p;
                v[u] = p < npc && i0 + 8 <= end ? *reinterpret_cast<const uint4*>(lr + i0)
                                                : make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int u = 0; u < kArgmaxUnroll; ++u) {
                const int64_t p = p0 + u * static_cast<int64_t>(blockDim.x);
                if (p >= npc) continue;
                const int64_t i0 = start + 8 * p;
                if (i0 + 8 <= end) {
                    const uint32_t w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float f = __uint_as_float((e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16));
                        const uint64_t k = make_key(f, i0 + e);
                        best = k > best ? k : best;
                    }
                } else {
                    for (int64_t i = i0; i < end; ++i) {
                        const uint64_t k = make_key(bf2f(lr[i]), i);
                        best = k > best ? k : best;
                    }
                }
            }
        }
    } else {
        for (int64_t i = start + threadIdx.x; i < end; i += blockDim.x) {
            const uint64_t k = make_key(bf2f(lr[i]), i);
            best = k > best ? k : best;
        }
    }
    best = block_max_u64(best, sh);
    if (threadIdx.x == 0) part[row * kSlices + slice] = best;
}

// One wave per row.
__global__ __launch_bounds__(256) void argmax_final_kernel(int64_t* __restrict__ out,
                                                           const uint64_t* __restrict__ part, int64_t rows) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const uint64_t best = wave_max_slices(part, r, threadIdx.x & 63);
    if ((threadIdx.x & 63) == 0) out[r] = key_index(best);
}

// Copies H elements (16-byte pieces when both rows allow them, each
// thread's pieces requested before its first store).
__device__ __forceinline__ void copy_row(uint16_t* __restrict__ dst, const uint16_t* __restrict__ src, int64_t H) {
    const bool vec = (H & 7) == 0 && ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 15) == 0;
    if (vec) {
        const int64_t n8 = H >> 3;
        for (int64_t k0 = threadIdx.x; k0 < n8; k0 += 4 * blockDim.x) {
            uint4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int64_t k = k0 + u * static_cast<int64_t>(blockDim.x);
                v[u] = k < n8 ? reinterpret_cast<const uint4*>(src)[k] : make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int64_t k = k0 + u * static_cast<int64_t>(blockDim.x);
                if (k < n8) reinterpret_cast<uint4*>(dst)[k] = v[u];
            }
        }
        return;
    }
    for (int64_t k = threadIdx.x; k < H; k += blockDim.x) dst[k] = src[k];
}

// One block per sequence b: the final argmax of its T verify rows, its
// accepted prefix, the committed-length update and its hidden-row copies.
__global__ __launch_bounds__(256) void verify_accept_kernel(
    const uint64_t* __restrict__ part, const uint16_t* __restrict__ hidden, int64_t H,
    const int64_t* __restrict__ ids, const int32_t* n_draft, int B, int T, int64_t* __restrict__ preds,
    int32_t* __restrict__ result, int32_t* target_len, int32_t* mtp_len, int64_t* __restrict__ next,
    uint16_t* rec_hidden, uint16_t* h_prev) {
    __shared__ int64_t pred_sh[kMaxAcceptRows];
    __shared__ int acc_sh, full_sh;
    const int b = blockIdx.x;
    const int lane = threadIdx.x & 63;
    for (int t = threadIdx.x >> 6; t < T; t += blockDim.x >> 6) {  // one wave per verify row
        const int64_t r = static_cast<int64_t>(b) * T + t;
        const int64_t p = key_index(wave_max_slices(part, r, lane));
        if (lane == 0) {
            preds[r] = p;
            pred_sh[t] = p;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const int k = n_draft ? n_draft[b] : T - 1;
        int a = 0;
        while (a < k && pred_sh[a] == ids[static_cast<int64_t>(b) * T + 1 + a]) ++a;
        const int full = a == k ? 1 : 0;
        result[b * 4 + 0] = a;
        result[b * 4 + 1] = full;
        result[b * 4 + 2] = static_cast<int32_t>(ids[static_cast<int64_t>(b) * T]);
        result[b * 4 + 3] = static_cast<int32_t>(pred_sh[a]);
        if (target_len) target_len[b] += a + 1;
        if (mtp_len && !full) mtp_len[b] -= k - a;
        next[b] = pred_sh[a];
        acc_sh = a;
        full_sh = full;
    }
    __syncthreads();
    if (hidden == nullptr) return;
    const uint16_t* src = hidden + (static_cast<int64_t>(b) * T + acc_sh) * H;
    if (rec_hidden) copy_row(rec_hidden + b * H, src, H);
    if (h_prev && full_sh) copy_row(h_prev + b * H, src, H);
}

__global__ void add_i32_kernel(int32_t* dst, const int32_t* delta, int32_t add, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) dst[i] += (delta ? delta[i] : 0) + add;
}

__global__ void copy_i64_strided_kernel(int64_t* dst, int64_t ds, const int64_t* src, int64_t ss, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) dst[i * ds] = src[i * ss];
}

// One block per sequence; only the sequences whose round ended in a
// rejection (result[b*4+1] == 0) take the correction row's outcome.
__global__ void correction_commit_kernel(const int32_t* __restrict__ result, const int64_t* __restrict__ corr_next,
                                         const uint16_t* __restrict__ corr_hidden, int64_t H, int64_t* next,
                                         uint16_t* h_prev, int32_t* target_len, int32_t* mtp_len) {
    const int b = blockIdx.x;
    if (result[b * 4 + 1] != 0) return;
    copy_row(h_prev + b * H, corr_hidden + b * H, H);
    if (threadIdx.x == 0) {
        next[b] = corr_next[b];
        target_len[b] += 1;
        mtp_len[b] += 1;
    }
}

// Counts draft i of a chained proposal per sequence.  Sequence b drafts
// again while every earlier draft of the round counted (ndraft[b] == i), its
// cap allows (i < cap[b]) and the candidate its previous draft wrote
// (vids[b*T + i]) is no end-of-sequence id: the reference keeps an EOS
// candidate as a proposal and ends the chain after it (generator.cc:845-847).
// Draft 0 starts every count.
__global__ void draft_chain_count_kernel(int64_t i, const int64_t* __restrict__ vids, int64_t T,
                                         const int32_t* __restrict__ cap, const int64_t* __restrict__ eos,
                                         int64_t n_eos, int32_t* ndraft, int64_t B) {
    const int64_t b = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= B) return;
    if (i == 0) {
        ndraft[b] = cap[b] > 0 ? 1 : 0;
        return;
    }
    if (ndraft[b] != i || i >= cap[b]) return;
    const int64_t tok = vids[b * T + i];
    for (int64_t e = 0; e < n_eos; ++e)
        if (eos[e] == tok) return;
    ndraft[b] = static_cast<int32_t>(i + 1);
}

void launch_partial(uint64_t* part, const uint16_t* logits, int64_t ld, int64_t V, int64_t rows, hipStream_t s) {
    const dim3 grid(kSlices, static_cast<unsigned>(rows));
    if (ld % 8 == 0 && aligned16(logits))
        argmax_partial_kernel<true><<<grid, dim3(256), 0, s>>>(part, logits, ld, V);
    else
        argmax_partial_kernel<false><<<grid, dim3(256), 0, s>>>(part, logits, ld, V);
}

}  // namespace

extern "C" {

int hai_draft_chain_count(int64_t i, const int64_t* vids, int64_t T, const int32_t* cap, const int64_t* eos,
                          int64_t n_eos, int32_t* ndraft, int64_t B, void* stream) {
    if (vids == nullptr || cap == nullptr || ndraft == nullptr || (eos == nullptr && n_eos > 0) || n_eos < 0 ||
        B < 0 || T < 2 || i < 0 || i >= T - 1)
        return invalid("draft_chain_count");
    if (B == 0) return HAI_OK;
    draft_chain_count_kernel<<<dim3(static_cast<unsigned>((B + 255) / 256)), dim3(256), 0, as_stream(stream)>>>(
        i, vids, T, cap, eos, n_eos, ndraft, B);
    return launched("draft_chain_count_kernel");
}

int hai_add_i32(int32_t* dst, const int32_t* delta, int32_t add, int64_t n, void* stream) {
    if (dst == nullptr || n < 0) return invalid("add_i32");
    if (n == 0) return HAI_OK;
    add_i32_kernel<<<dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, as_stream(stream)>>>(dst, delta, add,
                                                                                                        n);
    return launched("add_i32_kernel");
}

int hai_copy_i64_strided(int64_t* dst, int64_t dst_stride, const int64_t* src, int64_t src_stride, int64_t n,
                         void* stream) {
    if (dst == nullptr || src == nullptr || n < 0) return invalid("copy_i64_strided");
    if (n == 0) return HAI_OK;
    copy_i64_strided_kernel<<<dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, as_stream(stream)>>>(
        dst, dst_stride, src, src_stride, n);
    return launched("copy_i64_strided_kernel");
}

int hai_correction_commit_bf16(const int32_t* result, const int64_t* corr_next, const void* corr_hidden, int64_t H,
                               int64_t B, int64_t* next, void* h_prev, int32_t* target_len, int32_t* mtp_len,
                               void* stream) {
    if (result == nullptr || corr_next == nullptr || corr_hidden == nullptr || next == nullptr ||
        h_prev == nullptr || target_len == nullptr || mtp_len == nullptr || B < 0 || H <= 0)
        return invalid("correction_commit");
    if (B == 0) return HAI_OK;
    correction_commit_kernel<<<dim3(static_cast<unsigned>(B)), dim3(256), 0, as_stream(stream)>>>(
        result, corr_next, static_cast<const uint16_t*>(corr_hidden), H, next, static_cast<uint16_t*>(h_prev),
        target_len, mtp_len);
    return launched("correction_commit_kernel");
}

size_t hai_argmax_scratch_bytes(int64_t rows, int64_t V) {
    (void)V;
    return static_cast<size_t>(rows < 1 ? 1 : rows) * kSlices * sizeof(uint64_t);
}

int hai_argmax_rows_bf16(int64_t* out, const void* logits, int64_t ld, int64_t rows, int64_t V,
                         void* scratch, void* stream) {
    if (out == nullptr || logits == nullptr || scratch == nullptr || rows < 0 || V <= 0 || ld < V ||
        V > 0xfffffffell)
        return invalid("argmax_rows");
    if (rows == 0) return HAI_OK;
    const auto s = as_stream(stream);
    launch_partial(static_cast<uint64_t*>(scratch), static_cast<const uint16_t*>(logits), ld, V, rows, s);
    int rc = launched("argmax_partial_kernel");
    if (rc != HAI_OK) return rc;
    argmax_final_kernel<<<dim3(static_cast<unsigned>((rows + 3) / 4)), dim3(256), 0, s>>>(
        out, static_cast<const uint64_t*>(scratch), rows);
    return launched("argmax_final_kernel");
}

int hai_verify_argmax_accept_bf16(const void* logits, int64_t V, const void* hidden, int64_t H,
                                  const int64_t* ids, const int32_t* n_draft, int64_t B, int64_t T,
                                  int64_t* preds, int32_t* result, int32_t* target_len, int32_t* mtp_len,
                                  int64_t* next, void* rec_hidden, void* h_prev, void* scratch,
                                  void* stream) {
    if (logits == nullptr || ids == nullptr || preds == nullptr || result == nullptr || next == nullptr ||
        scratch == nullptr)
        return invalid("verify_argmax_accept: null pointer");
    if (B <= 0 || B > 64 || T <= 0 || T > kMaxAcceptRows || V <= 0 || V > 0xfffffffell ||
        (hidden != nullptr && H <= 0))
        return invalid("verify_argmax_accept: shape (1 <= B <= 64, 1 <= T <= 64)");
    const auto s = as_stream(stream);
    launch_partial(static_cast<uint64_t*>(scratch), static_cast<const uint16_t*>(logits), V, V, B * T, s);
    int rc = launched("argmax_partial_kernel");
    if (rc != HAI_OK) return rc;
    verify_accept_kernel<<<dim3(static_cast<unsigned>(B)), dim3(256), 0, s>>>(
        static_cast<const uint64_t*>(scratch), static_cast<const uint16_t*>(hidden), H, ids, n_draft, int(B),
        int(T), preds, result, target_len, mtp_len, next, static_cast<uint16_t*>(rec_hidden),
        static_cast<uint16_t*>(h_prev));
    return launched("verify_accept_kernel");
}

}  // extern "C"
