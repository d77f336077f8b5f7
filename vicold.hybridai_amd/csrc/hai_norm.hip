// hai_norm.hip -- row-wise small ops of the verify step: RMSNorm, the fused
// Q/gate RMSNorm+RoPE, the fused K RMSNorm+RoPE+cache append, embedding
// gather and the elementwise residual / SwiGLU kernels used by the Backend
// adaptor.  One 64-lane wave owns one row so that every reduction follows the
// canonical L64 order.
#include "hai_common.h"
#include "hai_device.h"

namespace {

using namespace hai;

// rmsnorm_kernel (hip_kernels.hip:105-137): 4 rows per 256-thread block.
// Rows up to 8192 wide are loaded once into registers (all loads in flight
// before the first use), reduced in L64 order and normalised from registers.
template <int NC>
__global__ __launch_bounds__(256) void rmsnorm_kernel(uint16_t* __restrict__ y, int64_t ldy,
                                                      const uint16_t* __restrict__ x, int64_t ldx,
                                                      const uint16_t* __restrict__ w, int64_t rows,
                                                      int H, float eps, float off) {
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    rmsnorm_row_wave<NC>(y + row * ldy, x + row * ldx, w, H, eps, off, lane);
}

// Rotate-half on the normalised values held in LDS (row of D fp32), first R
// dims: out_p = x c - y s, out_{p+R/2} = y c + x s (hip_kernels.hip:213-220).
__device__ __forceinline__ float rope_at(const float* row, int d, int R, const float* cs,
                                         const float* sn) {
    if (d >= R) return row[d];
    const int half = R / 2;
    const int p = d < half ? d : d - half;
    const float xv = row[p];
    const float yv = row[p + half];
    if (d < half) return fma_(xv, cs[p], -(yv * sn[p]));
    return fma_(yv, cs[p], xv * sn[p]);
}

// q_gate_rmsnorm_rope_kernel (hip_fused_kernels.hip:87-141): one wave per
// (row, head); q is normalised with (w+1), rotated and stored once; the gate
// half is copied.  `pair` = row * nq + head of this wave; qn = its LDS row.
// Every load that does not depend on the position (q, norm weight, gate,
// the cache length) is issued first, the rotation factors as soon as the
// length arrives.
__device__ __forceinline__ void q_gate_rmsnorm_rope_pair(
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ g_out, const uint16_t* __restrict__ src, int64_t ld_src,
    const uint16_t* __restrict__ wq, const float* __restrict__ rc, const float* __restrict__ rs, int64_t rope_pos,
    int B, int T, int nq, int D, int R, const int32_t* lens, int pos_add, float eps, int64_t pair, float* qn) {
    const int lane = threadIdx.x & 63;
    const bool active = pair < static_cast<int64_t>(B) * T * nq;
    int64_t m = 0;
    int h = 0;
    HeadPiece gp{{0u, 0u, 0u, 0u}};
    float cv[kRopeSlots], sv[kRopeSlots];
    if (active) {
        m = pair / nq;
        h = static_cast<int>(pair % nq);
        const uint16_t* s = src + m * ld_src + static_cast<int64_t>(h) * 2 * D;
        const HeadPiece qp = load_piece(s, D, lane);
        gp = load_piece(s + D, D, lane);
        float wv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) wv[e] = lane * 8 + e < D ? bf2f(wq[lane * 8 + e]) : 0.0f;
        const int b = static_cast<int>(m / T);
        const int t = static_cast<int>(m % T);
        int64_t pos = static_cast<int64_t>(lens ? lens[b] : 0) + pos_add + t;
        pos = pos < 0 ? 0 : (pos >= rope_pos ? rope_pos - 1 : pos);
        load_rope(cv, sv, rc + pos * (R / 2), rs + pos * (R / 2), D, R, lane);
        const float inv = 1.0f / csqrt(piece_sumsq(qp) / static_cast<float>(D) + eps);
        if (lane * 8 < D) {
#pragma unroll
            for (int e = 0; e < 8; ++e) qn[lane * 8 + e] = (qp.at(e) * inv) * (wv[e] + 1.0f);
        }
    }
    __syncthreads();
    if (!active) return;
    uint16_t* qo = q_out + (m * nq + h) * D;
    uint16_t* go = g_out + (m * nq + h) * D;
#pragma unroll
    for (int i = 0; i < kRopeSlots; ++i) {
        const int d = lane + 64 * i;
        if (d < D) qo[d] = f2bf(rope_reg(qn, d, R, cv[i], sv[i]));
    }
    if (lane * 8 < D) {
#pragma unroll
        for (int e = 0; e < 8; ++e) go[lane * 8 + e] = static_cast<uint16_t>(gp.w[e >> 1] >> (16 * (e & 1)));
    }
}

// K path (attention.cc:459-464) fused with append_kv_cache_kernel
// (hip_kernels.hip:295-308): kn = bf16(k*inv*(w+1)), then bf16(rope(kn))
// written to the cache row; V copied unchanged.  `pair` = row * nkv + head.
__device__ __forceinline__ void kv_rmsnorm_rope_append_pair(
    uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int64_t cap, const uint16_t* __restrict__ sk,
    const uint16_t* __restrict__ sv, int64_t ld_src, const uint16_t* __restrict__ wk, const float* __restrict__ rc,
    const float* __restrict__ rs, int64_t rope_pos, int B, int T, int nkv, int D, int R, const int32_t* lens,
    int pos_add, float eps, int64_t pair, float* kn) {
    const int lane = threadIdx.x & 63;
    const bool active = pair < static_cast<int64_t>(B) * T * nkv;
    int64_t m = 0;
    int h = 0;
    int64_t pos = -1;
    HeadPiece vp{{0u, 0u, 0u, 0u}};
    float cv[kRopeSlots], svr[kRopeSlots];
    if (active) {
        m = pair / nkv;
        h = static_cast<int>(pair % nkv);
        const uint16_t* s = sk + m * ld_src + static_cast<int64_t>(h) * D;
        const HeadPiece kp = load_piece(s, D, lane);
        vp = load_piece(sv + m * ld_src + static_cast<int64_t>(h) * D, D, lane);
        float wv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) wv[e] = lane * 8 + e < D ? bf2f(wk[lane * 8 + e]) : 0.0f;
        const int b = static_cast<int>(m / T);
        const int t = static_cast<int>(m % T);
        pos = static_cast<int64_t>(lens ? lens[b] : 0) + pos_add + t;
        const int64_t rp = pos < 0 ? 0 : (pos >= rope_pos ? rope_pos - 1 : pos);
        load_rope(cv, svr, rc + rp * (R / 2), rs + rp * (R / 2), D, R, lane);
        const float inv = 1.0f / csqrt(piece_sumsq(kp) / static_cast<float>(D) + eps);
        if (lane * 8 < D) {
#pragma unroll
            for (int e = 0; e < 8; ++e) kn[lane * 8 + e] = bfr((kp.at(e) * inv) * (wv[e] + 1.0f));
        }
    }
    __syncthreads();
    if (!active) return;
    if (pos < 0 || pos >= cap) return;
    const int b = static_cast<int>(m / T);
    const int64_t dst = ((static_cast<int64_t>(b) * cap + pos) * nkv + h) * D;
#pragma unroll
    for (int i = 0; i < kRopeSlots; ++i) {
        const int d = lane + 64 * i;
        if (d < D) kc[dst + d] = f2bf(rope_reg(kn, d, R, cv[i], svr[i]));
    }
    if (lane * 8 < D) {
#pragma unroll
        for (int e = 0; e < 8; ++e) vc[dst + lane * 8 + e] = static_cast<uint16_t>(vp.w[e >> 1] >> (16 * (e & 1)));
    }
}

__global__ __launch_bounds__(256) void q_gate_rmsnorm_rope_kernel(
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ g_out, const uint16_t* __restrict__ src,
    int64_t ld_src, const uint16_t* __restrict__ wq, const float* __restrict__ rc,
    const float* __restrict__ rs, int64_t rope_pos, int B, int T, int nq, int D, int R,
    const int32_t* lens, int pos_add, float eps) {
    __shared__ float qn[4][kMaxHeadDim];
    const int wave = threadIdx.x >> 6;
    q_gate_rmsnorm_rope_pair(q_out, g_out, src, ld_src, wq, rc, rs, rope_pos, B, T, nq, D, R, lens, pos_add, eps,
                             static_cast<int64_t>(blockIdx.x) * 4 + wave, qn[wave]);
}

__global__ __launch_bounds__(256) void kv_rmsnorm_rope_append_kernel(
    uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int64_t cap,
    const uint16_t* __restrict__ sk, const uint16_t* __restrict__ sv, int64_t ld_src,
    const uint16_t* __restrict__ wk, const float* __restrict__ rc, const float* __restrict__ rs,
    int64_t rope_pos, int B, int T, int nkv, int D, int R, const int32_t* lens, int pos_add,
    float eps) {
    __shared__ float kn[4][kMaxHeadDim];
    const int wave = threadIdx.x >> 6;
    kv_rmsnorm_rope_append_pair(kc, vc, cap, sk, sv, ld_src, wk, rc, rs, rope_pos, B, T, nkv, D, R, lens, pos_add,
                                eps, static_cast<int64_t>(blockIdx.x) * 4 + wave, kn[wave]);
}

// Both of the above in one launch: the first qblocks blocks take the q /
// gate heads, the rest the K / V heads (the two are independent).
struct QkvNormArgs {
    uint16_t *q_out, *g_out, *kc, *vc;
    const uint16_t *src, *wq, *wk;
    int64_t ld_src, cap, rope_pos;
    const float *rc, *rs;
    const int32_t* lens;
    int B, T, nq, nkv, D, R, pos_add, qblocks;
    float eps;
};
__global__ __launch_bounds__(256) void qkv_rmsnorm_rope_append_kernel(QkvNormArgs a) {
    __shared__ float buf[4][kMaxHeadDim];
    const int wave = threadIdx.x >> 6;
    if (static_cast<int>(blockIdx.x) < a.qblocks) {
        q_gate_rmsnorm_rope_pair(a.q_out, a.g_out, a.src, a.ld_src, a.wq, a.rc, a.rs, a.rope_pos, a.B, a.T, a.nq,
                                 a.D, a.R, a.lens, a.pos_add, a.eps, static_cast<int64_t>(blockIdx.x) * 4 + wave,
                                 buf[wave]);
    } else {
        const uint16_t* sk = a.src + 2 * static_cast<int64_t>(a.nq) * a.D;
        const uint16_t* sv = sk + static_cast<int64_t>(a.nkv) * a.D;
        kv_rmsnorm_rope_append_pair(a.kc, a.vc, a.cap, sk, sv, a.ld_src, a.wk, a.rc, a.rs, a.rope_pos, a.B, a.T,
                                    a.nkv, a.D, a.R, a.lens, a.pos_add, a.eps,
                                    static_cast<int64_t>(blockIdx.x - a.qblocks) * 4 + wave, buf[wave]);
    }
}

__global__ void append_kv_kernel(uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int64_t cap,
                                 const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int B,
                                 int T, int64_t row_width, const int32_t* lens, int pos_add) {
    const int64_t total = static_cast<int64_t>(B) * T * row_width;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t m = i / row_width;
        const int64_t c = i - m * row_width;
        const int b = static_cast<int>(m / T);
        const int t = static_cast<int>(m % T);
        const int64_t pos = static_cast<int64_t>(lens ? lens[b] : 0) + pos_add + t;
        if (pos < 0 || pos >= cap) continue;
        const int64_t dst = (static_cast<int64_t>(b) * cap + pos) * row_width + c;
        kc[dst] = k[i];
        vc[dst] = v[i];
    }
}

__global__ void add_kernel(uint16_t* y, const uint16_t* a, const uint16_t* b, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        y[i] = f2bf(bf2f(a[i]) + bf2f(b[i]));
}

__global__ void silu_mul_kernel(uint16_t* y, const uint16_t* g, const uint16_t* u, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        y[i] = f2bf(csilu(bf2f(g[i])) * bf2f(u[i]));
}

// embedding_gather_kernel (hip_kernels.hip:88-103): one block per id.
// VEC (rows of a multiple of 8 elements, 16-byte aligned): 16-byte pieces,
// kEmbUnroll per thread requested before the first store, so a row costs
// one round trip to memory instead of one per element a thread copies.
constexpr int kEmbUnroll = 4;
template <bool VEC>
__global__ void embedding_kernel(uint16_t* __restrict__ y, const uint16_t* __restrict__ table,
                                 const int64_t* __restrict__ ids, int64_t V, int64_t H) {
    const int64_t r = blockIdx.x;
    const int64_t id = ids[r];
    const bool ok = id >= 0 && id < V;
    if constexpr (VEC) {
        const int64_t n8 = H >> 3;
        const uint4* src = reinterpret_cast<const uint4*>(table + (ok ? id : 0) * H);
        uint4* dst = reinterpret_cast<uint4*>(y + r * H);
        for (int64_t k0 = threadIdx.x; k0 < n8; k0 += kEmbUnroll * blockDim.x) {
            uint4 v[kEmbUnroll];
#pragma unroll
            for (int u = 0; u < kEmbUnroll; ++u) {
                const int64_t k = k0 + u * static_cast<int64_t>(blockDim.x);
                v[u] = ok && k < n8 ? src[k] : make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int u = 0; u < kEmbUnroll; ++u) {
                const int64_t k = k0 + u * static_cast<int64_t>(blockDim.x);
                if (k < n8) dst[k] = v[u];
            }
        }
    } else {
        for (int64_t k = threadIdx.x; k < H; k += blockDim.x)
            y[r * H + k] = ok ? table[id * H + k] : static_cast<uint16_t>(0);
    }
}

// partial_rope_kernel (hip_kernels.hip:192-221): rotate-half on the first R
// dims of every head, the rest copied; one thread per element.
__global__ void partial_rope_kernel(uint16_t* __restrict__ dst, const uint16_t* __restrict__ src, int64_t n,
                                    int heads, int D, int R, const float* __restrict__ rc,
                                    const float* __restrict__ rs, int64_t rope_pos, int64_t pos0) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int d = static_cast<int>(i % D);
        if (d >= R) {
            dst[i] = src[i];
            continue;
        }
        const int64_t head = i / D;
        const int64_t t = head / heads;
        int64_t pos = pos0 + t;
        pos = pos < 0 ? 0 : (pos >= rope_pos ? rope_pos - 1 : pos);
        const int half = R / 2;
        const int p = d < half ? d : d - half;
        const float* cs = rc + pos * half;
        const float* sn = rs + pos * half;
        const float xv = bf2f(src[head * D + p]);
        const float yv = bf2f(src[head * D + p + half]);
        dst[i] = f2bf(d < half ? fma_(xv, cs[p], -(yv * sn[p])) : fma_(yv, cs[p], xv * sn[p]));
    }
}

unsigned grid_for(int64_t n) {
    const int64_t b = (n + 255) / 256;
    return static_cast<unsigned>(b < 1 ? 1 : (b > 65536 ? 65536 : b));
}

}  // namespace

extern "C" {

int hai_rmsnorm_bf16(void* y, int64_t ldy, const void* x, int64_t ldx, const void* w, int64_t rows,
                     int64_t H, float eps, int unit_offset, void* stream) {
    if (y == nullptr || x == nullptr || w == nullptr) return invalid("rmsnorm: null pointer");
    if (rows < 0 || H <= 0 || H % 8 != 0 || ldx % 8 != 0 || ldy % 8 != 0 || ldx < H || ldy < H)
        return invalid("rmsnorm: shape (need H%8==0, 8-aligned strides)");
    if (!aligned16(x) || !aligned16(y) || !aligned16(w)) return invalid("rmsnorm: 16-byte alignment");
    if (H > 16 * 512) return invalid("rmsnorm: H above 8192");
    if (rows == 0) return HAI_OK;
    const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
    auto* yy = static_cast<uint16_t*>(y);
    const auto* xx = static_cast<const uint16_t*>(x);
    const auto* ww = static_cast<const uint16_t*>(w);
    const float off = unit_offset ? 1.0f : 0.0f;
    const auto s = as_stream(stream);
    if (H <= 512) rmsnorm_kernel<1><<<grid, dim3(256), 0, s>>>(yy, ldy, xx, ldx, ww, rows, int(H), eps, off);
    else if (H <= 2048) rmsnorm_kernel<4><<<grid, dim3(256), 0, s>>>(yy, ldy, xx, ldx, ww, rows, int(H), eps, off);
    else if (H <= 6144) rmsnorm_kernel<12><<<grid, dim3(256), 0, s>>>(yy, ldy, xx, ldx, ww, rows, int(H), eps, off);
    else rmsnorm_kernel<16><<<grid, dim3(256), 0, s>>>(yy, ldy, xx, ldx, ww, rows, int(H), eps, off);
    return launched("rmsnorm_kernel");
}

int hai_add_bf16(void* y, const void* a, const void* b, int64_t n, void* stream) {
    if (y == nullptr || a == nullptr || b == nullptr || n < 0) return invalid("add");
    if (n == 0) return HAI_OK;
    add_kernel<<<dim3(grid_for(n)), dim3(256), 0, as_stream(stream)>>>(
        static_cast<uint16_t*>(y), static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b), n);
    return launched("add_kernel");
}

int hai_silu_mul_bf16(void* y, const void* g, const void* u, int64_t n, void* stream) {
    if (y == nullptr || g == nullptr || u == nullptr || n < 0) return invalid("silu_mul");
    if (n == 0) return HAI_OK;
    silu_mul_kernel<<<dim3(grid_for(n)), dim3(256), 0, as_stream(stream)>>>(
        static_cast<uint16_t*>(y), static_cast<const uint16_t*>(g), static_cast<const uint16_t*>(u), n);
    return launched("silu_mul_kernel");
}

int hai_embedding_gather_bf16(void* y, const void* table, const int64_t* ids, int64_t n_ids, int64_t V,
                              int64_t H, void* stream) {
    if (y == nullptr || table == nullptr || ids == nullptr || n_ids < 0 || V <= 0 || H <= 0)
        return invalid("embedding_gather");
    if (n_ids == 0) return HAI_OK;
    const dim3 grid(static_cast<unsigned>(n_ids));
    if (H % 8 == 0 && aligned16(y) && aligned16(table))
        embedding_kernel<true><<<grid, dim3(256), 0, as_stream(stream)>>>(
            static_cast<uint16_t*>(y), static_cast<const uint16_t*>(table), ids, V, H);
    else
        embedding_kernel<false><<<grid, dim3(256), 0, as_stream(stream)>>>(
            static_cast<uint16_t*>(y), static_cast<const uint16_t*>(table), ids, V, H);
    return launched("embedding_kernel");
}

int hai_q_gate_rmsnorm_rope_bf16(void* q_out, void* gate_out, const void* src, int64_t ld_src,
                                 const void* q_norm, const float* rope_cos, const float* rope_sin,
                                 int64_t rope_positions, int64_t B, int64_t T, int64_t nq, int64_t D,
                                 int64_t R, const int32_t* lens, int32_t pos_add, float eps,
                                 void* stream) {
    if (q_out == nullptr || gate_out == nullptr || src == nullptr || q_norm == nullptr ||
        rope_cos == nullptr || rope_sin == nullptr)
        return invalid("q_gate_rmsnorm_rope: null pointer");
    if (B < 0 || T < 0 || nq <= 0 || D <= 0 || D % 8 != 0 || D > kMaxHeadDim || R < 0 || R > D ||
        R % 2 != 0 || ld_src < 2 * nq * D || rope_positions <= 0)
        return invalid("q_gate_rmsnorm_rope: shape");
    if (!aligned16(src) || ld_src % 8 != 0) return invalid("q_gate_rmsnorm_rope: alignment");
    const int64_t pairs = B * T * nq;
    if (pairs == 0) return HAI_OK;
    q_gate_rmsnorm_rope_kernel<<<dim3(static_cast<unsigned>((pairs + 3) / 4)), dim3(256), 0,
                                 as_stream(stream)>>>(
        static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(gate_out), static_cast<const uint16_t*>(src),
        ld_src, static_cast<const uint16_t*>(q_norm), rope_cos, rope_sin, rope_positions, int(B), int(T),
        int(nq), int(D), int(R), lens, pos_add, eps);
    return launched("q_gate_rmsnorm_rope_kernel");
}

int hai_kv_rmsnorm_rope_append_bf16(void* k_cache, void* v_cache, int64_t cap, const void* src_k,
                                    const void* src_v, int64_t ld_src, const void* k_norm,
                                    const float* rope_cos, const float* rope_sin, int64_t rope_positions,
                                    int64_t B, int64_t T, int64_t nkv, int64_t D, int64_t R,
                                    const int32_t* lens, int32_t pos_add, float eps, void* stream) {
    if (k_cache == nullptr || v_cache == nullptr || src_k == nullptr || src_v == nullptr ||
        k_norm == nullptr || rope_cos == nullptr || rope_sin == nullptr)
        return invalid("kv_rmsnorm_rope_append: null pointer");
    if (cap <= 0 || B < 0 || T < 0 || nkv <= 0 || D <= 0 || D % 8 != 0 || D > kMaxHeadDim || R < 0 ||
        R > D || R % 2 != 0 || ld_src < nkv * D || rope_positions <= 0)
        return invalid("kv_rmsnorm_rope_append: shape");
    if (!aligned16(src_k) || !aligned16(src_v) || ld_src % 8 != 0)
        return invalid("kv_rmsnorm_rope_append: alignment (src_k, src_v 16-byte aligned, ld_src % 8 == 0)");
    const int64_t pairs = B * T * nkv;
    if (pairs == 0) return HAI_OK;
    kv_rmsnorm_rope_append_kernel<<<dim3(static_cast<unsigned>((pairs + 3) / 4)), dim3(256), 0,
                                    as_stream(stream)>>>(
        static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), cap,
        static_cast<const uint16_t*>(src_k), static_cast<const uint16_t*>(src_v), ld_src,
        static_cast<const uint16_t*>(k_norm), rope_cos, rope_sin, rope_positions, int(B), int(T), int(nkv),
        int(D), int(R), lens, pos_add, eps);
    return launched("kv_rmsnorm_rope_append_kernel");
}

int hai_qkv_rmsnorm_rope_append_bf16(void* q_out, void* gate_out, void* k_cache, void* v_cache, int64_t cap,
                                     const void* src, int64_t ld_src, const void* q_norm, const void* k_norm,
                                     const float* rope_cos, const float* rope_sin, int64_t rope_positions,
                                     int64_t B, int64_t T, int64_t nq, int64_t nkv, int64_t D, int64_t R,
                                     const int32_t* lens, int32_t pos_add, float eps, void* stream) {
    if (q_out == nullptr || gate_out == nullptr || k_cache == nullptr || v_cache == nullptr || src == nullptr ||
        q_norm == nullptr || k_norm == nullptr || rope_cos == nullptr || rope_sin == nullptr)
        return invalid("qkv_rmsnorm_rope_append: null pointer");
    if (cap <= 0 || B < 0 || T < 0 || nq <= 0 || nkv <= 0 || D <= 0 || D % 8 != 0 || D > kMaxHeadDim || R < 0 ||
        R > D || R % 2 != 0 || ld_src < (2 * nq + 2 * nkv) * D || rope_positions <= 0)
        return invalid("qkv_rmsnorm_rope_append: shape");
    if (!aligned16(src) || ld_src % 8 != 0) return invalid("qkv_rmsnorm_rope_append: alignment");
    const int64_t qpairs = B * T * nq, kvpairs = B * T * nkv;
    if (qpairs == 0) return HAI_OK;
    QkvNormArgs a;
    a.q_out = static_cast<uint16_t*>(q_out);
    a.g_out = static_cast<uint16_t*>(gate_out);
    a.kc = static_cast<uint16_t*>(k_cache);
    a.vc = static_cast<uint16_t*>(v_cache);
    a.src = static_cast<const uint16_t*>(src);
    a.wq = static_cast<const uint16_t*>(q_norm);
    a.wk = static_cast<const uint16_t*>(k_norm);
    a.ld_src = ld_src;
    a.cap = cap;
    a.rope_pos = rope_positions;
    a.rc = rope_cos;
    a.rs = rope_sin;
    a.lens = lens;
    a.B = int(B);
    a.T = int(T);
    a.nq = int(nq);
    a.nkv = int(nkv);
    a.D = int(D);
    a.R = int(R);
    a.pos_add = pos_add;
    a.qblocks = int((qpairs + 3) / 4);
    a.eps = eps;
    const unsigned blocks = static_cast<unsigned>(a.qblocks + (kvpairs + 3) / 4);
    qkv_rmsnorm_rope_append_kernel<<<dim3(blocks), dim3(256), 0, as_stream(stream)>>>(a);
    return launched("qkv_rmsnorm_rope_append_kernel");
}

int hai_partial_rope_bf16(void* dst, const void* src, int64_t T, int64_t heads, int64_t D, int64_t R,
                          const float* rope_cos, const float* rope_sin, int64_t rope_positions, int64_t pos0,
                          void* stream) {
    if (dst == nullptr || src == nullptr || rope_cos == nullptr || rope_sin == nullptr)
        return invalid("partial_rope: null pointer");
    if (T < 0 || heads <= 0 || D <= 0 || R < 0 || R > D || R % 2 != 0 || rope_positions <= 0)
        return invalid("partial_rope: shape");
    if (pos0 < 0 || pos0 + T > rope_positions) return invalid("partial_rope: positions beyond the RoPE table");
    const int64_t n = T * heads * D;
    if (n == 0) return HAI_OK;
    partial_rope_kernel<<<dim3(grid_for(n)), dim3(256), 0, as_stream(stream)>>>(
        static_cast<uint16_t*>(dst), static_cast<const uint16_t*>(src), n, int(heads), int(D), int(R), rope_cos,
        rope_sin, rope_positions, pos0);
    return launched("partial_rope_kernel");
}

int hai_append_kv_bf16(void* k_cache, void* v_cache, int64_t cap, const void* k, const void* v, int64_t B,
                       int64_t T, int64_t row_width, const int32_t* lens, int32_t pos_add, void* stream) {
    if (k_cache == nullptr || v_cache == nullptr || k == nullptr || v == nullptr || cap <= 0 || B < 0 ||
        T < 0 || row_width <= 0)
        return invalid("append_kv");
    if (lens == nullptr && (pos_add < 0 || pos_add + T > cap))
        return invalid("append_kv: rows exceed cache capacity");
    const int64_t n = B * T * row_width;
    if (n == 0) return HAI_OK;
    append_kv_kernel<<<dim3(grid_for(n)), dim3(256), 0, as_stream(stream)>>>(
        static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), cap,
        static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v), int(B), int(T), row_width, lens,
        pos_add);
    return launched("append_kv_kernel");
}

}  // extern "C"
