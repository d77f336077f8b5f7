// hai_attention.hip -- multi-query gated GQA verify over the KV cache
// (replaces cached_gqa_head256_wave64_kernel, hip_kernels.hip:759-844, and
// the T=1 variant at :567-675).
//
// The reference walks every key serially in one wave per (head, query).
// Here the keys are split into fixed 64-key chunks by absolute index:
//   pass 1 (one block per chunk x KV head x sequence): the chunk's K and V
//     tiles are staged once in LDS and shared by every query of that KV head
//     (T tokens x nq/nkv heads); lane = key computes the score with a
//     sequential fma over D, the chunk max and the exp-sum are wave
//     reductions, and P.V is a sequential fma over the chunk's keys with
//     lane = output dim;
//   pass 2 (one wave per query): chunk partials are merged against the
//     global max in chunk order, then divided, gated and stored.
// The chunking is by absolute key index, so a query's result does not depend
// on T, on the batch or on how many blocks run: verify rows and replayed
// rows are bit-identical, and the CPU oracle follows the same order.
#include "hai_common.h"
#include "hai_device.h"

namespace {

using namespace hai;

constexpr int kChunk = 64;
constexpr int kQBatch = 32;  // queries processed per pass over the staged tile

__host__ __device__ constexpr int64_t partial_stride(int D) { return D + 2; }

template <int D>
__global__ __launch_bounds__(256) void gqa_partial_kernel(
    float* __restrict__ scratch, const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, int64_t cap, int T, int nq, int nkv, const int32_t* lens,
    int len_add, int nchunk, float scale) {
    constexpr int KP = D / 2 + 1;  // padded dword stride of a K row in LDS
    __shared__ uint32_t Ks[kChunk * KP];
    __shared__ uint16_t Vs[kChunk * D];
    __shared__ float Qs[kQBatch * D];
    __shared__ float Ps[kQBatch * kChunk];

    const int chunk = blockIdx.x;
    const int kvh = blockIdx.y;
    const int b = blockIdx.z;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t L = static_cast<int64_t>(lens ? lens[b] : 0) + len_add;
    const int64_t key0 = static_cast<int64_t>(chunk) * kChunk;
    if (key0 >= L) return;
    const int nkeys = static_cast<int>(min(static_cast<int64_t>(kChunk), L - key0));
    const int group = nq / nkv;
    const int nqry = T * group;

    // Stage K (padded, bf16 pairs) and V tiles of this chunk; rows past L are zero.
    const int64_t seq_base = static_cast<int64_t>(b) * cap;
    for (int e = tid; e < kChunk * (D / 8); e += 256) {
        const int j = e / (D / 8);
        const int d8 = (e % (D / 8)) * 8;
        uint4 kd = make_uint4(0u, 0u, 0u, 0u), vd = kd;
        if (j < nkeys) {
            const int64_t off = ((seq_base + key0 + j) * nkv + kvh) * D + d8;
            kd = *reinterpret_cast<const uint4*>(kc + off);
            vd = *reinterpret_cast<const uint4*>(vc + off);
        }
        uint32_t* kr = Ks + j * KP + d8 / 2;
        kr[0] = kd.x; kr[1] = kd.y; kr[2] = kd.z; kr[3] = kd.w;
        *reinterpret_cast<uint4*>(Vs + j * D + d8) = vd;
    }

    for (int qb = 0; qb < nqry; qb += kQBatch) {
        const int nb = min(kQBatch, nqry - qb);
        __syncthreads();
        for (int e = tid; e < nb * D; e += 256) {
            const int i = e / D;
            const int d = e % D;
            const int qi = qb + i;
            const int t = qi / group;
            const int h = kvh * group + qi % group;
            Qs[i * D + d] = bf2f(q[((static_cast<int64_t>(b) * T + t) * nq + h) * D + d]);
        }
        __syncthreads();
        // Scores, chunk max and exp-sum: one query per wave at a time.
        for (int i = wave; i < nb; i += 4) {
            const int qi = qb + i;
            const int t = qi / group;
            const int h = kvh * group + qi % group;
            const int64_t qpos = L - T + t;
            const int64_t kj = key0 + lane;
            const bool valid = lane < nkeys && kj <= qpos;
            float s = 0.0f;
            if (valid) {
                const uint32_t* kr = Ks + lane * KP;
                const float* qr = Qs + i * D;
#pragma unroll 8
                for (int d2 = 0; d2 < D / 2; ++d2) {
                    const uint32_t kk = kr[d2];
                    s = fma_(qr[2 * d2], lo_bf(kk), s);
                    s = fma_(qr[2 * d2 + 1], hi_bf(kk), s);
                }
                s = s * scale;
            }
            const float m = wave_max64(valid ? s : __uint_as_float(0xff800000u));
            const float p = valid ? cexp(s - m) : 0.0f;
            const float l = wave_sum64(p);
            Ps[i * kChunk + lane] = p;
            if (lane == 0) {
                float* part = scratch + ((((static_cast<int64_t>(b) * T + t) * nq + h) * nchunk) + chunk) *
                                            partial_stride(D);
                part[0] = m;
                part[1] = l;
            }
        }
        __syncthreads();
        // P.V: lane = output dim, sequential over the chunk's keys.
        for (int i = wave; i < nb; i += 4) {
            const int qi = qb + i;
            const int t = qi / group;
            const int h = kvh * group + qi % group;
            const int64_t qpos = L - T + t;
            const int64_t lim = qpos - key0 + 1;
            const int nj = static_cast<int>(lim < nkeys ? (lim < 0 ? 0 : lim) : nkeys);
            float* part = scratch + ((((static_cast<int64_t>(b) * T + t) * nq + h) * nchunk) + chunk) *
                                        partial_stride(D);
            for (int d = lane; d < D; d += 64) {
                float o = 0.0f;
                for (int j = 0; j < nj; ++j) o = fma_(Ps[i * kChunk + j], bf2f(Vs[j * D + d]), o);
                part[2 + d] = o;
            }
        }
    }
}

template <int D>
__global__ __launch_bounds__(256) void gqa_combine_kernel(
    uint16_t* __restrict__ out, const float* __restrict__ scratch, const uint16_t* gate, int B, int T,
    int nq, const int32_t* lens, int len_add, int nchunk) {
    const int lane = threadIdx.x & 63;
    const int64_t qidx = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (qidx >= static_cast<int64_t>(B) * T * nq) return;
    const int64_t m = qidx / nq;
    const int b = static_cast<int>(m / T);
    const int t = static_cast<int>(m % T);
    const int64_t L = static_cast<int64_t>(lens ? lens[b] : 0) + len_add;
    const int64_t qpos = L - T + t;
    const int nch = static_cast<int>(qpos / kChunk) + 1;
    const float* base = scratch + qidx * nchunk * partial_stride(D);
    float M = __uint_as_float(0xff800000u);
    for (int c = lane; c < nch; c += 64) M = fmaxf(M, base[c * partial_stride(D)]);
    M = wave_max64(M);
    constexpr int PER = (D + 63) / 64;
    float O[PER];
#pragma unroll
    for (int r = 0; r < PER; ++r) O[r] = 0.0f;
    float Ls = 0.0f;
    for (int c = 0; c < nch; ++c) {
        const float* part = base + c * partial_stride(D);
        const float wgt = cexp(part[0] - M);
        Ls = fma_(part[1], wgt, Ls);
#pragma unroll
        for (int r = 0; r < PER; ++r) {
            const int d = lane + 64 * r;
            if (d < D) O[r] = fma_(part[2 + d], wgt, O[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < PER; ++r) {
        const int d = lane + 64 * r;
        if (d < D) {
            float o = O[r] / Ls;
            if (gate != nullptr) o = o * csigmoid(bf2f(gate[qidx * D + d]));
            out[qidx * D + d] = f2bf(o);
        }
    }
}

template <int D>
int launch(uint16_t* out, const uint16_t* q, const uint16_t* gate, const uint16_t* kc, const uint16_t* vc,
           int64_t cap, float* scratch, int B, int T, int nq, int nkv, const int32_t* lens, int len_add,
           int nchunk, hipStream_t s) {
    const float scale = 1.0f / __builtin_sqrtf(static_cast<float>(D));
    gqa_partial_kernel<D><<<dim3(nchunk, nkv, B), dim3(256), 0, s>>>(scratch, q, kc, vc, cap, T, nq, nkv,
                                                                     lens, len_add, nchunk, scale);
    int rc = launched("gqa_partial_kernel");
    if (rc != HAI_OK) return rc;
    const int64_t nqry = static_cast<int64_t>(B) * T * nq;
    gqa_combine_kernel<D><<<dim3(static_cast<unsigned>((nqry + 3) / 4)), dim3(256), 0, s>>>(
        out, scratch, gate, B, T, nq, lens, len_add, nchunk);
    return launched("gqa_combine_kernel");
}

}  // namespace

extern "C" {

size_t hai_gqa_scratch_bytes(int64_t B, int64_t T, int64_t nq, int64_t D, int64_t max_len) {
    const int64_t nchunk = (max_len + kChunk - 1) / kChunk;
    return static_cast<size_t>(B * T * nq * (nchunk < 1 ? 1 : nchunk) * partial_stride(int(D))) *
           sizeof(float);
}

int hai_gqa_verify_bf16(void* out, const void* q, const void* gate, const void* k_cache,
                        const void* v_cache, int64_t cap, void* scratch, int64_t B, int64_t T, int64_t nq,
                        int64_t nkv, int64_t D, const int32_t* lens, int32_t len_add, int64_t max_len,
                        void* stream) {
    if (out == nullptr || q == nullptr || k_cache == nullptr || v_cache == nullptr || scratch == nullptr)
        return invalid("gqa_verify: null pointer");
    if (B < 0 || T < 0 || nq <= 0 || nkv <= 0 || nq % nkv != 0 || cap <= 0 || max_len <= 0 ||
        max_len > cap || T > max_len)
        return invalid("gqa_verify: shape");
    if (lens == nullptr && (len_add < T || len_add > max_len))
        return invalid("gqa_verify: cache length must cover the T new rows and stay within max_len");
    if (!aligned16(k_cache) || !aligned16(v_cache)) return invalid("gqa_verify: alignment");
    if (B == 0 || T == 0) return HAI_OK;
    const int nchunk = static_cast<int>((max_len + kChunk - 1) / kChunk);
    const auto s = as_stream(stream);
    auto* o = static_cast<uint16_t*>(out);
    const auto* qq = static_cast<const uint16_t*>(q);
    const auto* g = static_cast<const uint16_t*>(gate);
    const auto* kc = static_cast<const uint16_t*>(k_cache);
    const auto* vc = static_cast<const uint16_t*>(v_cache);
    auto* sc = static_cast<float*>(scratch);
    switch (D) {
        case 64: return launch<64>(o, qq, g, kc, vc, cap, sc, int(B), int(T), int(nq), int(nkv), lens, len_add, nchunk, s);
        case 128: return launch<128>(o, qq, g, kc, vc, cap, sc, int(B), int(T), int(nq), int(nkv), lens, len_add, nchunk, s);
        case 256: return launch<256>(o, qq, g, kc, vc, cap, sc, int(B), int(T), int(nq), int(nkv), lens, len_add, nchunk, s);
        default: return invalid("gqa_verify: head_dim must be 64, 128 or 256");
    }
}

}  // extern "C"
