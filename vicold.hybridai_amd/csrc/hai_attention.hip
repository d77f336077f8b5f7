// hai_attention.hip -- multi-query gated GQA verify over the KV cache
// (replaces cached_gqa_head256_wave64_kernel, hip_kernels.hip:759-844, and
// the T=1 variant at :567-675).
//
// The reference walks every key serially in one wave per (head, query).
// Here the keys are split into fixed 64-key chunks by absolute index:
//   pass 1 (one block per chunk x group of queries of one KV head x
//     sequence): the chunk's K and V tiles are staged in LDS with all loads
//     in flight at once; the waves take the group's queries in turn: lane =
//     key computes the score with a sequential fma over D, the chunk max and
//     the exp-sum are wave reductions, and P.V is a sequential fma over the
//     chunk's keys with lane = pair of output dims; a wave carries up to six
//     queries at once, so each K / V element is unpacked once for all of
//     them.  The group is every query
//     of the KV head (all T x nq/nkv of them: K and V are read once) when the
//     chunks alone give the grid enough blocks (long caches, batches), else
//     four queries per block;
//   pass 2 (one wave per query): chunk partials are merged against the
//     global max in chunk order (loads batched eight chunks deep), then
//     divided, gated and stored.
// The chunking is by absolute key index, so a query's result does not depend
// on T, on the batch or on how many blocks run: verify rows and replayed
// rows are bit-identical, and the CPU oracle follows the same order.
#include "hai_common.h"
#include "hai_device.h"

namespace {

using namespace hai;

constexpr int kChunk = 64;
constexpr int kWaves = 4;
// chunk grid (chunks x KV heads x sequences) from which a block serves every
// query of its KV head (measured on MI355X: the C2 shape, 256 chunk blocks,
// 35.9 -> 27.0 us; C3 and C4 unchanged)
constexpr int64_t kFullGroupBlocks = 256;

__host__ __device__ constexpr int64_t partial_stride(int D) { return D + 2; }

// grid (chunk, query group x KV head, sequence): the block stages one 64-key
// chunk of one KV head and serves qpb of that head's queries.  Each wave takes
// up to QG of them at a time: a K or V element is unpacked once and feeds the
// QG queries' fma chains (each chain keeps its own sequential order).
template <int D, int QG, int W>
__global__ __launch_bounds__(64 * W) void gqa_partial_kernel(
    float* __restrict__ scratch, const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, int64_t cap, int T, int nq, int nkv, const int32_t* lens,
    int len_add, int nchunk, float scale, int qpb) {
    constexpr int KP = D / 2 + 4;          // dword stride of a staged K row (16-byte pad)
    constexpr int VP = D / 2;              // dword stride of a staged V row
    constexpr int ROW16 = D / 8;           // 16-byte pieces per row
    constexpr int NT = 64 * W;             // threads
    constexpr int NLD = kChunk * ROW16 / NT;   // pieces per thread and tile
    constexpr int QPL = D / 64;            // query elements per lane
    constexpr int NPAIR = (D / 2 + 63) / 64;  // value pairs per lane (lanes past D / 2 idle when D = 64)
    static_assert(NLD >= 1 && kChunk * ROW16 % NT == 0, "tile must split over the block");
    __shared__ uint32_t Ks[kChunk * KP];
    __shared__ uint32_t Vs[kChunk * VP];
    __shared__ __align__(16) float Qs[W][QG][D];
    __shared__ __align__(16) float Ps[W][QG][kChunk];

    const int chunk = blockIdx.x;
    const int kvh = blockIdx.y % nkv;
    const int qgrp = blockIdx.y / nkv;
    const int b = blockIdx.z;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = wave_index();
    const int64_t L = static_cast<int64_t>(lens ? lens[b] : 0) + len_add;
    const int64_t key0 = static_cast<int64_t>(chunk) * kChunk;
    const int group = nq / nkv;
    const int nqry = T * group;
    const int q_begin = qgrp * qpb;
    const int q_end = min(nqry, q_begin + qpb);
    if (key0 >= L || q_begin >= nqry) return;
    const int nkeys = static_cast<int>(min(static_cast<int64_t>(kChunk), L - key0));

    // query qi of this KV head: token qi / group, head kvh * group + qi % group
    auto q_row = [&](int qi) {
        return q + ((static_cast<int64_t>(b) * T + qi / group) * nq + kvh * group + qi % group) * D;
    };
    // pass p of wave w serves queries q_begin + (W p + w) QG + [0, QG)
    uint16_t qv[QG][QPL];
    auto load_q = [&](int base) {
#pragma unroll
        for (int qq = 0; qq < QG; ++qq)
            if (base + qq < q_end) {
                const uint16_t* qrow = q_row(base + qq);
#pragma unroll
                for (int r = 0; r < QPL; ++r) qv[qq][r] = qrow[lane + 64 * r];
            }
    };
    // The wave's first queries are loaded alongside the K / V tiles.
    load_q(q_begin + wave * QG);

    // Stage the chunk's K and V rows: every load is issued before the first
    // LDS store; rows past the cache length read as zeros (buffer range).
    {
        const int64_t off0 = ((static_cast<int64_t>(b) * cap + key0) * nkv + kvh) * D;
        const uint32_t bytes = static_cast<uint32_t>((static_cast<int64_t>(nkeys - 1) * nkv * D + D) * 2);
        const __amdgpu_buffer_rsrc_t rk = make_rsrc(kc + off0, bytes);
        const __amdgpu_buffer_rsrc_t rv = make_rsrc(vc + off0, bytes);
        u32x4 kd[NLD], vd[NLD];
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const int e = tid + NT * i;
            const int j = e / ROW16;
            const uint32_t off = static_cast<uint32_t>((j * nkv * D + (e % ROW16) * 8) * 2);
            kd[i] = bload(rk, off, 0);
            vd[i] = bload(rv, off, 0);
        }
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const int e = tid + NT * i;
            const int j = e / ROW16;
            const int p = (e % ROW16) * 4;
            *reinterpret_cast<u32x4*>(Ks + j * KP + p) = kd[i];
            *reinterpret_cast<u32x4*>(Vs + j * VP + p) = vd[i];
        }
    }
    __syncthreads();

    auto wave_sync = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    for (int base = q_begin + wave * QG; base < q_end; base += W * QG) {
        const int nw = min(QG, q_end - base);
#pragma unroll
        for (int qq = 0; qq < QG; ++qq)
#pragma unroll
            for (int r = 0; r < QPL; ++r) Qs[wave][qq][lane + 64 * r] = qq < nw ? bf2f(qv[qq][r]) : 0.0f;
        // the wave's next queries are in flight while these are computed
        if (base + W * QG < q_end) load_q(base + W * QG);
        wave_sync();

        // Scores: lane = key, sequential fma over D for every query.
        float s[QG];
#pragma unroll
        for (int qq = 0; qq < QG; ++qq) s[qq] = 0.0f;
        {
            const uint32_t* kr = Ks + lane * KP;
#pragma unroll 2
            for (int p = 0; p < D / 2; p += 4) {
                const u32x4 kk = *reinterpret_cast<const u32x4*>(kr + p);
                const float k8[8] = {lo_bf(kk[0]), hi_bf(kk[0]), lo_bf(kk[1]), hi_bf(kk[1]),
                                     lo_bf(kk[2]), hi_bf(kk[2]), lo_bf(kk[3]), hi_bf(kk[3])};
#pragma unroll
                for (int qq = 0; qq < QG; ++qq) {
                    const float4 qa = *reinterpret_cast<const float4*>(&Qs[wave][qq][2 * p]);
                    const float4 qb = *reinterpret_cast<const float4*>(&Qs[wave][qq][2 * p + 4]);
                    float sv = s[qq];
                    sv = fma_(qa.x, k8[0], sv);
                    sv = fma_(qa.y, k8[1], sv);
                    sv = fma_(qa.z, k8[2], sv);
                    sv = fma_(qa.w, k8[3], sv);
                    sv = fma_(qb.x, k8[4], sv);
                    sv = fma_(qb.y, k8[5], sv);
                    sv = fma_(qb.z, k8[6], sv);
                    sv = fma_(qb.w, k8[7], sv);
                    s[qq] = sv;
                }
            }
        }
        // per query: chunk max, exp-sum and probabilities (zero past the causal limit)
        int nj_max = 0;
#pragma unroll
        for (int qq = 0; qq < QG; ++qq) {
            if (qq < nw) {
                const int qi = base + qq;
                const int t = qi / group;
                const int h = kvh * group + qi % group;
                const int64_t qpos = L - T + t;
                const bool valid = lane < nkeys && key0 + lane <= qpos;
                const float sc = s[qq] * scale;
                const float m = wave_max64(valid ? sc : __uint_as_float(0xff800000u));
                const float pr = valid ? cexp(sc - m) : 0.0f;
                const float l = wave_sum64(pr);
                Ps[wave][qq][lane] = pr;
                float* part =
                    scratch + ((((static_cast<int64_t>(b) * T + t) * nq + h) * nchunk) + chunk) * partial_stride(D);
                if (lane == 0) {
                    part[0] = m;
                    part[1] = l;
                }
                const int64_t lim = qpos - key0 + 1;
                const int nj = static_cast<int>(lim < nkeys ? (lim < 0 ? 0 : lim) : nkeys);
                nj_max = max(nj_max, nj);
            } else {
                Ps[wave][qq][lane] = 0.0f;
            }
        }
        wave_sync();

        // P.V: lane owns value pairs (2i, 2i+1), i = lane + 64r; sequential over
        // keys.  Keys past a query's causal limit carry probability 0, and
        // fma(0, v, o) == o for the finite staged values, so running every
        // query to the longest limit does not change a bit.
        float o[QG][NPAIR][2];
#pragma unroll
        for (int qq = 0; qq < QG; ++qq)
#pragma unroll
            for (int r = 0; r < NPAIR; ++r) o[qq][r][0] = o[qq][r][1] = 0.0f;
        const int nj4 = (nj_max + 3) & ~3;
        for (int j0 = 0; j0 < nj4; j0 += 4) {
            float4 p4[QG];
#pragma unroll
            for (int qq = 0; qq < QG; ++qq) p4[qq] = *reinterpret_cast<const float4*>(&Ps[wave][qq][j0]);
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                float vlo[NPAIR], vhi[NPAIR];
#pragma unroll
                for (int r = 0; r < NPAIR; ++r) {
                    const uint32_t vv = lane + 64 * r < D / 2 ? Vs[(j0 + jj) * VP + lane + 64 * r] : 0u;
                    vlo[r] = lo_bf(vv);
                    vhi[r] = hi_bf(vv);
                }
#pragma unroll
                for (int qq = 0; qq < QG; ++qq) {
                    const float pj = jj == 0 ? p4[qq].x : jj == 1 ? p4[qq].y : jj == 2 ? p4[qq].z : p4[qq].w;
#pragma unroll
                    for (int r = 0; r < NPAIR; ++r) {
                        o[qq][r][0] = fma_(pj, vlo[r], o[qq][r][0]);
                        o[qq][r][1] = fma_(pj, vhi[r], o[qq][r][1]);
                    }
                }
            }
        }
#pragma unroll
        for (int qq = 0; qq < QG; ++qq) {
            if (qq < nw) {
                const int qi = base + qq;
                const int t = qi / group;
                const int h = kvh * group + qi % group;
                float* part =
                    scratch + ((((static_cast<int64_t>(b) * T + t) * nq + h) * nchunk) + chunk) * partial_stride(D);
#pragma unroll
                for (int r = 0; r < NPAIR; ++r)
                    if (lane + 64 * r < D / 2)
                        *reinterpret_cast<float2*>(part + 2 + 2 * (lane + 64 * r)) =
                            make_float2(o[qq][r][0], o[qq][r][1]);
            }
        }
        wave_sync();  // Qs / Ps are rewritten by the next pass
    }
}

// One wave per query: chunk partials merged in chunk order against the
// global max, then divided, gated and rounded.
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
    constexpr int64_t PS = partial_stride(D);
    const float* base = scratch + qidx * nchunk * PS;
    float M = __uint_as_float(0xff800000u);
    for (int c = lane; c < nch; c += 64) M = fmaxf(M, base[c * PS]);
    M = wave_max64(M);
    constexpr int PER = D / 64;
    float O[PER];
#pragma unroll
    for (int r = 0; r < PER; ++r) O[r] = 0.0f;
    float Ls = 0.0f;
    for (int c0 = 0; c0 < nch; c0 += 64) {
        const int nt = min(64, nch - c0);
        float w = 0.0f, lc = 0.0f;
        if (lane < nt) {
            const float* part = base + (c0 + lane) * PS;
            w = cexp(part[0] - M);
            lc = part[1];
        }
        for (int cb = 0; cb < nt; cb += 8) {
            float pv[8][PER];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int cc = min(cb + u, nt - 1);
                const float* part = base + (c0 + cc) * PS + 2;
#pragma unroll
                for (int r = 0; r < PER; ++r) pv[u][r] = part[lane + 64 * r];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (cb + u < nt) {
                    const float wc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), cb + u));
                    const float lcc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lc), cb + u));
                    Ls = fma_(lcc, wc, Ls);
#pragma unroll
                    for (int r = 0; r < PER; ++r) O[r] = fma_(pv[u][r], wc, O[r]);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < PER; ++r) {
        const int d = lane + 64 * r;
        float o = O[r] / Ls;
        if (gate != nullptr) o = o * csigmoid(bf2f(gate[qidx * D + d]));
        out[qidx * D + d] = f2bf(o);
    }
}

template <int D>
int launch(uint16_t* out, const uint16_t* q, const uint16_t* gate, const uint16_t* kc, const uint16_t* vc,
           int64_t cap, float* scratch, int B, int T, int nq, int nkv, const int32_t* lens, int len_add,
           int nchunk, hipStream_t s) {
    const float scale = 1.0f / __builtin_sqrtf(static_cast<float>(D));
    // Queries per block: all of the KV head's when the chunks alone fill the
    // GPU (K / V read once), else the fewest multiple of four that does.
    const int nqry = T * (nq / nkv);
    const int64_t base = static_cast<int64_t>(nchunk) * nkv * B;
    const int64_t max_groups = (nqry + kWaves - 1) / kWaves;
    const int64_t want = base >= kFullGroupBlocks ? 1 : (kFullGroupBlocks + base - 1) / base;
    const int64_t groups = want < max_groups ? want : max_groups;
    const int qpb = static_cast<int>(kWaves * ((max_groups + groups - 1) / groups));
    const int qgroups = (nqry + qpb - 1) / qpb;
    // Waves and queries per wave: up to 8 queries per block on 4 waves (two
    // blocks fit a CU), more on 8 waves of up to 3 (one block per CU, the K /
    // V tile shared by all of them); larger groups take several passes.
    const dim3 grid(nchunk, nkv * qgroups, B);
    if (qpb <= 4)
        gqa_partial_kernel<D, 1, 4><<<grid, dim3(256), 0, s>>>(scratch, q, kc, vc, cap, T, nq, nkv, lens, len_add,
                                                               nchunk, scale, qpb);
    else if (qpb <= 8)
        gqa_partial_kernel<D, 2, 4><<<grid, dim3(256), 0, s>>>(scratch, q, kc, vc, cap, T, nq, nkv, lens, len_add,
                                                               nchunk, scale, qpb);
    else if (qpb <= 16)
        gqa_partial_kernel<D, 2, 8><<<grid, dim3(512), 0, s>>>(scratch, q, kc, vc, cap, T, nq, nkv, lens, len_add,
                                                               nchunk, scale, qpb);
    else
        gqa_partial_kernel<D, 3, 8><<<grid, dim3(512), 0, s>>>(scratch, q, kc, vc, cap, T, nq, nkv, lens, len_add,
                                                               nchunk, scale, qpb);
    int rc = launched("gqa_partial_kernel");
    if (rc != HAI_OK) return rc;
    const int64_t nall = static_cast<int64_t>(B) * T * nq;
    gqa_combine_kernel<D><<<dim3(static_cast<unsigned>((nall + 3) / 4)), dim3(256), 0, s>>>(
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
