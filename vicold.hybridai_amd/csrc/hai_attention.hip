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
#include <atomic>
#include <cstdint>
#include <cstdlib>
#include <initializer_list>
#include <mutex>
#include <string>

#include "hai_common.h"
#include "hai_device.h"
#include "hai_gemm_common.h"

namespace {

using namespace hai;

constexpr int kChunk = 64;
constexpr int kWaves = 4;
// chunk grid (chunks x KV heads x sequences) from which a block serves every
// query of its KV head (measured on MI355X: the C2 shape, 256 chunk blocks,
// 35.9 -> 27.0 us; C3 and C4 unchanged)
constexpr int64_t kFullGroupBlocks = 256;

__host__ __device__ constexpr int64_t partial_stride(int D) { return D + 2; }

// The q / k RMSNorm(+1) + partial RoPE (+ K/V cache append) of
// hai_qkv_rmsnorm_rope_append_bf16, done inside the partial kernel (FUSE):
// projection rows b*T + t hold [q_h | gate_h] for the nq heads, then the nkv
// K heads, then the nkv V heads.
struct QkvFuse {
    const uint16_t* proj;
    int64_t ld;
    const uint16_t *wq, *wk;
    const float *rc, *rs;
    int64_t rope_pos;
    int R;
    float eps;
    uint16_t* gate_out;  // [B*T][nq][D], the gate halves copied for the merge pass
    uint16_t *kc, *vc;   // the caches, written at the T new positions
};

__device__ __forceinline__ void wave_fence_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Query head h of projection row `row` (position pos): the bf16 values
// q_gate_rmsnorm_rope_pair stores, element lane + 64 r in qv[r]; the gate
// half copied to gate_out when copy_gate.  scratch: D floats of the wave.
template <int D>
__device__ __forceinline__ void fused_q_row(uint16_t (&qv)[D / 64], const QkvFuse& F, int64_t row, int h, int nq,
                                            int64_t pos, bool copy_gate, float* scratch, int lane) {
    const uint16_t* src = F.proj + row * F.ld + static_cast<int64_t>(h) * 2 * D;
    const HeadPiece qp = load_piece(src, D, lane);
    HeadPiece gp{{0u, 0u, 0u, 0u}};
    if (copy_gate) gp = load_piece(src + D, D, lane);
    float wv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) wv[e] = lane * 8 + e < D ? bf2f(F.wq[lane * 8 + e]) : 0.0f;
    const int64_t rp = pos < 0 ? 0 : (pos >= F.rope_pos ? F.rope_pos - 1 : pos);
    float cv[kRopeSlots], sv[kRopeSlots];
    load_rope(cv, sv, F.rc + rp * (F.R / 2), F.rs + rp * (F.R / 2), D, F.R, lane);
    const float inv = 1.0f / csqrt(piece_sumsq(qp) / static_cast<float>(D) + F.eps);
    if (lane * 8 < D) {
#pragma unroll
        for (int e = 0; e < 8; ++e) scratch[lane * 8 + e] = (qp.at(e) * inv) * (wv[e] + 1.0f);
    }
    wave_fence_sync();
#pragma unroll
    for (int r = 0; r < D / 64; ++r) qv[r] = f2bf(rope_reg(scratch, lane + 64 * r, F.R, cv[r], sv[r]));
    if (copy_gate && lane * 8 < D) {
        uint16_t* go = F.gate_out + (row * nq + h) * D + lane * 8;
#pragma unroll
        for (int e = 0; e < 8; ++e) go[e] = static_cast<uint16_t>(gp.w[e >> 1] >> (16 * (e & 1)));
    }
    wave_fence_sync();  // scratch is rewritten next
}

// K / V head kvh of projection row `row` at position pos, as
// kv_rmsnorm_rope_append_pair computes it, into the staged rows ks_row /
// vs_row (and the caches at pos when append).  scratch: D floats of the wave.
template <int D>
__device__ __forceinline__ void fused_kv_row(uint32_t* ks_row, uint32_t* vs_row, const QkvFuse& F, int64_t row,
                                             int kvh, int nq, int nkv, int64_t pos, int64_t cache_row, bool append,
                                             float* scratch, int lane) {
    const uint16_t* sk = F.proj + row * F.ld + static_cast<int64_t>(2 * nq + kvh) * D;
    const uint16_t* sv = F.proj + row * F.ld + static_cast<int64_t>(2 * nq + nkv + kvh) * D;
    const HeadPiece kp = load_piece(sk, D, lane);
    const HeadPiece vp = load_piece(sv, D, lane);
    float wv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) wv[e] = lane * 8 + e < D ? bf2f(F.wk[lane * 8 + e]) : 0.0f;
    const int64_t rp = pos < 0 ? 0 : (pos >= F.rope_pos ? F.rope_pos - 1 : pos);
    float cv[kRopeSlots], sv2[kRopeSlots];
    load_rope(cv, sv2, F.rc + rp * (F.R / 2), F.rs + rp * (F.R / 2), D, F.R, lane);
    const float inv = 1.0f / csqrt(piece_sumsq(kp) / static_cast<float>(D) + F.eps);
    if (lane * 8 < D) {
#pragma unroll
        for (int e = 0; e < 8; ++e) scratch[lane * 8 + e] = bfr((kp.at(e) * inv) * (wv[e] + 1.0f));
    }
    wave_fence_sync();
    uint16_t* kr = reinterpret_cast<uint16_t*>(ks_row);
#pragma unroll
    for (int r = 0; r < D / 64; ++r) {
        const int d = lane + 64 * r;
        const uint16_t kv = f2bf(rope_reg(scratch, d, F.R, cv[r], sv2[r]));
        kr[d] = kv;
        if (append) F.kc[cache_row * D + d] = kv;
    }
    if (lane * 8 < D) {
        *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(vs_row) + lane * 8) =
            make_uint4(vp.w[0], vp.w[1], vp.w[2], vp.w[3]);
        if (append) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                F.vc[cache_row * D + lane * 8 + e] = static_cast<uint16_t>(vp.w[e >> 1] >> (16 * (e & 1)));
        }
    }
    wave_fence_sync();  // scratch is rewritten next
}

// grid (chunk, query group x KV head, sequence): the block stages one 64-key
// chunk of one KV head and serves qpb of that head's queries.  Each wave takes
// up to QG of them at a time: a K or V element is unpacked once and feeds the
// QG queries' fma chains (each chain keeps its own sequential order).
// FUSE: the queries are normalised and rotated here from the projection rows
// (fused_q_row), the chunk's rows at the T new positions are built from them
// (fused_kv_row: the cache is not read there, and the first query group's
// block writes them to it), and the chunk-0 blocks copy the gate halves; the
// values are those of hai_qkv_rmsnorm_rope_append_bf16 followed by the plain
// kernel, bit for bit.
template <int D, int QG, int W, bool FUSE = false>
__global__ __launch_bounds__(64 * W) void gqa_partial_kernel(
    float* __restrict__ scratch, const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, int64_t cap, int T, int nq, int nkv, const int32_t* lens,
    int len_add, int nchunk, float scale, int qpb, QkvFuse F) {
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
        if constexpr (FUSE) return;  // computed at the start of the pass (fused_q_row)
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
    if constexpr (FUSE) {
        // the chunk's rows at the new positions L - T .. L - 1, one wave each
        const int64_t first_new = L - T;
        const int j0 = first_new > key0 ? static_cast<int>(first_new - key0) : 0;
        for (int j = j0 + wave; j < nkeys; j += W) {
            const int64_t pos = key0 + j;
            const int64_t t = pos - first_new;
            fused_kv_row<D>(Ks + j * KP, Vs + j * VP, F, static_cast<int64_t>(b) * T + t, kvh, nq, nkv, pos,
                            (static_cast<int64_t>(b) * cap + pos) * nkv + kvh, qgrp == 0 && pos < cap,
                            &Qs[wave][0][0], lane);
        }
        __syncthreads();
    }

    auto wave_sync = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    for (int base = q_begin + wave * QG; base < q_end; base += W * QG) {
        const int nw = min(QG, q_end - base);
        if constexpr (FUSE) {
#pragma unroll
            for (int qq = 0; qq < QG; ++qq)
                if (qq < nw) {
                    const int qi = base + qq;
                    const int t = qi / group;
                    fused_q_row<D>(qv[qq], F, static_cast<int64_t>(b) * T + t, kvh * group + qi % group, nq,
                                   L - T + t, chunk == 0, &Qs[wave][qq][0], lane);
                }
        }
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

// Chunk partials of one query merged in chunk order against the global
// max, then divided, gated and rounded.
template <int D>
__global__ __launch_bounds__(D) void gqa_combine_kernel(
    uint16_t* __restrict__ out, const float* __restrict__ scratch, const uint16_t* gate, int B, int T,
    int nq, const int32_t* lens, int len_add, int nchunk) {
    // One block per query row, thread d owns output dimension d.  The chunk
    // weights w_c = exp(m_c - M) and sums l_c are formed once per batch of D
    // chunks into LDS; then each thread folds its dimension over the chunks
    // in order, with a batch's loads all issued before the first fma (the
    // latency of one batch, not of every eighth chunk).  The fma order per
    // element, and Ls's, are those of the chunk loop they replace, so the
    // result is unchanged bit for bit.
    constexpr int kBatch = 32;  // chunk loads in flight per thread
    __shared__ float w_sh[D], l_sh[D], red[D / 64];
    const int tid = threadIdx.x;
    const int64_t qidx = blockIdx.x;
    const int64_t m = qidx / nq;
    const int b = static_cast<int>(m / T);
    const int t = static_cast<int>(m % T);
    const int64_t L = static_cast<int64_t>(lens ? lens[b] : 0) + len_add;
    const int64_t qpos = L - T + t;
    const int nch = static_cast<int>(qpos / kChunk) + 1;
    constexpr int64_t PS = partial_stride(D);
    const float* base = scratch + qidx * nchunk * PS;
    float M = __uint_as_float(0xff800000u);
    for (int c = tid; c < nch; c += D) M = fmaxf(M, base[c * PS]);
    M = wave_max64(M);
    if constexpr (D > 64) {
        if ((tid & 63) == 0) red[tid >> 6] = M;
        __syncthreads();
#pragma unroll
        for (int i = 0; i < D / 64; ++i) M = fmaxf(M, red[i]);
    }
    float O = 0.0f, Ls = 0.0f;
    for (int c0 = 0; c0 < nch; c0 += D) {
        const int nt = min(D, nch - c0);
        __syncthreads();  // the previous batch's weights are read
        if (tid < nt) {
            const float* part = base + (c0 + tid) * PS;
            w_sh[tid] = cexp(part[0] - M);
            l_sh[tid] = part[1];
        }
        __syncthreads();
        for (int cb = 0; cb < nt; cb += kBatch) {
            float pv[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int cc = min(cb + u, nt - 1);
                pv[u] = base[(c0 + cc) * PS + 2 + tid];
            }
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                if (cb + u < nt) {
                    const float wc = w_sh[cb + u];
                    Ls = fma_(l_sh[cb + u], wc, Ls);
                    O = fma_(pv[u], wc, O);
                }
            }
        }
    }
    float o = O / Ls;
    if (gate != nullptr) o = o * csigmoid(bf2f(gate[qidx * D + tid]));
    out[qidx * D + tid] = f2bf(o);
}

template <int D, bool FUSE = false>
int launch(uint16_t* out, const uint16_t* q, const uint16_t* gate, const uint16_t* kc, const uint16_t* vc,
           int64_t cap, float* scratch, int B, int T, int nq, int nkv, const int32_t* lens, int len_add,
           int nchunk, hipStream_t s, const QkvFuse& F = QkvFuse{}) {
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
        gqa_partial_kernel<D, 1, 4, FUSE><<<grid, dim3(256), 0, s>>>(scratch, q, kc, vc, cap, T, nq, nkv, lens,
                                                                     len_add, nchunk, scale, qpb, F);
    else if (qpb <= 8)
        gqa_partial_kernel<D, 2, 4, FUSE><<<grid, dim3(256), 0, s>>>(scratch, q, kc, vc, cap, T, nq, nkv, lens,
                                                                     len_add, nchunk, scale, qpb, F);
    else if (qpb <= 16)
        gqa_partial_kernel<D, 2, 8, FUSE><<<grid, dim3(512), 0, s>>>(scratch, q, kc, vc, cap, T, nq, nkv, lens,
                                                                     len_add, nchunk, scale, qpb, F);
    else
        gqa_partial_kernel<D, 3, 8, FUSE><<<grid, dim3(512), 0, s>>>(scratch, q, kc, vc, cap, T, nq, nkv, lens,
                                                                     len_add, nchunk, scale, qpb, F);
    int rc = launched("gqa_partial_kernel");
    if (rc != HAI_OK) return rc;
    const int64_t nall = static_cast<int64_t>(B) * T * nq;
    gqa_combine_kernel<D><<<dim3(static_cast<unsigned>(nall)), dim3(D), 0, s>>>(out, scratch, gate, B, T, nq, lens,
                                                                             len_add, nchunk);
    return launched("gqa_combine_kernel");
}

// ---------------------------------------------------------------------------
// Tolerance mode: the same attention with Q.K^T and P.V on the matrix cores
// (v_mfma_f32_16x16x32_bf16), for the batched verify / draft steps whose
// exact form is VALU-bound (one fp32 fma per K or V element per query).
//
// A wave is an independent flash-decoder over its own keys: each step it
// takes KS consecutive keys (32, or 64 at D = 64), computes S^T = K . Q^T for
// up to 32 queries (one or two 16-query tiles; K rows are the A operand, read
// straight from the cache, Q rows the B operand, kept in registers), updates
// a running max and exp-sum per query (base-2, scores pre-scaled by
// log2(e) / sqrt(D)), and accumulates O^T = V^T . P^T with P rounded to bf16.
// V^T is the A operand, so the step's V rows are transposed 8 x 8 in
// registers and staged in the wave's own LDS tile.  Block waves interleave
// their steps over the block's key range (wave w takes keys 4s + w in units
// of KS), the block merges its four waves in LDS and writes one partial per
// query: O[D], max, sum.  A second pass merges the partials of the splits.
// Every step's loads for the next step are in flight while it computes.
// ---------------------------------------------------------------------------

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kMfmaWaves = 4;
constexpr int kCombineBlockSplits = 16;  // splits per query row from which the merge takes a block per row
constexpr int kMfmaMaxSteps = 16;          // steps per wave and block
constexpr int64_t kMfmaTargetBlocks = 512; // blocks the split count aims for when the occupancy is unknown
constexpr int kMfmaMinBlockKeys = 128;     // keys of the smallest block (one 32-key step per wave)

__host__ __device__ constexpr int mfma_step_keys(int D) { return D == 64 ? 64 : 32; }
__host__ __device__ constexpr int64_t mfma_part_stride(int D) { return D + 4; }

__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma16(u32x4 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), b, c, 0, 0, 0);
}

// The running max of a query moves only when a score exceeds it by more than
// this (base-2 units), so most steps skip rescaling O; probabilities then stay
// below 2^kRescaleSlack, far inside bf16 / fp32 range.
constexpr float kRescaleSlack = 8.0f;

template <int D, int QT>
struct MfmaAttnShape {
    static constexpr int KS = mfma_step_keys(D);  // keys per wave step
    static constexpr int NKT = KS / 16;           // 16-key score tiles per step
    static constexpr int NJ = D / 32;             // 32-dim slabs of a score
    static constexpr int NDT = D / 16;            // 16-dim output tiles
    static constexpr int PR = D / 8;              // 16-byte pieces of a K / V row
    static constexpr int KG = 64 / PR;            // keys per V load instruction
    static constexpr int NB = KS / (8 * KG);      // 8 x 8 transposes per lane and step
    static constexpr int VTP = KS + 8;            // staged V^T row: KS keys + 16-byte pad
    static constexpr int QROWS = 16 * QT;
    static constexpr int MP = D + 4;              // merge-buffer row, floats
    static constexpr int VT_BYTES = kMfmaWaves * D * VTP * 2;
    static constexpr int MERGE_BYTES = 2 * QROWS * MP * 4 + 4 * QROWS * 4;
    static constexpr int QP = D + 8;              // staged Q row, bf16 elements
    static constexpr int Q_BYTES = QROWS * QP * 2;
    static constexpr int LDS_BYTES = (VT_BYTES > MERGE_BYTES ? VT_BYTES : MERGE_BYTES) + Q_BYTES;
    static_assert(NB >= 1 && NB * 8 * KG == KS, "a step's V rows must split into 8 x 8 transposes");
};

// grid (split, query group x KV head, sequence); block = 4 waves.
template <int D, int QT>
__global__ __launch_bounds__(256) void gqa_mfma_partial_kernel(
    float* __restrict__ part, const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, int64_t cap, int T, int nq, int nkv, const int32_t* lens, int len_add,
    int nsplit, int steps, float scale_log2) {
    using S = MfmaAttnShape<D, QT>;
    constexpr int KS = S::KS, NKT = S::NKT, NJ = S::NJ, NDT = S::NDT, PR = S::PR, KG = S::KG, NB = S::NB;
    constexpr int VTP = S::VTP, QROWS = S::QROWS, MP = S::MP;
    constexpr float kNegInf = -__builtin_huge_valf();
    __shared__ __align__(16) unsigned char lds[S::LDS_BYTES];

    const int split = blockIdx.x;
    const int kvh = blockIdx.y % nkv;
    const int qgrp = blockIdx.y / nkv;
    const int b = blockIdx.z;
    const int lane = threadIdx.x & 63;
    const int wave = wave_index();
    const int li = lane & 15;
    const int kg = lane >> 4;
    const int64_t L = static_cast<int64_t>(lens ? lens[b] : 0) + len_add;
    const int block_keys = steps * kMfmaWaves * KS;
    const int64_t kb0 = static_cast<int64_t>(split) * block_keys;
    if (kb0 >= L) return;  // uniform over the block: no partial (the merge pass skips it)
    const int nkeys = static_cast<int>(min(static_cast<int64_t>(block_keys), L - kb0));
    const int group = nq / nkv;
    const int nqry = T * group;
    const int q_begin = qgrp * QROWS;

    // The group's Q rows, staged once in LDS (the B operand of the scores:
    // lane (li, kg) reads query 16 qt + li, dims 32 j + 8 kg + [0, 8)).
    // Padding queries are zero and get the last token's causal limit; their
    // results are not stored.
    uint16_t* qs = reinterpret_cast<uint16_t*>(lds + (S::LDS_BYTES - S::Q_BYTES));
    for (int e = threadIdx.x; e < QROWS * PR; e += 256) {
        const int r = e / PR, c = (e % PR) * 8;
        const int qi = q_begin + r;
        u32x4 v = u32x4{0, 0, 0, 0};
        if (qi < nqry) {
            const int64_t row = (static_cast<int64_t>(b) * T + qi / group) * nq + kvh * group + qi % group;
            v = *reinterpret_cast<const u32x4*>(q + row * D + c);
        }
        *reinterpret_cast<u32x4*>(qs + r * S::QP + c) = v;
    }
    // keys [kb0, kb0 + lim) of the block are visible to the lane's queries
    int lim[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int qi = q_begin + 16 * qt + li;
        const int64_t qpos = L - T + (qi < nqry ? qi / group : T - 1);
        const int64_t n = qpos - kb0 + 1;
        lim[qt] = static_cast<int>(n < 0 ? 0 : (n < nkeys ? n : nkeys));
    }

    // The block's K / V rows: keys [kb0, kb0 + nkeys) of head kvh; loads past
    // them return zeros and their scores are masked.
    const uint32_t kst = static_cast<uint32_t>(nkv * D * 2);  // bytes between consecutive keys
    const int64_t off0 = ((static_cast<int64_t>(b) * cap + kb0) * nkv + kvh) * D;
    const uint32_t bytes = static_cast<uint32_t>((static_cast<int64_t>(nkeys - 1) * nkv * D + D) * 2);
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(kc + off0, bytes);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vc + off0, bytes);
    // wave steps that hold at least one key visible to some query of the
    // group (the group's last query sees the most: queries are in token
    // order); steps past it would only add zero probabilities
    int nvis = nkeys;
    {
        const int q_last = min(q_begin + QROWS, nqry) - 1;
        const int64_t vis = (L - T + q_last / group) - kb0 + 1;
        if (vis < nvis) nvis = static_cast<int>(vis < 0 ? 0 : vis);
    }
    int wsteps = 0;
    while (wsteps < steps && (wsteps * kMfmaWaves + wave) * KS < nvis) ++wsteps;

    u32x4 kr[NKT][NJ];
    u32x4 vr[NB][8];
    // K rows (A operand): lane (li, kg) takes key 16 kt + li, dims 32 j + 8 kg + [0, 8)
    auto load_k = [&](int s) {
        const uint32_t k0 = static_cast<uint32_t>((s * kMfmaWaves + wave) * KS);
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                kr[kt][j] = bload(rk, (k0 + 16 * kt + li) * kst + (32 * j + 8 * kg) * 2, 0);
    };
    // V rows for the transpose: lane takes piece lane % PR (dims 8 (lane % PR)
    // + [0, 8)) of keys 8 (KG bb + lane / PR) + i, i = 0..7
    const int vp = lane % PR;
    const int vh = lane / PR;
    auto load_v = [&](int s) {
        const uint32_t k0 = static_cast<uint32_t>((s * kMfmaWaves + wave) * KS);
#pragma unroll
        for (int bb = 0; bb < NB; ++bb)
#pragma unroll
            for (int i = 0; i < 8; ++i) vr[bb][i] = bload(rv, (k0 + 8 * (KG * bb + vh) + i) * kst + vp * 16, 0);
    };
    // V^T tile of the wave: row d holds the step's KS keys of dim d
    uint16_t* vt = reinterpret_cast<uint16_t*>(lds) + wave * D * VTP;
    auto stage_v = [&] {
#pragma unroll
        for (int bb = 0; bb < NB; ++bb)
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                // dword w of row r: keys 2w, 2w + 1 of dim 8 vp + r
                const uint32_t sel = (r & 1) ? 0x07060302u : 0x05040100u;
                u32x4 o;
#pragma unroll
                for (int w = 0; w < 4; ++w)
                    o[w] = __builtin_amdgcn_perm(vr[bb][2 * w + 1][r >> 1], vr[bb][2 * w][r >> 1], sel);
                *reinterpret_cast<u32x4*>(vt + (8 * vp + r) * VTP + 8 * (KG * bb + vh)) = o;
            }
    };
    auto wave_sync = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };

    float m[QT], l[QT];
    f32x4 o[QT][NDT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        m[qt] = kNegInf;
        l[qt] = 0.0f;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) o[qt][dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }

    if (wsteps > 0) {
        load_k(0);
        load_v(0);
    }
    __syncthreads();  // Q staged
    for (int s = 0; s < wsteps; ++s) {
        wave_sync();  // the previous step's V^T reads precede these writes
        stage_v();
        if (s + 1 < wsteps) load_v(s + 1);
        f32x4 st[NKT][QT];
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                st[kt][qt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const u32x4 qv = *reinterpret_cast<const u32x4*>(qs + (16 * qt + li) * S::QP + 32 * j + 8 * kg);
                    st[kt][qt] = mfma16(kr[kt][j], qv, st[kt][qt]);
                }
            }
        if (s + 1 < wsteps) load_k(s + 1);

        // lane (li, kg) holds the scores of query li for keys 16 kt + 4 kg + i
        // (block-relative key index key_l + 16 kt + i)
        const int key_l = (s * kMfmaWaves + wave) * KS + 4 * kg;
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            float mx = kNegInf;
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float x = key_l + 16 * kt + i < lim[qt] ? st[kt][qt][i] * scale_log2 : kNegInf;
                    st[kt][qt][i] = x;
                    mx = fmaxf(mx, x);
                }
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const bool grow = mx > m[qt] + kRescaleSlack;  // true for the first visible key
            if (__builtin_amdgcn_ballot_w64(grow) != 0) {  // wave-uniform
                const float mn = grow ? mx : m[qt];
                const float alpha = grow ? __builtin_amdgcn_exp2f(m[qt] - mn) : 1.0f;  // 0 from -inf
                l[qt] *= alpha;
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) o[qt][dt] *= alpha;
                m[qt] = mn;
            }
            const float sub = m[qt] == kNegInf ? 0.0f : m[qt];  // no visible key yet: every p is 0
            float ps = 0.0f;
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float p = __builtin_amdgcn_exp2f(st[kt][qt][i] - sub);
                    st[kt][qt][i] = p;
                    ps += p;
                }
            l[qt] += ps;
        }
        wave_sync();  // V^T of this step is in LDS
#pragma unroll
        for (int ks = 0; ks < NKT / 2; ++ks) {
            // P^T operand: keys 32 ks + 4 kg + [0, 4) then 32 ks + 16 + 4 kg + [0, 4)
            bf16x8 pop[QT];
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                const f32x4 a = st[2 * ks][qt], c = st[2 * ks + 1][qt];
                pop[qt] = bf16x8{static_cast<__bf16>(a[0]), static_cast<__bf16>(a[1]), static_cast<__bf16>(a[2]),
                                 static_cast<__bf16>(a[3]), static_cast<__bf16>(c[0]), static_cast<__bf16>(c[1]),
                                 static_cast<__bf16>(c[2]), static_cast<__bf16>(c[3])};
            }
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                const uint16_t* vrow = vt + (16 * dt + li) * VTP + 32 * ks + 4 * kg;
                const uint2 lo = *reinterpret_cast<const uint2*>(vrow);
                const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 16);
                const u32x4 a = u32x4{lo.x, lo.y, hi.x, hi.y};
#pragma unroll
                for (int qt = 0; qt < QT; ++qt) o[qt][dt] = mfma16(a, pop[qt], o[qt][dt]);
            }
        }
    }
    // full exp-sum of each query over the lane's four key groups
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        l[qt] += __shfl_xor(l[qt], 16);
        l[qt] += __shfl_xor(l[qt], 32);
    }

    // Merge the four waves: 2 -> 0 and 3 -> 1, then 1 -> 0.  O^T layout: lane
    // (li, kg) holds dims 16 dt + 4 kg + [0, 4) of query 16 qt + li.
    __syncthreads();  // every wave is done with its V^T tile
    float* mb = reinterpret_cast<float*>(lds);  // [2][QROWS][MP]
    float* ml = mb + 2 * QROWS * MP;            // [2][2][QROWS]: max, sum
    auto put = [&](int slot) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            float* row = mb + (slot * QROWS + 16 * qt + li) * MP + 4 * kg;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) *reinterpret_cast<f32x4*>(row + 16 * dt) = o[qt][dt];
            if (kg == 0) {
                ml[(slot * 2) * QROWS + 16 * qt + li] = m[qt];
                ml[(slot * 2 + 1) * QROWS + 16 * qt + li] = l[qt];
            }
        }
    };
    auto merge = [&](int slot) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            const float mo = ml[(slot * 2) * QROWS + 16 * qt + li];
            const float lo = ml[(slot * 2 + 1) * QROWS + 16 * qt + li];
            const float M = fmaxf(m[qt], mo);
            const bool empty = M == kNegInf;
            const float a = empty ? 0.0f : __builtin_amdgcn_exp2f(m[qt] - M);
            const float c = empty ? 0.0f : __builtin_amdgcn_exp2f(mo - M);
            l[qt] = fma_(l[qt], a, lo * c);
            m[qt] = M;
            const float* row = mb + (slot * QROWS + 16 * qt + li) * MP + 4 * kg;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(row + 16 * dt);
                o[qt][dt] = o[qt][dt] * a + v * c;
            }
        }
    };
    if (wave >= 2) put(wave - 2);
    __syncthreads();
    if (wave < 2) merge(wave);
    __syncthreads();
    if (wave == 1) put(0);
    __syncthreads();
    if (wave != 0) return;
    merge(0);
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int qi = q_begin + 16 * qt + li;
        if (qi >= nqry) continue;
        const int64_t row = (static_cast<int64_t>(b) * T + qi / group) * nq + kvh * group + qi % group;
        float* dst = part + (row * nsplit + split) * mfma_part_stride(D);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) *reinterpret_cast<f32x4*>(dst + 16 * dt + 4 * kg) = o[qt][dt];
        if (kg == 0) {
            dst[D] = m[qt];
            dst[D + 1] = l[qt];
        }
    }
}

// The splits' partials of one query merged against the global max (base
// 2), divided, gated and rounded: one block per query row, thread d owns
// output dimension d, the split weights formed once per batch in LDS and a
// batch's loads all issued before the first fma (the order of every sum is
// the split order).
template <int D>
__global__ __launch_bounds__(D) void gqa_mfma_combine_kernel(uint16_t* __restrict__ out,
                                                             const float* __restrict__ part, const uint16_t* gate,
                                                             int B, int T, int nq, const int32_t* lens,
                                                             int len_add, int nsplit, int block_keys) {
    constexpr int kBatch = 32;
    __shared__ float w_sh[D], l_sh[D], red[D / 64];
    const int tid = threadIdx.x;
    const int64_t qidx = blockIdx.x;
    const int b = static_cast<int>(qidx / (static_cast<int64_t>(T) * nq));
    const int64_t L = static_cast<int64_t>(lens ? lens[b] : 0) + len_add;
    const int nv = static_cast<int>(min(static_cast<int64_t>(nsplit), (L + block_keys - 1) / block_keys));
    constexpr int64_t PS = mfma_part_stride(D);
    const float* base = part + qidx * nsplit * PS;
    float M = -__builtin_huge_valf();
    for (int c = tid; c < nv; c += D) M = fmaxf(M, base[c * PS + D]);
    M = wave_max64(M);
    if constexpr (D > 64) {
        if ((tid & 63) == 0) red[tid >> 6] = M;
        __syncthreads();
#pragma unroll
        for (int i = 0; i < D / 64; ++i) M = fmaxf(M, red[i]);
    }
    float O = 0.0f, Ls = 0.0f;
    for (int c0 = 0; c0 < nv; c0 += D) {
        const int nt = min(D, nv - c0);
        __syncthreads();  // the previous batch's weights are read
        if (tid < nt) {
            const float* p = base + (c0 + tid) * PS;
            w_sh[tid] = __builtin_amdgcn_exp2f(p[D] - M);
            l_sh[tid] = p[D + 1];
        }
        __syncthreads();
        for (int cb = 0; cb < nt; cb += kBatch) {
            float ov[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) ov[u] = base[(c0 + min(cb + u, nt - 1)) * PS + tid];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                if (cb + u < nt) {
                    const float w = w_sh[cb + u];
                    Ls = fma_(l_sh[cb + u], w, Ls);
                    O = fma_(ov[u], w, O);
                }
            }
        }
    }
    float v = O / Ls;
    if (gate != nullptr) v = v * csigmoid(bf2f(gate[qidx * D + tid]));
    out[qidx * D + tid] = f2bf(v);
}

// The same merge with one wave per query row (four rows per block): the
// form for prompt chunks, whose many query rows hold few splits each.
template <int D>
__global__ __launch_bounds__(256) void gqa_mfma_combine_wave_kernel(uint16_t* __restrict__ out,
                                                               const float* __restrict__ part, const uint16_t* gate,
                                                               int B, int T, int nq, const int32_t* lens,
                                                               int len_add, int nsplit, int block_keys) {
    const int lane = threadIdx.x & 63;
    const int64_t qidx = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (qidx >= static_cast<int64_t>(B) * T * nq) return;
    const int b = static_cast<int>(qidx / (static_cast<int64_t>(T) * nq));
    const int64_t L = static_cast<int64_t>(lens ? lens[b] : 0) + len_add;
    const int nv = static_cast<int>(min(static_cast<int64_t>(nsplit), (L + block_keys - 1) / block_keys));
    constexpr int64_t PS = mfma_part_stride(D);
    const float* base = part + qidx * nsplit * PS;
    float M = -__builtin_huge_valf();
    for (int c = lane; c < nv; c += 64) M = fmaxf(M, base[c * PS + D]);
    M = wave_max64(M);
    constexpr int PER = D / 64;
    float O[PER];
#pragma unroll
    for (int r = 0; r < PER; ++r) O[r] = 0.0f;
    float Ls = 0.0f;
    int c = 0;
    for (; c + 4 <= nv; c += 4) {
        float mv[4], lv[4], ov[4][PER];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float* p = base + (c + u) * PS;
            mv[u] = p[D];
            lv[u] = p[D + 1];
#pragma unroll
            for (int r = 0; r < PER; ++r) ov[u][r] = p[lane + 64 * r];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float w = __builtin_amdgcn_exp2f(mv[u] - M);
            Ls = fma_(lv[u], w, Ls);
#pragma unroll
            for (int r = 0; r < PER; ++r) O[r] = fma_(ov[u][r], w, O[r]);
        }
    }
    for (; c < nv; ++c) {
        const float* p = base + c * PS;
        const float w = __builtin_amdgcn_exp2f(p[D] - M);
        Ls = fma_(p[D + 1], w, Ls);
#pragma unroll
        for (int r = 0; r < PER; ++r) O[r] = fma_(p[lane + 64 * r], w, O[r]);
    }
#pragma unroll
    for (int r = 0; r < PER; ++r) {
        const int d = lane + 64 * r;
        float v = O[r] / Ls;
        if (gate != nullptr) v = v * csigmoid(bf2f(gate[qidx * D + d]));
        out[qidx * D + d] = f2bf(v);
    }
}

// ---------------------------------------------------------------------------
// Prompt chunks: flash attention with a block's K / V tiles shared by its
// waves.  Block = 4 waves x 32 query rows (one KV head, one sequence); each
// wave walks every key its rows see, 64 keys per tile (two 32-key score tiles):
//   S^T = K Q^T  on v_mfma_f32_32x32x16_bf16 (K rows the A operand from LDS,
//                Q^T the B operand held in registers for the whole kernel);
//   online softmax per query (base 2, the running max moved only past the
//                same slack as gqa_mfma_partial_kernel, P rounded to bf16);
//   O^T += V^T P^T  (V^T staged transposed in LDS; the result tile of S^T is
//                the B operand of this product as it stands, under the key
//                order 4 lh + q % 4 + 8 (q / 4) of k slot q).
// K reaches LDS by global -> LDS copies, 16-byte piece p of key row r at
// slot (D / 8) r + (p ^ (r % 16)); V through registers, transposed 8 keys x 8
// dims per thread.  One barrier per tile.  The gated output O / l *
// sigmoid(gate) is written directly: no split partials and no merge pass.
// Same tolerance mode as the matrix-core verify attention.
// ---------------------------------------------------------------------------
constexpr int kFaRows = 128;  // query rows per block
constexpr int kFaKeys = 64;   // keys per tile (two 32-key score tiles)

template <int D>
struct FaShape {
    static constexpr int KP = D / 8;               // 16-byte pieces of a K row
    static constexpr int K_SLOTS = kFaKeys * KP;   // K tile, 16-byte slots
    static constexpr int VTR = kFaKeys + 8;        // V^T row: the tile's keys + 16-byte pad (bf16)
    static constexpr int STAGE_BYTES = K_SLOTS * 16 + D * VTR * 2;
    static constexpr int LDS_BYTES = 2 * STAGE_BYTES;
    static constexpr int KCOPY = K_SLOTS / 256;    // copy instructions per thread and tile
    static constexpr int NKK = D / 16;             // 16-dim k steps of S^T
    static constexpr int NDT = D / 32;             // 32-dim tiles of O^T
    static constexpr int NST = kFaKeys / 32;       // score tiles per key tile
};

template <int D>
__global__ __launch_bounds__(256) void gqa_fa_kernel(uint16_t* __restrict__ out, const uint16_t* __restrict__ q,
                                                     const uint16_t* __restrict__ gate, const uint16_t* kc,
                                                     const uint16_t* vc, int64_t cap, int T, int nq, int nkv,
                                                     const int32_t* lens, int len_add, float scale_log2) {
    using S = FaShape<D>;
    constexpr int NST = S::NST;
    static_assert(D % 32 == 0 && S::K_SLOTS % 256 == 0 && kFaKeys % 32 == 0, "tile shapes");
    constexpr float kNegInf = -__builtin_huge_valf();
    extern __shared__ __align__(16) unsigned char fa_lds[];
    const int qblk = blockIdx.x;
    const int kvh = blockIdx.y;
    const int b = blockIdx.z;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = wave_index();
    const int lc = lane & 31;
    const int lh = lane >> 5;
    const int group = nq / nkv;
    const int nqry = T * group;
    const int64_t L = static_cast<int64_t>(lens ? lens[b] : 0) + len_add;
    const int q0 = qblk * kFaRows;
    // the lane's query (padding rows past nqry take the last token and are not stored)
    const int qi = q0 + 32 * wave + lc;
    const int tq = qi < nqry ? qi / group : T - 1;
    const int64_t lim = L - T + tq + 1;  // keys [0, lim) are visible
    const int t_last = (min(q0 + kFaRows, nqry) - 1) / group;
    const int64_t nkeys = L - T + t_last + 1;  // keys any query of the block sees
    const int ntiles = static_cast<int>((nkeys + kFaKeys - 1) / kFaKeys);

    // Q^T operand: k step kk holds dims 16 kk + 8 lh + [0, 8) of the lane's query
    u32x4 qr[S::NKK];
    {
        const int64_t row = (static_cast<int64_t>(b) * T + tq) * nq + kvh * group + (qi < nqry ? qi % group : 0);
        const uint16_t* qp = q + row * D + 8 * lh;
#pragma unroll
        for (int kk = 0; kk < S::NKK; ++kk) qr[kk] = *reinterpret_cast<const u32x4*>(qp + 16 * kk);
    }

    const uint16_t* kbase = kc + (static_cast<int64_t>(b) * cap * nkv + kvh) * D;
    const uint16_t* vbase = vc + (static_cast<int64_t>(b) * cap * nkv + kvh) * D;
    const int64_t kstride = static_cast<int64_t>(nkv) * D;  // elements between consecutive keys
    auto key_row = [&](int64_t key) { return min(key, L - 1) * kstride; };  // keys past L: the last row (masked)
    // K copies: instruction i of this wave covers slots (4 i + wave) * 64 + lane
    auto copy_k = [&](int tile, int buf) {
        u32x4* dst = reinterpret_cast<u32x4*>(fa_lds + buf * S::STAGE_BYTES);
#pragma unroll
        for (int i = 0; i < S::KCOPY; ++i) {
            const int s = (4 * i + wave) * 64 + lane;
            const int r = s / S::KP, p = (s % S::KP) ^ (r & 15);
            const uint16_t* src = kbase + key_row(static_cast<int64_t>(tile) * kFaKeys + r) + 8 * p;
            __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(dst + (4 * i + wave) * 64),
                                             16, 0, 0);
        }
    };
    // V: thread (kq = tid / (D / 8), dp = tid % (D / 8)) loads keys VK kq + [0, VK) x dims 8 dp + [0, 8)
    constexpr int VT_DIMS = D / 8;
    constexpr int VK = kFaKeys * VT_DIMS / 256;  // keys per thread (8 at D = 256)
    static_assert(VK == 4 || VK == 8, "V block per thread");
    const int vkq = tid / VT_DIMS, vdp = tid % VT_DIMS;
    u32x4 vr[VK];
    auto load_v = [&](int tile) {
#pragma unroll
        for (int i = 0; i < VK; ++i)
            vr[i] = *reinterpret_cast<const u32x4*>(
                vbase + key_row(static_cast<int64_t>(tile) * kFaKeys + VK * vkq + i) + 8 * vdp);
    };
    auto stage_v = [&](int buf) {
        uint16_t* vt = reinterpret_cast<uint16_t*>(fa_lds + buf * S::STAGE_BYTES + S::K_SLOTS * 16);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            // keys VK kq .. VK kq + VK - 1 of dim 8 dp + j
            const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
            uint32_t d[VK / 2];
#pragma unroll
            for (int w = 0; w < VK / 2; ++w) d[w] = __builtin_amdgcn_perm(vr[2 * w + 1][j >> 1], vr[2 * w][j >> 1], sel);
            uint16_t* dst = vt + (8 * vdp + j) * S::VTR + VK * vkq;
            if constexpr (VK == 8) *reinterpret_cast<u32x4*>(dst) = u32x4{d[0], d[1], d[2], d[3]};
            else *reinterpret_cast<uint2*>(dst) = make_uint2(d[0], d[1]);
        }
    };

    float m = kNegInf, l = 0.0f;
    f32x16 o[S::NDT];
#pragma unroll
    for (int dt = 0; dt < S::NDT; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[dt][i] = 0.0f;

    if (ntiles > 0) {
        copy_k(0, 0);
        load_v(0);
        stage_v(0);
    }
    __syncthreads();
    const int ksw = lc & 15;  // swizzle of the lane's K rows
    for (int j = 0; j < ntiles; ++j) {
        const int buf = j & 1;
        if (j + 1 < ntiles) {
            copy_k(j + 1, buf ^ 1);
            load_v(j + 1);
        }
        const u32x4* ks = reinterpret_cast<const u32x4*>(fa_lds + buf * S::STAGE_BYTES);
        const uint16_t* vt = reinterpret_cast<const uint16_t*>(fa_lds + buf * S::STAGE_BYTES + S::K_SLOTS * 16);
        // ---- S^T = K Q^T per 32-key score tile t: row = key 32 t + 8 (i / 4) + 4 lh + i % 4, column = the
        // lane's query; the tiles' chains interleaved ----
        f32x16 st[NST];
#pragma unroll
        for (int t = 0; t < NST; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) st[t][i] = 0.0f;
#pragma unroll
        for (int kk = 0; kk < S::NKK; ++kk)
#pragma unroll
            for (int t = 0; t < NST; ++t) {
                const u32x4 ka = ks[(32 * t + lc) * S::KP + ((2 * kk + lh) ^ ksw)];
                st[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, ka),
                                                               __builtin_bit_cast(bf16x8, qr[kk]), st[t], 0, 0, 0);
            }
        // ---- online softmax of the lane's query over the tile ----
        const int64_t k0 = static_cast<int64_t>(j) * kFaKeys;
        float mx = kNegInf;
#pragma unroll
        for (int t = 0; t < NST; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int64_t key = k0 + 32 * t + 8 * (i >> 2) + 4 * lh + (i & 3);
                const float x = key < lim ? st[t][i] * scale_log2 : kNegInf;
                st[t][i] = x;
                mx = fmaxf(mx, x);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const bool grow = mx > m + kRescaleSlack;  // true for the first visible key
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
            const float mn = grow ? mx : m;
            const float alpha = grow ? __builtin_amdgcn_exp2f(m - mn) : 1.0f;  // 0 from -inf
            l *= alpha;
#pragma unroll
            for (int dt = 0; dt < S::NDT; ++dt) o[dt] *= alpha;
            m = mn;
        }
        const float sub = m == kNegInf ? 0.0f : m;  // no visible key yet: every p is 0
        float ps = 0.0f;
#pragma unroll
        for (int t = 0; t < NST; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float p = __builtin_amdgcn_exp2f(st[t][i] - sub);
                st[t][i] = p;
                ps += p;
            }
        l += ps;
        // ---- O^T += V^T P^T: k step s covers keys 16 s + (4 lh + q % 4 + 8 (q / 4)), q the k slot ----
#pragma unroll
        for (int s = 0; s < 2 * NST; ++s) {
            const f32x16& sp = st[s >> 1];
            const int e = 8 * (s & 1);
            const bf16x8 pb = bf16x8{static_cast<__bf16>(sp[e]), static_cast<__bf16>(sp[e + 1]),
                                     static_cast<__bf16>(sp[e + 2]), static_cast<__bf16>(sp[e + 3]),
                                     static_cast<__bf16>(sp[e + 4]), static_cast<__bf16>(sp[e + 5]),
                                     static_cast<__bf16>(sp[e + 6]), static_cast<__bf16>(sp[e + 7])};
#pragma unroll
            for (int dt = 0; dt < S::NDT; ++dt) {
                const uint16_t* vrow = vt + (32 * dt + lc) * S::VTR + 16 * s + 4 * lh;
                const uint2 lo = *reinterpret_cast<const uint2*>(vrow);
                const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 8);
                const u32x4 va = u32x4{lo.x, lo.y, hi.x, hi.y};
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, va), pb, o[dt], 0, 0, 0);
            }
        }
        if (j + 1 < ntiles) stage_v(buf ^ 1);
        __syncthreads();  // the next tile is staged; this tile's buffer is free
    }

    // ---- O / l * sigmoid(gate), rounded: lane holds dims 32 dt + 8 (i / 4) + 4 lh + i % 4 ----
    if (qi >= nqry) return;
    l += __shfl_xor(l, 32);
    const int64_t row = (static_cast<int64_t>(b) * T + tq) * nq + kvh * group + qi % group;
#pragma unroll
    for (int dt = 0; dt < S::NDT; ++dt)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
            const int d = 32 * dt + 8 * g4 + 4 * lh;
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = o[dt][4 * g4 + e] / l;
            if (gate != nullptr) {
                const uint2 gv = *reinterpret_cast<const uint2*>(gate + row * D + d);
                v[0] *= csigmoid(lo_bf(gv.x));
                v[1] *= csigmoid(hi_bf(gv.x));
                v[2] *= csigmoid(lo_bf(gv.y));
                v[3] *= csigmoid(hi_bf(gv.y));
            }
            *reinterpret_cast<uint2*>(out + row * D + d) = make_uint2(f2bf2(v[0], v[1]), f2bf2(v[2], v[3]));
        }
}

// Compute units of the current device (one GPU model per process).
inline int attn_device_cus() {
    static std::atomic<int> cached{0};
    const int known = cached.load(std::memory_order_relaxed);
    if (known > 0) return known;
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0) {
        cached.store(cus, std::memory_order_relaxed);
        return cus;
    }
    return 256;  // MI355X
}

// The flash form for prompt chunks (HAI_ATTN_FA=0, read once per process,
// keeps the split form for every shape).
inline bool fa_enabled() {
    static const bool on = [] {
        const char* e = std::getenv("HAI_ATTN_FA");
        return e == nullptr || e[0] != '0';
    }();
    return on;
}

// Split plan of the matrix-core path: steps per wave (block = 4 waves x steps
// x KS keys) and the number of splits covering max_len.
struct MfmaPlan {
    int qt, qgroups, steps, nsplit, block_keys;
};

// `target`: the blocks the device holds at once (occupancy x CUs), so that
// every split runs in one round: at D = 256 a wave takes a whole SIMD and
// 512 blocks would leave a second, partly empty round (C4: 416 blocks on 256
// CUs).
inline MfmaPlan mfma_plan(int D, int64_t B, int64_t T, int64_t nq, int64_t nkv, int64_t max_len, int64_t target) {
    MfmaPlan p{};
    const int64_t nqry = T * (nq / nkv);
    p.qt = nqry <= 16 ? 1 : 2;
    p.qgroups = static_cast<int>((nqry + 16 * p.qt - 1) / (16 * p.qt));
    const int step_keys = kMfmaWaves * mfma_step_keys(D);
    const int64_t units = (max_len + step_keys - 1) / step_keys;  // block steps covering max_len
    const int64_t pairs = nkv * p.qgroups * B;
    const int64_t per_pair = target >= pairs ? target / pairs : 1;  // splits per (head, sequence)
    int64_t steps = (units + per_pair - 1) / per_pair;
    steps = steps < 1 ? 1 : (steps > kMfmaMaxSteps ? kMfmaMaxSteps : steps);
    p.steps = static_cast<int>(steps);
    p.block_keys = p.steps * step_keys;
    p.nsplit = static_cast<int>((max_len + p.block_keys - 1) / p.block_keys);
    return p;
}

template <int D>
int launch_mfma(uint16_t* out, const uint16_t* q, const uint16_t* gate, const uint16_t* kc, const uint16_t* vc,
                int64_t cap, float* scratch, int B, int T, int nq, int nkv, const int32_t* lens, int len_add,
                int64_t max_len, hipStream_t s) {
    const int64_t nqry = static_cast<int64_t>(T) * (nq / nkv);
    if constexpr (D == 256) {
        // prompt chunks: whole key ranges per block of 128 query rows, when
        // those blocks fill the device (fewer, and the split form's key
        // splits spread the work wider: 1 x 1024 rows 105 against 111 us)
        constexpr size_t shmem = FaShape<D>::LDS_BYTES;
        const int64_t fa_blocks = (nqry + kFaRows - 1) / kFaRows * nkv * B;
        if (nqry >= kFaRows && fa_enabled() && fa_blocks >= attn_device_cus()) {
            static std::atomic<uint8_t> allowed[64];
            int dev = 0;
            if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return invalid("gqa_verify_mfma: device");
            if (!allowed[dev].load(std::memory_order_acquire)) {
                const int rc = check_hip(hipFuncSetAttribute(reinterpret_cast<const void*>(gqa_fa_kernel<D>),
                                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                                             static_cast<int>(shmem)),
                                         "hipFuncSetAttribute");
                if (rc != HAI_OK) return rc;
                allowed[dev].store(1, std::memory_order_release);
            }
            const dim3 grid(static_cast<unsigned>((nqry + kFaRows - 1) / kFaRows), nkv, B);
            const float sl2 = 1.4426950408889634f / __builtin_sqrtf(static_cast<float>(D));
            gqa_fa_kernel<D><<<grid, dim3(256), shmem, s>>>(out, q, gate, kc, vc, cap, T, nq, nkv, lens, len_add, sl2);
            return launched("gqa_fa_kernel");
        }
    }
    const void* kern = nqry <= 16 ? reinterpret_cast<const void*>(gqa_mfma_partial_kernel<D, 1>)
                                  : reinterpret_cast<const void*>(gqa_mfma_partial_kernel<D, 2>);
    const int64_t resident = resident_blocks(kern, 0);
    const MfmaPlan p = mfma_plan(D, B, T, nq, nkv, max_len, resident > 0 ? resident : kMfmaTargetBlocks);
    const float scale_log2 = 1.4426950408889634f / __builtin_sqrtf(static_cast<float>(D));
    const dim3 grid(p.nsplit, nkv * p.qgroups, B);
    if (p.qt == 1)
        gqa_mfma_partial_kernel<D, 1><<<grid, dim3(256), 0, s>>>(scratch, q, kc, vc, cap, T, nq, nkv, lens, len_add,
                                                                 p.nsplit, p.steps, scale_log2);
    else
        gqa_mfma_partial_kernel<D, 2><<<grid, dim3(256), 0, s>>>(scratch, q, kc, vc, cap, T, nq, nkv, lens, len_add,
                                                                 p.nsplit, p.steps, scale_log2);
    int rc = launched("gqa_mfma_partial_kernel");
    if (rc != HAI_OK) return rc;
    const int64_t nall = static_cast<int64_t>(B) * T * nq;
    // a block per query row when a row merges many splits (decode), a wave
    // per row when there are many rows of few splits (prompt chunks); the
    // two forms give the same bits
    if (p.nsplit >= kCombineBlockSplits)
        gqa_mfma_combine_kernel<D><<<dim3(static_cast<unsigned>(nall)), dim3(D), 0, s>>>(
            out, scratch, gate, B, T, nq, lens, len_add, p.nsplit, p.block_keys);
    else
        gqa_mfma_combine_wave_kernel<D><<<dim3(static_cast<unsigned>((nall + 3) / 4)), dim3(256), 0, s>>>(
            out, scratch, gate, B, T, nq, lens, len_add, p.nsplit, p.block_keys);
    return launched("gqa_mfma_combine_kernel");
}

// ---- the allocation-free entry point --------------------------------------
// hai_gqa_verify_noalloc_bf16 keeps its split-KV partials in this file-scope
// device array instead of a caller workspace: each GPU the library runs on
// holds its own copy (kGqaNoAllocScratchBytes) from module load until the
// process ends.  Host code never passes the array's name to a kernel (on
// the host it is only a stand-in for the symbol): the device address comes
// from hipGetSymbolAddress, resolved once per device with that device
// current on the entry point's first call there, and kept per device.
constexpr size_t kGqaNoAllocScratchBytes = size_t{16} << 20;
static __device__ __align__(256) float gqa_noalloc_scratch[kGqaNoAllocScratchBytes / sizeof(float)];

constexpr int kMaxNoAllocDevices = 64;
std::atomic<float*> g_noalloc_ptr[kMaxNoAllocDevices];
std::mutex g_noalloc_mu;

// The product of the factors as a byte count, or SIZE_MAX when a factor is
// negative or the product overflows.
size_t checked_product(std::initializer_list<int64_t> factors) {
    uint64_t p = 1;
    for (const int64_t v : factors)
        if (v < 0 || __builtin_mul_overflow(p, static_cast<uint64_t>(v), &p)) return SIZE_MAX;
    return static_cast<size_t>(p);
}

int noalloc_scratch(float** out) {
    int dev = 0;
    int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
    if (rc != HAI_OK) return rc;
    if (dev < 0 || dev >= kMaxNoAllocDevices) return invalid("gqa_verify_noalloc: device ordinal above 63");
    float* p = g_noalloc_ptr[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        std::lock_guard<std::mutex> lock(g_noalloc_mu);
        p = g_noalloc_ptr[dev].load(std::memory_order_acquire);
        if (p == nullptr) {
            void* sym = nullptr;
            rc = check_hip(hipGetSymbolAddress(&sym, HIP_SYMBOL(gqa_noalloc_scratch)), "hipGetSymbolAddress");
            if (rc != HAI_OK) return rc;
            p = static_cast<float*>(sym);
            g_noalloc_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return HAI_OK;
}

}  // namespace

extern "C" {

int hai_gqa_verify_noalloc_bf16(void* out, const void* q, const void* gate, const void* k_cache,
                                const void* v_cache, int64_t cap, int64_t B, int64_t T, int64_t nq, int64_t nkv,
                                int64_t D, const int32_t* lens, int32_t len_add, int64_t max_len, void* stream) {
    // every operand of the size bounded before the size is computed
    if (B < 0 || T < 0 || nq <= 0 || nkv <= 0 || max_len <= 0 || B > INT32_MAX || T > INT32_MAX ||
        nq > INT32_MAX || max_len > INT32_MAX)
        return invalid("gqa_verify_noalloc: shape");
    if (D != 64 && D != 128 && D != 256) return invalid("gqa_verify_noalloc: head_dim must be 64, 128 or 256");
    const size_t need = hai_gqa_scratch_bytes(B, T, nq, D, max_len);
    if (need > kGqaNoAllocScratchBytes)
        return invalid(("gqa_verify_noalloc: the partials need " + std::to_string(need) +
                        " bytes, above the fixed 16 MiB scratch (use hai_gqa_verify_bf16 with a workspace)")
                           .c_str());
    float* ptr = nullptr;
    const int rc = noalloc_scratch(&ptr);
    if (rc != HAI_OK) return rc;
    return hai_gqa_verify_bf16(out, q, gate, k_cache, v_cache, cap, ptr, B, T, nq, nkv, D, lens, len_add, max_len,
                               stream);
}

size_t hai_gqa_scratch_bytes(int64_t B, int64_t T, int64_t nq, int64_t D, int64_t max_len) {
    if (D < 0 || D > INT32_MAX || max_len < 0) return SIZE_MAX;
    const int64_t nchunk = (max_len + kChunk - 1) / kChunk;
    return checked_product({B, T, nq, nchunk < 1 ? 1 : nchunk, partial_stride(int(D)), int64_t{sizeof(float)}});
}

int hai_gqa_verify_bf16(void* out, const void* q, const void* gate, const void* k_cache,
                        const void* v_cache, int64_t cap, void* scratch, int64_t B, int64_t T, int64_t nq,
                        int64_t nkv, int64_t D, const int32_t* lens, int32_t len_add, int64_t max_len,
                        void* stream) {
    if (out == nullptr || q == nullptr || k_cache == nullptr || v_cache == nullptr || scratch == nullptr)
        return invalid("gqa_verify: null pointer");
    if (B < 0 || T < 0 || nq <= 0 || nkv <= 0 || nq % nkv != 0 || cap <= 0 || max_len <= 0 ||
        max_len > cap || T > max_len || B > INT32_MAX || nq > INT32_MAX || max_len > INT32_MAX)
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

int hai_gqa_verify_fused_bf16(void* out, void* gate_out, const void* proj, int64_t ld_proj, const void* q_norm,
                              const void* k_norm, const float* rope_cos, const float* rope_sin,
                              int64_t rope_positions, int64_t R, float eps, void* k_cache, void* v_cache,
                              int64_t cap, void* scratch, int64_t B, int64_t T, int64_t nq, int64_t nkv, int64_t D,
                              const int32_t* lens, int32_t len_add, int64_t max_len, void* stream) {
    if (out == nullptr || gate_out == nullptr || proj == nullptr || q_norm == nullptr || k_norm == nullptr ||
        rope_cos == nullptr || rope_sin == nullptr || k_cache == nullptr || v_cache == nullptr || scratch == nullptr)
        return invalid("gqa_verify_fused: null pointer");
    if (B < 0 || T < 0 || nq <= 0 || nkv <= 0 || nq % nkv != 0 || cap <= 0 || max_len <= 0 || max_len > cap ||
        T > max_len || B > INT32_MAX || nq > INT32_MAX || max_len > INT32_MAX || R < 0 || R > D || R % 2 != 0 ||
        rope_positions <= 0 || ld_proj < (2 * nq + 2 * nkv) * D)
        return invalid("gqa_verify_fused: shape");
    if (lens == nullptr && (len_add < T || len_add > max_len))
        return invalid("gqa_verify_fused: cache length must cover the T new rows and stay within max_len");
    if (!aligned16(k_cache) || !aligned16(v_cache) || !aligned16(proj) || ld_proj % 8 != 0)
        return invalid("gqa_verify_fused: alignment");
    if (B == 0 || T == 0) return HAI_OK;
    const int nchunk = static_cast<int>((max_len + kChunk - 1) / kChunk);
    QkvFuse F;
    F.proj = static_cast<const uint16_t*>(proj);
    F.ld = ld_proj;
    F.wq = static_cast<const uint16_t*>(q_norm);
    F.wk = static_cast<const uint16_t*>(k_norm);
    F.rc = rope_cos;
    F.rs = rope_sin;
    F.rope_pos = rope_positions;
    F.R = int(R);
    F.eps = eps;
    F.gate_out = static_cast<uint16_t*>(gate_out);
    F.kc = static_cast<uint16_t*>(k_cache);
    F.vc = static_cast<uint16_t*>(v_cache);
    const auto s = as_stream(stream);
    auto* o = static_cast<uint16_t*>(out);
    const auto* kc = static_cast<const uint16_t*>(k_cache);
    const auto* vc = static_cast<const uint16_t*>(v_cache);
    auto* sc = static_cast<float*>(scratch);
    const auto* g = static_cast<const uint16_t*>(gate_out);
    switch (D) {
        case 64: return launch<64, true>(o, nullptr, g, kc, vc, cap, sc, int(B), int(T), int(nq), int(nkv), lens, len_add, nchunk, s, F);
        case 128: return launch<128, true>(o, nullptr, g, kc, vc, cap, sc, int(B), int(T), int(nq), int(nkv), lens, len_add, nchunk, s, F);
        case 256: return launch<256, true>(o, nullptr, g, kc, vc, cap, sc, int(B), int(T), int(nq), int(nkv), lens, len_add, nchunk, s, F);
        default: return invalid("gqa_verify_fused: head_dim must be 64, 128 or 256");
    }
}

size_t hai_gqa_mfma_plan_scratch_bytes(int64_t B, int64_t T, int64_t nq, int64_t nkv, int64_t D,
                                       int64_t max_len) {
    if (B <= 0 || T <= 0 || nq <= 0 || nkv <= 0 || nq % nkv != 0 || max_len <= 0) return 0;
    if (D != 64 && D != 128 && D != 256) return hai_gqa_mfma_scratch_bytes(B, T, nq, D, max_len);
    const int64_t nqry = T * (nq / nkv);
    const void* kern = nullptr;
    switch (D) {
        case 64: kern = nqry <= 16 ? reinterpret_cast<const void*>(gqa_mfma_partial_kernel<64, 1>)
                                   : reinterpret_cast<const void*>(gqa_mfma_partial_kernel<64, 2>); break;
        case 128: kern = nqry <= 16 ? reinterpret_cast<const void*>(gqa_mfma_partial_kernel<128, 1>)
                                    : reinterpret_cast<const void*>(gqa_mfma_partial_kernel<128, 2>); break;
        default: kern = nqry <= 16 ? reinterpret_cast<const void*>(gqa_mfma_partial_kernel<256, 1>)
                                   : reinterpret_cast<const void*>(gqa_mfma_partial_kernel<256, 2>); break;
    }
    const int64_t resident = resident_blocks(kern, 0);
    const MfmaPlan p = mfma_plan(int(D), B, T, nq, nkv, max_len, resident > 0 ? resident : kMfmaTargetBlocks);
    return static_cast<size_t>(B * T * nq * p.nsplit * mfma_part_stride(int(D))) * sizeof(float);
}

size_t hai_gqa_mfma_scratch_bytes(int64_t B, int64_t T, int64_t nq, int64_t D, int64_t max_len) {
    // at most one split per kMfmaMinBlockKeys keys
    const int64_t nsplit = (max_len + kMfmaMinBlockKeys - 1) / kMfmaMinBlockKeys;
    return static_cast<size_t>(B * T * nq * (nsplit < 1 ? 1 : nsplit) * mfma_part_stride(int(D))) * sizeof(float);
}

int hai_gqa_verify_mfma_bf16(void* out, const void* q, const void* gate, const void* k_cache,
                             const void* v_cache, int64_t cap, void* scratch, int64_t B, int64_t T, int64_t nq,
                             int64_t nkv, int64_t D, const int32_t* lens, int32_t len_add, int64_t max_len,
                             void* stream) {
    if (out == nullptr || q == nullptr || k_cache == nullptr || v_cache == nullptr || scratch == nullptr)
        return invalid("gqa_verify_mfma: null pointer");
    if (B < 0 || T < 0 || nq <= 0 || nkv <= 0 || nq % nkv != 0 || cap <= 0 || max_len <= 0 ||
        max_len > cap || T > max_len)
        return invalid("gqa_verify_mfma: shape");
    if (lens == nullptr && (len_add < T || len_add > max_len))
        return invalid("gqa_verify_mfma: cache length must cover the T new rows and stay within max_len");
    if (!aligned16(k_cache) || !aligned16(v_cache) || !aligned16(q) || !aligned16(scratch))
        return invalid("gqa_verify_mfma: alignment");
    if (B == 0 || T == 0) return HAI_OK;
    const auto s = as_stream(stream);
    auto* o = static_cast<uint16_t*>(out);
    const auto* qq = static_cast<const uint16_t*>(q);
    const auto* g = static_cast<const uint16_t*>(gate);
    const auto* kc = static_cast<const uint16_t*>(k_cache);
    const auto* vc = static_cast<const uint16_t*>(v_cache);
    auto* sc = static_cast<float*>(scratch);
    switch (D) {
        case 64: return launch_mfma<64>(o, qq, g, kc, vc, cap, sc, int(B), int(T), int(nq), int(nkv), lens, len_add, max_len, s);
        case 128: return launch_mfma<128>(o, qq, g, kc, vc, cap, sc, int(B), int(T), int(nq), int(nkv), lens, len_add, max_len, s);
        case 256: return launch_mfma<256>(o, qq, g, kc, vc, cap, sc, int(B), int(T), int(nq), int(nkv), lens, len_add, max_len, s);
        default: return invalid("gqa_verify_mfma: head_dim must be 64, 128 or 256");
    }
}

}  // extern "C"
