// backend_parity.cc -- the MI355X hybridai::Backend seen the way the
// reference's ops see it: created by name through BackendRegistry
// ("hip"), driven only through the Backend virtuals, every result compared
// bit for bit with the CPU oracle (oracle/liboracle.so).
//
//   backend_parity --cpu   registry, kernel-registry keys and the
//                          NotImplemented fallbacks (no device calls)
//   backend_parity         the above plus every path virtual on the GPU
//
// Exit status 0 when every check passes; each failure prints one line.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "mi355x_backend.h"
#include "oracle.h"

using namespace hybridai;

namespace {

int g_fail = 0, g_pass = 0;

void expect(bool ok, const std::string& what) {
    if (ok) {
        ++g_pass;
    } else {
        ++g_fail;
        std::printf("FAIL %s\n", what.c_str());
    }
}

void expect_ok(const Status& st, const std::string& what) {
    expect(st.ok(), what + (st.ok() ? "" : " -> " + st.message()));
}

uint16_t to_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}
float from_bf16(uint16_t h) {
    const uint32_t u = static_cast<uint32_t>(h) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

struct Bf16 {
    std::vector<uint16_t> bits;
    std::vector<float> f;  // the same values as float
};

Bf16 random_bf16(std::mt19937& rng, size_t n, float scale = 1.0f) {
    std::normal_distribution<float> nd(0.0f, scale);
    Bf16 r;
    r.bits.resize(n);
    r.f.resize(n);
    for (size_t i = 0; i < n; ++i) {
        r.bits[i] = to_bf16(nd(rng));
        r.f[i] = from_bf16(r.bits[i]);
    }
    return r;
}

struct Dev {
    Backend* be;
    std::shared_ptr<Buffer> make(size_t bytes) { return be->create_buffer(bytes, MemoryType::Device); }
    template <typename T>
    std::shared_ptr<Buffer> up(const std::vector<T>& h) {
        auto b = make(h.size() * sizeof(T));
        expect_ok(be->memcpy_h2d(b.get(), h.data(), h.size() * sizeof(T)), "upload");
        return b;
    }
    template <typename T>
    std::vector<T> down(const Buffer* b, size_t n) {
        std::vector<T> h(n);
        expect_ok(be->memcpy_d2h(h.data(), b, n * sizeof(T)), "download");
        return h;
    }
};

// got: bf16 bits; want: oracle floats already rounded to bf16.
void same_bits(const std::vector<uint16_t>& got, const std::vector<float>& want, const std::string& what) {
    size_t bad = 0, first = 0;
    for (size_t i = 0; i < want.size(); ++i)
        if (got[i] != to_bf16(want[i])) {
            if (bad++ == 0) first = i;
        }
    expect(bad == 0, what + (bad ? " (" + std::to_string(bad) + " mismatches, first at " + std::to_string(first) +
                                       ")"
                                 : ""));
}

void check_cpu(Backend* be) {
    expect(std::string(be->name()) == "hip", "backend name");
    expect(be->device().backend() == "hip" && be->device().type() == DeviceType::DiscreteGPU, "backend device");
    for (DeviceType t : {DeviceType::DiscreteGPU, DeviceType::IntegratedGPU})
        expect(ops::KernelRegistry::instance().has_kernel(ops::KernelKey{"noop", t, DType::FP32}),
               "noop kernel registered");
    // Forms outside the path report NotImplemented before touching the device.
    Status st = be->gemm(nullptr, nullptr, nullptr, DType::FP32, DType::FP32, DType::FP32, DType::FP32, false, true,
                         2, 3, 8, 1.0f, 0.0f);
    expect(st.code() == StatusCode::NotImplemented, "fp32 gemm falls back");
    st = be->add(nullptr, nullptr, nullptr, DType::FP32, 4);
    expect(st.code() == StatusCode::NotImplemented, "fp32 add falls back");
    st = be->cast(nullptr, nullptr, DType::FP32, DType::BF16, 4);
    expect(st.code() == StatusCode::NotImplemented, "cast is optional");
    st = be->gemm(nullptr, nullptr, nullptr, DType::BF16, DType::BF16, DType::BF16, DType::FP32, false, true, 0, 3,
                  8, 1.0f, 0.0f);
    expect(st.code() == StatusCode::InvalidArgument, "gemm rejects m = 0");
}

void check_gpu(Backend* be) {
    Dev d{be};
    std::mt19937 rng(1234);

    // gemm: Linear Y = X W^T; 20 rows (two 16-row batches of one launch) and
    // a 512-row prompt at the 27B hidden size (32 batches, the weights
    // streamed once by the launch)
    for (const int64_t M : {int64_t{20}, int64_t{512}}) {
        const int64_t N = M == 20 ? 300 : 5120, K = M == 20 ? 256 : 5120;
        auto x = random_bf16(rng, M * K), w = random_bf16(rng, N * K, 0.05f);
        auto dx = d.up(x.bits), dw = d.up(w.bits), dy = d.make(M * N * 2);
        expect_ok(be->gemm(dy.get(), dx.get(), dw.get(), DType::BF16, DType::BF16, DType::BF16, DType::FP32, false,
                           true, M, N, K, 1.0f, 0.0f),
                  "gemm");
        std::vector<float> want(M * N);
        orc_gemm(x.f.data(), w.f.data(), want.data(), M, N, K, 1);
        same_bits(d.down<uint16_t>(dy.get(), M * N), want, "gemm M=" + std::to_string(M));
    }
    {  // add, silu_mul
        const int64_t n = 1000;
        auto a = random_bf16(rng, n), b = random_bf16(rng, n);
        auto da = d.up(a.bits), db = d.up(b.bits), dy = d.make(n * 2);
        std::vector<float> want(n);
        expect_ok(be->add(dy.get(), da.get(), db.get(), DType::BF16, n), "add");
        orc_add(a.f.data(), b.f.data(), want.data(), n, 1);
        same_bits(d.down<uint16_t>(dy.get(), n), want, "add");
        expect_ok(be->silu_mul(dy.get(), da.get(), db.get(), DType::BF16, n), "silu_mul");
        orc_silu_mul(a.f.data(), b.f.data(), want.data(), n, 1);
        same_bits(d.down<uint16_t>(dy.get(), n), want, "silu_mul");
    }
    {  // embedding_gather (out-of-range ids give zero rows)
        const int64_t V = 50, H = 64;
        auto tab = random_bf16(rng, V * H);
        std::vector<int64_t> ids = {3, 0, 49, 50, -1, 7};
        auto dt = d.up(tab.bits), di = d.up(ids), dy = d.make(ids.size() * H * 2);
        expect_ok(be->embedding_gather(dy.get(), dt.get(), di.get(), DType::BF16, ids.size(), V, H), "embedding");
        std::vector<float> want(ids.size() * H);
        orc_embedding(tab.f.data(), ids.data(), want.data(), ids.size(), V, H);
        same_bits(d.down<uint16_t>(dy.get(), want.size()), want, "embedding_gather");
    }
    for (bool unit : {true, false}) {  // rmsnorm
        const int64_t rows = 3, H = 256;
        auto x = random_bf16(rng, rows * H), w = random_bf16(rng, H, 0.02f);
        auto dx = d.up(x.bits), dw = d.up(w.bits), dy = d.make(rows * H * 2);
        expect_ok(be->rmsnorm(dy.get(), dx.get(), dw.get(), DType::BF16, rows, H, 1e-6f, unit), "rmsnorm");
        std::vector<float> want(rows * H);
        orc_rmsnorm(x.f.data(), w.f.data(), want.data(), rows, H, 1e-6f, unit ? 1 : 0, 1);
        same_bits(d.down<uint16_t>(dy.get(), want.size()), want, unit ? "rmsnorm(+1)" : "rmsnorm");
    }
    {  // partial_rope
        const int64_t T = 3, heads = 4, D = 64, R = 16, pos = 5;
        auto x = random_bf16(rng, T * heads * D);
        auto dx = d.up(x.bits), dy = d.make(x.bits.size() * 2);
        expect_ok(be->partial_rope(dy.get(), dx.get(), DType::BF16, T, heads, D, R, pos, 1.0e7f), "partial_rope");
        std::vector<float> want(x.f.size());
        orc_partial_rope(x.f.data(), want.data(), T, heads, D, R, pos, 1.0e7f, 1);
        same_bits(d.down<uint16_t>(dy.get(), want.size()), want, "partial_rope");
    }
    {  // q_gate_rmsnorm_rope
        const int64_t T = 2, nq = 4, D = 64, R = 16, pos = 9;
        auto src = random_bf16(rng, T * nq * 2 * D), w = random_bf16(rng, D, 0.02f);
        auto ds = d.up(src.bits), dw = d.up(w.bits), dq = d.make(T * nq * D * 2), dg = d.make(T * nq * D * 2);
        expect_ok(be->q_gate_rmsnorm_rope(dq.get(), dg.get(), ds.get(), dw.get(), DType::BF16, T, nq, D, R, pos,
                                          1.0e7f, 1e-6f, true),
                  "q_gate_rmsnorm_rope");
        std::vector<float> wq(T * nq * D), wg(T * nq * D);
        orc_q_gate_rmsnorm_rope(src.f.data(), w.f.data(), wq.data(), wg.data(), T, nq, D, R, pos, 1.0e7f, 1e-6f, 1, 1);
        same_bits(d.down<uint16_t>(dq.get(), wq.size()), wq, "q_gate_rmsnorm_rope q");
        same_bits(d.down<uint16_t>(dg.get(), wg.size()), wg, "q_gate_rmsnorm_rope gate");
    }
    {  // append_kv_cache + cached_gqa + cached_gqa_with_current_token
        const int64_t nq = 4, nkv = 2, D = 64, cap = 100, L = 70, T = 3, row = nkv * D;
        auto k = random_bf16(rng, L * row), v = random_bf16(rng, L * row);
        auto kc = d.make(cap * row * 2), vc = d.make(cap * row * 2);
        auto dk1 = d.up(std::vector<uint16_t>(k.bits.begin(), k.bits.begin() + 50 * row));
        auto dv1 = d.up(std::vector<uint16_t>(v.bits.begin(), v.bits.begin() + 50 * row));
        auto dk2 = d.up(std::vector<uint16_t>(k.bits.begin() + 50 * row, k.bits.end()));
        auto dv2 = d.up(std::vector<uint16_t>(v.bits.begin() + 50 * row, v.bits.end()));
        expect_ok(be->append_kv_cache(kc.get(), vc.get(), dk1.get(), dv1.get(), DType::BF16, 50, nkv, D, 0, cap),
                  "append at 0");
        expect_ok(be->append_kv_cache(kc.get(), vc.get(), dk2.get(), dv2.get(), DType::BF16, 20, nkv, D, 50, cap),
                  "append at offset");
        Status st = be->append_kv_cache(kc.get(), vc.get(), dk2.get(), dv2.get(), DType::BF16, 20, nkv, D, 90, cap);
        expect(st.code() == StatusCode::InvalidArgument, "append past capacity rejected");
        auto got_k = d.down<uint16_t>(kc.get(), L * row);
        expect(got_k == k.bits, "appended keys");
        auto q = random_bf16(rng, T * nq * D), g = random_bf16(rng, T * nq * D);
        auto dq = d.up(q.bits), dg = d.up(g.bits), dy = d.make(T * nq * D * 2);
        expect_ok(be->cached_gqa(dy.get(), dq.get(), kc.get(), vc.get(), dg.get(), DType::BF16, T, L, nq, nkv, D),
                  "cached_gqa");
        std::vector<float> want(T * nq * D);
        orc_attention(q.f.data(), g.f.data(), k.f.data(), v.f.data(), want.data(), T, L, nq, nkv, D, 1);
        same_bits(d.down<uint16_t>(dy.get(), want.size()), want, "cached_gqa");
        // the last query row alone, its key/value row passed separately
        auto q1 = Bf16{std::vector<uint16_t>(q.bits.end() - nq * D, q.bits.end()),
                       std::vector<float>(q.f.end() - nq * D, q.f.end())};
        auto g1 = Bf16{std::vector<uint16_t>(g.bits.end() - nq * D, g.bits.end()),
                       std::vector<float>(g.f.end() - nq * D, g.f.end())};
        auto dq1 = d.up(q1.bits), dg1 = d.up(g1.bits), dy1 = d.make(nq * D * 2);
        auto ck = d.up(std::vector<uint16_t>(k.bits.end() - row, k.bits.end()));
        auto cv = d.up(std::vector<uint16_t>(v.bits.end() - row, v.bits.end()));
        expect_ok(be->cached_gqa_with_current_token(dy1.get(), dq1.get(), kc.get(), vc.get(), ck.get(), cv.get(),
                                                    dg1.get(), DType::BF16, L, nq, nkv, D),
                  "cached_gqa_with_current_token");
        std::vector<float> want1(nq * D);
        orc_attention(q1.f.data(), g1.f.data(), k.f.data(), v.f.data(), want1.data(), 1, L, nq, nkv, D, 1);
        same_bits(d.down<uint16_t>(dy1.get(), want1.size()), want1, "cached_gqa_with_current_token");
    }
    for (bool gated : {true, false}) {  // causal_gqa (uncached prompt attention, hip_kernels.hip:223-293)
        const int64_t nq = 4, nkv = 2, D = 64, S = 70;  // two query chunks of the backend's 64
        auto q = random_bf16(rng, S * nq * D), g = random_bf16(rng, S * nq * D);
        auto k = random_bf16(rng, S * nkv * D), v = random_bf16(rng, S * nkv * D);
        auto dq = d.up(q.bits), dg = d.up(g.bits), dk = d.up(k.bits), dv = d.up(v.bits);
        auto dy = d.make(S * nq * D * 2);
        expect_ok(be->causal_gqa(dy.get(), dq.get(), dk.get(), dv.get(), gated ? dg.get() : nullptr, DType::BF16, S,
                                 nq, nkv, D),
                  "causal_gqa");
        std::vector<float> want(S * nq * D);
        orc_attention(q.f.data(), gated ? g.f.data() : nullptr, k.f.data(), v.f.data(), want.data(), S, S, nq, nkv,
                      D, 1);
        same_bits(d.down<uint16_t>(dy.get(), want.size()), want, gated ? "causal_gqa gated" : "causal_gqa");
        auto small = d.make(16);
        Status st = be->causal_gqa(small.get(), dq.get(), dk.get(), dv.get(), nullptr, DType::BF16, S, nq, nkv, D);
        expect(st.code() == StatusCode::InvalidArgument, "causal_gqa short dst rejected");
    }
    {  // cached_gqa_with_current_token as a T=1 decode drives it (attention.cc:561-571): the
       // current K/V row is passed separately, the call stores it at cache_len-1
       // (hip_kernels.hip:466-476) and the caller only advances the length
        const int64_t nq = 4, nkv = 2, D = 64, cap = 80, L = 65, row = nkv * D;
        auto k = random_bf16(rng, (L + 1) * row), v = random_bf16(rng, (L + 1) * row);
        auto kc = d.make(cap * row * 2), vc = d.make(cap * row * 2);
        expect_ok(be->memset(kc.get(), 0, cap * row * 2), "zero K cache");
        expect_ok(be->memset(vc.get(), 0, cap * row * 2), "zero V cache");
        auto dk = d.up(std::vector<uint16_t>(k.bits.begin(), k.bits.begin() + (L - 1) * row));
        auto dv = d.up(std::vector<uint16_t>(v.bits.begin(), v.bits.begin() + (L - 1) * row));
        expect_ok(be->append_kv_cache(kc.get(), vc.get(), dk.get(), dv.get(), DType::BF16, L - 1, nkv, D, 0, cap),
                  "prefix rows");
        for (int64_t step = 0; step < 2; ++step) {
            const int64_t len = L + step;  // rows 0..len-2 cached, row len-1 is the current token
            auto q = random_bf16(rng, nq * D), g = random_bf16(rng, nq * D);
            auto dq = d.up(q.bits), dg = d.up(g.bits), dy = d.make(nq * D * 2);
            auto ck = d.up(std::vector<uint16_t>(k.bits.begin() + (len - 1) * row, k.bits.begin() + len * row));
            auto cv = d.up(std::vector<uint16_t>(v.bits.begin() + (len - 1) * row, v.bits.begin() + len * row));
            const std::string tag = " (decode step " + std::to_string(step) + ")";
            expect_ok(be->cached_gqa_with_current_token(dy.get(), dq.get(), kc.get(), vc.get(), ck.get(), cv.get(),
                                                        dg.get(), DType::BF16, len, nq, nkv, D),
                      "cached_gqa_with_current_token" + tag);
            std::vector<float> want(nq * D);
            orc_attention(q.f.data(), g.f.data(), k.f.data(), v.f.data(), want.data(), 1, len, nq, nkv, D, 1);
            same_bits(d.down<uint16_t>(dy.get(), want.size()), want, "current-token output" + tag);
            expect(d.down<uint16_t>(kc.get(), len * row) ==
                       std::vector<uint16_t>(k.bits.begin(), k.bits.begin() + len * row),
                   "K cache holds the current row" + tag);
            expect(d.down<uint16_t>(vc.get(), len * row) ==
                       std::vector<uint16_t>(v.bits.begin(), v.bits.begin() + len * row),
                   "V cache holds the current row" + tag);
        }
        auto dq = d.make(nq * D * 2), dy = d.make(nq * D * 2), small = d.make((L - 1) * row * 2);
        Status st = be->cached_gqa_with_current_token(dy.get(), dq.get(), small.get(), small.get(), dq.get(),
                                                      dq.get(), nullptr, DType::BF16, L, nq, nkv, D);
        expect(st.code() == StatusCode::InvalidArgument, "caches must hold cache_len rows");
    }
    {  // deltanet_grouped_conv + deltanet_recurrent on the reference layouts
        const int64_t nk = 2, nv = 4, dk = 64, dv = 64, Kc = 4, T = 5;
        const int64_t kw = nk * dk, vw = nv * dv, C = 2 * kw + vw;
        auto qkv = random_bf16(rng, T * C), cw = random_bf16(rng, C * Kc, 0.5f), cs = random_bf16(rng, C * (Kc - 1));
        auto dqkv = d.up(qkv.bits), dcw = d.up(cw.bits), dcs = d.up(cs.bits);
        auto dq = d.make(T * kw * 2), dk_ = d.make(T * kw * 2), dvv = d.make(T * vw * 2);
        expect_ok(be->deltanet_grouped_conv(dq.get(), dk_.get(), dvv.get(), dcs.get(), dqkv.get(), dcw.get(),
                                            DType::BF16, T, nk, nv, dk, dv, Kc),
                  "deltanet_grouped_conv");
        std::vector<float> st_f = cs.f, wq(T * kw), wk(T * kw), wv(T * vw);
        orc_deltanet_conv(qkv.f.data(), cw.f.data(), st_f.data(), wq.data(), wk.data(), wv.data(), T, nk, nv, dk, dv,
                          Kc, 1);
        same_bits(d.down<uint16_t>(dq.get(), wq.size()), wq, "conv q");
        same_bits(d.down<uint16_t>(dk_.get(), wk.size()), wk, "conv k");
        same_bits(d.down<uint16_t>(dvv.get(), wv.size()), wv, "conv v");
        same_bits(d.down<uint16_t>(dcs.get(), st_f.size()), st_f, "conv state");

        for (int64_t TR : {int64_t{3}, int64_t{20}}) {
            auto q = random_bf16(rng, TR * kw), k = random_bf16(rng, TR * kw), v = random_bf16(rng, TR * vw);
            auto a = random_bf16(rng, TR * nv), b = random_bf16(rng, TR * nv), z = random_bf16(rng, TR * vw);
            auto al = random_bf16(rng, nv, 0.5f), dt = random_bf16(rng, nv, 0.5f), nw = random_bf16(rng, dv, 0.1f);
            std::normal_distribution<float> nd(0.0f, 0.1f);
            std::vector<float> state(nv * dk * dv);
            for (auto& s : state) s = nd(rng);
            auto bq = d.up(q.bits), bk = d.up(k.bits), bv = d.up(v.bits), ba = d.up(a.bits), bb = d.up(b.bits),
                 bz = d.up(z.bits), bal = d.up(al.bits), bdt = d.up(dt.bits), bnw = d.up(nw.bits),
                 bst = d.up(state), bo = d.make(TR * vw * 2);
            expect_ok(be->deltanet_recurrent(bo.get(), bst.get(), bq.get(), bk.get(), bv.get(), ba.get(), bb.get(),
                                             bal.get(), bdt.get(), bnw.get(), bz.get(), DType::BF16, TR, nk, nv, dk,
                                             dv, 1e-6f),
                      "deltanet_recurrent");
            std::vector<float> want(TR * vw), st2 = state;
            orc_deltanet_recurrent(q.f.data(), k.f.data(), v.f.data(), a.f.data(), b.f.data(), z.f.data(),
                                   al.f.data(), dt.f.data(), nw.f.data(), st2.data(), want.data(), TR, nk, nv, dk, dv,
                                   1e-6f, 1);
            same_bits(d.down<uint16_t>(bo.get(), want.size()), want, "recurrent out T=" + std::to_string(TR));
            auto got_st = d.down<float>(bst.get(), st2.size());
            expect(std::memcmp(got_st.data(), st2.data(), st2.size() * 4) == 0,
                   "recurrent state T=" + std::to_string(TR));
        }
    }
    {  // argmax_rows / argmax_last_row (ties -> first index)
        const int64_t rows = 3, cols = 1000;
        auto x = random_bf16(rng, rows * cols);
        x.bits[1 * cols + 10] = x.bits[1 * cols + 700] = to_bf16(50.0f);
        for (size_t i = 0; i < x.f.size(); ++i) x.f[i] = from_bf16(x.bits[i]);
        auto dx = d.up(x.bits), dy = d.make(rows * 8);
        std::vector<int64_t> want(rows);
        orc_argmax_rows(x.f.data(), want.data(), rows, cols);
        expect_ok(be->argmax_rows(dy.get(), dx.get(), DType::BF16, rows, cols), "argmax_rows");
        expect(d.down<int64_t>(dy.get(), rows) == want, "argmax_rows ids");
        expect_ok(be->argmax_last_row(dy.get(), dx.get(), DType::BF16, rows, cols), "argmax_last_row");
        expect(d.down<int64_t>(dy.get(), 1)[0] == want[rows - 1], "argmax_last_row id");
    }
    {  // copies, memset, streams and events
        std::vector<uint16_t> h(256);
        for (size_t i = 0; i < h.size(); ++i) h[i] = static_cast<uint16_t>(i * 7);
        auto a = d.up(h), b = d.make(512);
        auto s = be->create_stream();
        auto e0 = be->create_event(), e1 = be->create_event();
        expect(s && e0 && e1, "stream and events");
        expect_ok(be->memset(b.get(), 0, 512, s.get()), "memset");
        expect_ok(e0->record(s.get()), "event record");
        expect_ok(be->copy_to_offset(b.get(), 128, a.get(), 64, 256, s.get()), "copy_to_offset");
        expect_ok(e1->record(s.get()), "event record");
        expect_ok(e1->synchronize(), "event synchronize");
        double ms = -1.0;
        expect_ok(e1->elapsed_time_since(*e0, &ms), "elapsed");
        expect(ms >= 0.0, "elapsed time");
        auto got = d.down<uint8_t>(b.get(), 512);
        bool ok = true;
        for (int i = 0; i < 512; ++i) {
            const uint8_t want = (i >= 128 && i < 384) ? reinterpret_cast<const uint8_t*>(h.data())[64 + i - 128] : 0;
            ok = ok && got[i] == want;
        }
        expect(ok, "copy_to_offset contents");
        {  // create_buffer recycles blocks of released buffers (the reference's pool, hip_backend.cc:380-500)
            auto* mb = dynamic_cast<MI355XBackend*>(be);
            expect(mb != nullptr, "backend type");
            void* first = nullptr;
            {
                auto t = be->create_buffer(3000, MemoryType::Device);
                expect(t != nullptr && t->size() == 3000, "pooled buffer size");
                first = t->data();
            }
            expect(mb->pooled_bytes(MemoryType::Device) >= 3072, "released block kept for reuse");
            auto t2 = be->create_buffer(2900, MemoryType::Device);  // same 3072-byte class
            expect(t2 != nullptr && t2->data() == first, "block reused for a request of the same class");
            auto big = be->create_buffer(size_t{16} << 20, MemoryType::Device);
            expect(big != nullptr && big->size() == (size_t{16} << 20), "large buffer bypasses the pool");
        }
        auto pinned = be->create_buffer(64, MemoryType::HostPinned);
        expect(pinned != nullptr && pinned->memory_type() == MemoryType::HostPinned, "pinned buffer");
        expect_ok(be->synchronize(), "synchronize");
    }
}

}  // namespace

int main(int argc, char** argv) {
    const bool cpu_only = argc > 1 && std::strcmp(argv[1], "--cpu") == 0;
    InitializeHipBackend();
    expect(BackendRegistry::instance().has_backend("hip"), "\"hip\" registered");
    auto be = BackendRegistry::instance().create_backend(Device(0, DeviceType::DiscreteGPU, "hip"));
    expect(be != nullptr, "create_backend(hip)");
    if (!be) return 1;
    check_cpu(be.get());
    if (!cpu_only) {
        if (!be->is_available()) {
            std::printf("FAIL no HIP device visible\n");
            return 1;
        }
        check_gpu(be.get());
    }
    std::printf("%s: %d checks passed, %d failed\n", cpu_only ? "backend (cpu)" : "backend (gpu)", g_pass, g_fail);
    return g_fail == 0 ? 0 : 1;
}
