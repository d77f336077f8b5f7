"""Pins the CPU oracle against the reference's own known-answer tests
(tests/hip_kernels_test.cc in Dustray/Vicold.HybridAI), restated here with the
same inputs and tolerances.  The reference runs them on its FP32 kernel
instantiations, so the oracle is called with round_out=False unless the KAT
is a bf16 one."""
import math

import numpy as np
import pytest

from _hai import orc


def bf(x):
    return orc.round_bf16(np.asarray(x, np.float32))


def test_cast_round_trip():  # hip_kernels_test.cc:67-85
    x = np.array([-3.25, -0.5, 0.0, 1.125, 9.75], np.float32)
    assert np.array_equal(orc.round_bf16(x), x)
    # RNE tie cases: 1 + 2^-8 rounds to 1 (even), 1 + 3*2^-8 rounds up.
    ties = np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8, -(1 + 2 ** -8)], np.float32)
    assert list(orc.round_bf16(ties)) == [1.0, 1 + 2 ** -6, -1.0]
    assert np.isnan(orc.round_bf16(np.array([np.nan], np.float32))[0])


def test_bf16_transpose_weight_gemm():  # :87-131
    a = bf([1.25, -2.0, 0.5, 3.0, -1.0, 0.75, 2.5, -0.5]).reshape(2, 4)
    w = bf([0.5, 1.0, -1.5, 2.0, -2.0, 0.25, 1.0, -0.75, 1.5, -0.5, 0.75, 1.25]).reshape(3, 4)
    got = orc.gemm(a, w, round_out=True)
    want = bf(a.astype(np.float64) @ w.astype(np.float64).T)
    assert np.allclose(got, want, atol=1e-3)


def test_embedding_add_argmax():  # :133-165
    emb = np.array([0, 1, 2, 3, 10, 11, 12, 13, 20, 21, 22, 23], np.float32).reshape(3, 4)
    g = orc.embedding(emb, [2, 0])
    added = orc.add(g, np.full_like(g, 0.5), round_out=False)
    assert list(added.reshape(-1)) == [20.5, 21.5, 22.5, 23.5, 0.5, 1.5, 2.5, 3.5]
    assert orc.argmax_rows(added[-1:])[0] == 3


def test_batched_argmax_rows_tie_break():  # :167-196 (first index wins)
    v = np.array([[1, 9, 3, 9, -1, 2, 0], [-4, -3, -2, -1, 0, 1, 8], [5, 5, 4, 3, 2, 1, 0]], np.float32)
    assert list(orc.argmax_rows(v)) == [1, 6, 0]
    assert list(orc.argmax_rows(bf(v))) == [1, 6, 0]
    nan_row = np.array([[np.nan, np.nan], [-np.inf, -np.inf], [np.nan, 2.0]], np.float32)
    assert list(orc.argmax_rows(nan_row)) == [0, 0, 1]


def test_rmsnorm_silu_mul():  # :242-291
    x = np.array([[1, 2, 3, 4], [-1, -2, -3, -4]], np.float32)
    w = np.array([0.0, 0.5, -0.25, 1.0], np.float32)
    got = orc.rmsnorm(x, w, 1e-6, unit_offset=True, round_out=False)
    for r in range(2):
        inv = 1.0 / math.sqrt(float((x[r] ** 2).sum()) / 4 + 1e-6)
        assert np.allclose(got[r], x[r] * inv * (1 + w), atol=1e-5)
    gate = np.array([-2.0, -0.5, 0.0, 1.5], np.float32)
    up = np.array([1.0, 2.0, 3.0, -4.0], np.float32)
    silu = gate / (1 + np.exp(-gate.astype(np.float64)))
    assert np.allclose(orc.silu_mul(gate, up, round_out=False), silu * up, atol=1e-6)


def test_partial_rope():  # :293-347 (rotate-half, R=2, offset 3)
    q = np.arange(1, 17, dtype=np.float32).reshape(2, 2, 4)
    got = orc.partial_rope(q, 2, 2, 4, 2, 3, 1e4)
    for s in range(2):
        th = s + 3.0
        c, sn = math.cos(th), math.sin(th)
        for h in range(2):
            x0, x1 = q[s, h, 0], q[s, h, 1]
            assert abs(got[s, h, 0] - (x0 * c - x1 * sn)) < 1e-5
            assert abs(got[s, h, 1] - (x1 * c + x0 * sn)) < 1e-5
            assert got[s, h, 2] == q[s, h, 2] and got[s, h, 3] == q[s, h, 3]


def _qgate_expected(src, w, T, nq, D, pos0, base, eps):
    out = np.zeros((T, nq, D))
    for t in range(T):
        for h in range(nq):
            s = src[t, h * 2 * D:h * 2 * D + D].astype(np.float64)
            inv = 1.0 / math.sqrt((s * s).sum() / D + eps)
            n = s * inv * (w.astype(np.float64) + 1)
            th = pos0 + t
            c0, s0 = math.cos(th), math.sin(th)
            c1, s1 = math.cos(th / math.sqrt(base)), math.sin(th / math.sqrt(base))
            out[t, h] = [n[0] * c0 - n[2] * s0, n[1] * c1 - n[3] * s1, n[2] * c0 + n[0] * s0, n[3] * c1 + n[1] * s1]
    return out


def test_fused_q_gate_rmsnorm_rope_fp32():  # :423-479
    src = np.array([1, 2, 3, 4, -4, 0.5, 2, -1, -2, 1, 0.5, 3, 1.5, -2, 0.25, 4,
                    4, -1, 2, 0.25, 0.25, 3, -2, 1.5, 0.5, 3, -2, 1.5, -1, 2, 0.75, -3], np.float32).reshape(2, 16)
    w = np.array([0.0, 0.25, -0.5, 1.0], np.float32)
    q, g = orc.q_gate_rmsnorm_rope(src, w, 2, 2, 4, 4, 5, 1e4, 1e-6, True, round_out=False)
    assert np.allclose(q, _qgate_expected(src, w, 2, 2, 4, 5, 1e4, 1e-6), atol=1e-5)
    for t in range(2):
        for h in range(2):
            assert np.array_equal(g[t, h], src[t, h * 8 + 4:h * 8 + 8])


def test_fused_q_gate_rmsnorm_rope_bf16():  # :481-550
    src = bf([1, -2, 0.5, 3, 4, -1, 2, 0.25, -0.5, 3, -2, 1.5, -3, 0.75, 1, 2]).reshape(1, 16)
    w = bf([0.0, 0.25, -0.5, 1.0])
    q, g = orc.q_gate_rmsnorm_rope(src, w, 1, 2, 4, 4, 2, 1e4, 1e-6, True, round_out=True)
    want = bf(_qgate_expected(src, w, 1, 2, 4, 2, 1e4, 1e-6).astype(np.float32))
    assert np.allclose(q, want, atol=1e-3)


def _softmax_attn(q, k, v, scale):
    s = (q.astype(np.float64) @ k.astype(np.float64).T) * scale
    p = np.exp(s - s.max())
    return (p / p.sum()) @ v.astype(np.float64)


def test_causal_gqa_with_gate():  # :552-603 (gate 0 -> x0.5)
    q = np.array([1, 0, 0, 1, 1, 1, -1, 1], np.float32).reshape(2, 2, 2)
    k = np.array([1, 0, 0, 1], np.float32).reshape(2, 1, 2)
    v = np.array([2, 4, 6, 8], np.float32).reshape(2, 1, 2)
    got = orc.attention(q, np.zeros_like(q), k, v, 2, 2, 2, 1, 2, round_out=False)
    for t in range(2):
        for h in range(2):
            want = _softmax_attn(q[t, h], k[:t + 1, 0], v[:t + 1, 0], 1 / math.sqrt(2)) * 0.5
            assert np.allclose(got[t, h], want, atol=1e-5)


def test_causal_gqa_head256():  # :605-675 (analytic inputs)
    T, nq, nkv, D = 3, 4, 2, 256
    idx_q = np.arange(T * nq * D)
    idx_kv = np.arange(T * nkv * D)
    q = (((idx_q * 17) % 29 - 14) / 19.0).astype(np.float32).reshape(T, nq, D)
    gate = (((idx_q * 7) % 13 - 6) / 5.0).astype(np.float32).reshape(T, nq, D)
    k = (((idx_kv * 11) % 31 - 15) / 23.0).astype(np.float32).reshape(T, nkv, D)
    v = (((idx_kv * 5) % 37 - 18) / 17.0).astype(np.float32).reshape(T, nkv, D)
    got = orc.attention(q, gate, k, v, T, T, nq, nkv, D, round_out=False)
    for t in range(T):
        for h in range(nq):
            kv = h // 2
            want = _softmax_attn(q[t, h], k[:t + 1, kv], v[:t + 1, kv], 1 / 16.0)
            want = want / (1 + np.exp(-gate[t, h].astype(np.float64)))
            assert np.allclose(got[t, h], want, atol=2e-5)


def test_kv_cache_append_and_decode():  # :677-735
    keys = np.array([1, 0, 0, 1, 1, 1], np.float32).reshape(3, 1, 2)
    vals = np.array([2, 4, 6, 8, 10, 12], np.float32).reshape(3, 1, 2)
    q = np.array([1, 1, -1, 1], np.float32).reshape(1, 2, 2)
    got = orc.attention(q, None, keys, vals, 1, 3, 2, 1, 2, round_out=False)
    for h in range(2):
        assert np.allclose(got[0, h], _softmax_attn(q[0, h], keys[:, 0], vals[:, 0], 1 / math.sqrt(2)), atol=1e-5)


def test_cached_gqa_with_current_token():  # :818-897
    kc = np.array([1, 0, 0, 1, 2, 0, 0, 2, 0, 1, 1, 0, 0, 2, 2, 0, -1, 0.5, 2, -0.25, 0.75, -2, 0.5, 1.5],
                  np.float32).reshape(3, 2, 4)
    vc = np.array([1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, -3, 1, 5, 2, 4, -2, 6, 0.5],
                  np.float32).reshape(3, 2, 4)
    q = np.array([0.5, 1, -0.25, 2, -1, 0.25, 0.75, 1.5, 2, -0.5, 1, 0.25, -0.75, 1.25, -1, 0.5],
                 np.float32).reshape(1, 4, 4)
    got = orc.attention(q, np.zeros_like(q), kc, vc, 1, 3, 4, 2, 4, round_out=False)
    for h in range(4):
        want = _softmax_attn(q[0, h], kc[:, h // 2], vc[:, h // 2], 0.5) * 0.5
        assert np.allclose(got[0, h], want, atol=1e-5)


def test_bf16_cached_gqa():  # :899-957
    q = bf([1.25, -0.5, -0.75, 1.5]).reshape(1, 2, 2)
    k = bf([1, 0.5, -0.5, 1, 0.75, 1.25]).reshape(3, 1, 2)
    v = bf([2, -1, 0.5, 3, -2, 1.5]).reshape(3, 1, 2)
    got = orc.attention(q, None, k, v, 1, 3, 2, 1, 2, round_out=True)
    for h in range(2):
        want = bf(_softmax_attn(q[0, h], k[:, 0], v[:, 0], 1 / math.sqrt(2)).astype(np.float32))
        assert np.allclose(got[0, h], want, atol=1e-3)


def _silu(x):
    return x / (1 + math.exp(-x))


def test_deltanet_conv_flat_layout():  # :996-1020 and :1022-1058
    qkv = np.arange(1, 9, dtype=np.float32).reshape(1, 8)
    w = np.tile(np.array([0, 1], np.float32), 8).reshape(8, 2)
    q, k, v, _ = orc.deltanet_conv(qkv, w, np.zeros((8, 1), np.float32), 1, 2, 4, 1, 1, 2, round_out=False)
    assert np.allclose(np.concatenate([q[0], k[0], v[0]]), [_silu(x) for x in range(1, 9)], atol=1e-6)
    w2 = np.stack([np.zeros(8), np.arange(1, 9)], axis=1).astype(np.float32)
    q, k, v, _ = orc.deltanet_conv(qkv, w2, np.zeros((8, 1), np.float32), 1, 2, 4, 1, 1, 2, round_out=False)
    assert np.allclose(np.concatenate([q[0], k[0], v[0]]), [_silu(x * x) for x in range(1, 9)], atol=1e-6)


def test_deltanet_conv_chunked_equals_full():  # :1060-1147
    qkv = np.array([[1, 2, 3, 4, 5, 6, 7, 8], [2, 3, 4, 5, 6, 7, 8, 9], [3, 4, 5, 6, 7, 8, 9, 10]], np.float32)
    w = np.array([0.1, 0.2, 1.0, 0.2, 0.3, 0.9, 0.3, 0.4, 0.8, 0.4, 0.5, 0.7, 0.5, 0.6, 0.6, 0.6, 0.7, 0.5,
                  0.7, 0.8, 0.4, 0.8, 0.9, 0.3], np.float32).reshape(8, 3)
    st0 = np.zeros((8, 2), np.float32)
    qf, kf, vf, stf = orc.deltanet_conv(qkv, w, st0, 3, 2, 4, 1, 1, 3, round_out=False)
    q1, k1, v1, st1 = orc.deltanet_conv(qkv[:2], w, st0, 2, 2, 4, 1, 1, 3, round_out=False)
    q2, k2, v2, st2 = orc.deltanet_conv(qkv[2:], w, st1, 1, 2, 4, 1, 1, 3, round_out=False)
    assert np.array_equal(np.concatenate([q1, q2]), qf) and np.array_equal(np.concatenate([v1, v2]), vf)
    assert np.array_equal(st2, stf)


def _delta_args():
    return dict(q=np.array([1, 0, 0, 1], np.float32).reshape(2, 2), k=np.array([1, 1, 1, -1], np.float32).reshape(2, 2),
                v=np.array([2, 4, 6, 8], np.float32).reshape(2, 2), a=np.array([[0.1], [-0.2]], np.float32),
                b=np.array([[0.3], [-0.4]], np.float32), z=np.array([0.5, 1.0, -0.5, 2.0], np.float32).reshape(2, 2))


def test_deltanet_recurrent_chunked_equals_full():  # :1149-1205
    d = _delta_args()
    al, dt, nw = np.array([-1.0], np.float32), np.array([0.2], np.float32), np.array([1.0, 0.75], np.float32)
    st = np.zeros((1, 2, 2), np.float32)
    full, stf = orc.deltanet_recurrent(d["q"], d["k"], d["v"], d["a"], d["b"], d["z"], al, dt, nw, st, 2, 1, 1, 2, 2,
                                       round_out=False)
    parts = []
    s = st
    for t in range(2):
        o, s = orc.deltanet_recurrent(d["q"][t:t + 1], d["k"][t:t + 1], d["v"][t:t + 1], d["a"][t:t + 1],
                                      d["b"][t:t + 1], d["z"][t:t + 1], al, dt, nw, s, 1, 1, 1, 2, 2, round_out=False)
        parts.append(o)
    assert np.array_equal(np.concatenate(parts), full) and np.array_equal(s, stf)


def test_deltanet_recurrent_closed_form_2x2():  # :1207-1272
    q, k, v = np.array([[1.0, 2.0]], np.float32), np.array([[2.0, -1.0]], np.float32), np.array([[3.0, -2.0]], np.float32)
    a, b = np.array([[0.25]], np.float32), np.array([[-0.4]], np.float32)
    al, dt = np.array([-0.7], np.float32), np.array([0.15], np.float32)
    nw, z = np.array([1.25, 0.75], np.float32), np.array([[0.5, -1.0]], np.float32)
    s0 = np.array([0.5, -0.25, 1.0, 0.75], np.float32).reshape(1, 2, 2)
    out, st = orc.deltanet_recurrent(q, k, v, a, b, z, al, dt, nw, s0, 1, 1, 1, 2, 2, round_out=False)
    qn = 1 / math.sqrt(5 + 1e-6) / math.sqrt(2)
    kn = 1 / math.sqrt(5 + 1e-6)
    decay = math.exp(-math.exp(-0.7) * math.log1p(math.exp(0.25 + 0.15)))
    beta = 1 / (1 + math.exp(0.4))
    S = s0[0].astype(np.float64) * decay
    o = np.zeros(2)
    for j in range(2):
        r = sum(k[0, i] * kn * S[i, j] for i in range(2))
        c = v[0, j] - r
        for i in range(2):
            S[i, j] += beta * k[0, i] * kn * c
        o[j] = sum(q[0, i] * qn * S[i, j] for i in range(2))
    inv = 1 / math.sqrt((o * o).mean() + 1e-6)
    want = [o[j] * inv * nw[j] * _silu(z[0, j]) for j in range(2)]
    assert np.allclose(out[0], want, atol=1e-5)
    assert np.allclose(st[0], S, atol=1e-5)


def test_deltanet_qwen_shape_vs_fp64():  # shapes of :1274-1454, sin-generated inputs
    nk, nv, dk, dv = 16, 48, 128, 128

    def mk(n, sc, bias):
        return (np.sin(np.arange(n, dtype=np.float32) * np.float32(sc)) + np.float32(bias)).astype(np.float32)

    q = mk(nk * dk, 0.013, 0.1).reshape(1, -1)
    k = mk(nk * dk, 0.017, -0.2).reshape(1, -1)
    v = mk(nv * dv, 0.011, 0.3).reshape(1, -1)
    z = mk(nv * dv, 0.019, -0.1).reshape(1, -1)
    nw = mk(dv, 0.023, 1.0)
    s0 = mk(nv * dk * dv, 0.007, 0.02).reshape(nv, dk, dv)
    a = np.full((1, nv), 0.15, np.float32)
    b = np.full((1, nv), -0.35, np.float32)
    al = np.full(nv, -0.7, np.float32)
    dt = np.full(nv, 0.2, np.float32)
    out, st = orc.deltanet_recurrent(q, k, v, a, b, z, al, dt, nw, s0, 1, nk, nv, dk, dv, round_out=False)
    # fp64 restatement of the same delta rule
    decay = math.exp(-math.exp(-0.7) * math.log1p(math.exp(0.35)))
    beta = 1 / (1 + math.exp(0.35))
    for h in (0, 17, 47):
        g = h // 3
        qq = q[0, g * dk:(g + 1) * dk].astype(np.float64)
        kk = k[0, g * dk:(g + 1) * dk].astype(np.float64)
        qn = qq / math.sqrt((qq * qq).sum() + 1e-6) / math.sqrt(dk)
        kn = kk / math.sqrt((kk * kk).sum() + 1e-6)
        S = s0[h].astype(np.float64) * decay
        r = kn @ S
        S = S + beta * np.outer(kn, v[0, h * dv:(h + 1) * dv] - r)
        o = qn @ S
        inv = 1 / math.sqrt((o * o).mean() + 1e-6)
        zz = z[0, h * dv:(h + 1) * dv].astype(np.float64)
        want = o * inv * nw * (zz / (1 + np.exp(-zz)))
        assert np.allclose(out[0, h * dv:(h + 1) * dv], want, atol=1e-5, rtol=1e-5)
        assert np.allclose(st[h], S, atol=1e-5)
