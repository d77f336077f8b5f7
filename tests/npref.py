"""Float64 restatement of the reference's hybrid-model forward, for pinning
the CPU oracle's composition (TEST INFRASTRUCTURE ONLY).

Written from the reference's formulas, independently of the oracle's C++:
plain numpy float64 with no fixed reduction order, bf16 rounding (RNE) only
where the reference stores a bf16 tensor.  The oracle's results must agree
with it to bf16 rounding; a structural mistake (a swapped concat, a wrong
hidden row, a shifted RoPE position, a missing +1 in a norm) moves them by
O(1).  Every function cites the reference it restates.

Weights come from the oracle model (``orc.Model.tensor``) under its tensor
ids: slot * 64 + kind, slot 0 shared, 1 MTP shared, 2 + i target layer i,
1024 + j MTP layer j.
"""
from __future__ import annotations

import numpy as np

# kinds of a decoder-layer slot
IN_LN, POST_LN, IN_QKV, IN_Z, IN_A, IN_B, CONV, A_LOG, DT_BIAS, LIN_NORM, OUT_PROJ = range(11)
Q_PROJ, K_PROJ, V_PROJ, O_PROJ, Q_NORM, K_NORM, GATE, UP, DOWN = range(11, 20)
# kinds of slot 0 and slot 1
EMBED, FINAL_NORM, LM_HEAD = 0, 1, 2
FC, MTP_NORM, PRE_EMB, PRE_HID = 0, 1, 2, 3


def tid(slot, kind):
    return slot * 64 + kind


def bf(x):
    """float64 -> nearest bf16 value (RNE through float32), as float64."""
    u = np.ascontiguousarray(np.asarray(x, np.float64).astype(np.float32)).view(np.uint32).astype(np.uint64)
    r = (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32)
    return r.view(np.float32).astype(np.float64)


def rmsnorm(x, w, eps, off=1.0):
    """qwen_rmsnorm_reference -> RMSNorm::forward (rmsnorm.cc:35-96):
    x / sqrt(mean(x^2) + eps) * (w + 1), stored bf16."""
    x = np.asarray(x, np.float64)
    inv = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return bf(x * inv * (np.asarray(w, np.float64) + off))


def linear(x, W):
    """Linear::forward (linear.cc:117-179): bf16(x . W^T), W [N, K]."""
    return bf(np.asarray(x, np.float64) @ np.asarray(W, np.float64).T)


def silu(x):
    return x / (1.0 + np.exp(-x))


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def rope(x, pos, R, base):
    """partial_rope_kernel (hip_kernels.hip:192-221): rotate-half on the
    first R dims of every head, theta_p = pos / base^(2p/R); x [..., D] in
    float64, pos broadcast over the leading axis."""
    x = np.array(x, np.float64)
    half = R // 2
    p = np.arange(half, dtype=np.float64)
    theta = np.asarray(pos, np.float64).reshape(-1, *([1] * (x.ndim - 1))) / base ** (2.0 * p / R)
    c, s = np.cos(theta), np.sin(theta)
    a, b = x[..., :half].copy(), x[..., half:R].copy()
    x[..., :half] = a * c - b * s
    x[..., half:R] = b * c + a * s
    return x


class Weights:
    def __init__(self, model):
        self.m = model
        self.cfg = model.cfg

    def __call__(self, slot, kind, shape=None):
        t = self.m.tensor(tid(slot, kind)).astype(np.float64)
        return t.reshape(shape) if shape is not None else t


def attention_layer(W, slot, xn, cache, pos0):
    """qwen_attention_reference -> GatedGQAAttention::forward_cached
    (attention.cc:301-599) with hip_fused_kernels.hip:87-141 for Q and
    attention.cc:459-464 for K: q_proj rows per head are [q | gate]; q is
    RMSNorm(+1)'d and rotated, then stored once; K is RMSNorm(+1)'d, stored,
    rotated, stored; V raw; rows appended at pos0..; query t attends keys
    0..pos0+t with scale 1/sqrt(D); out * sigmoid(gate) stored; o_proj.
    cache = dict(k=[...], v=[...]) lists of [nkv, D] rows, extended."""
    c = W.cfg
    H, nq, nkv, D, R = c["hidden"], c["num_q_heads"], c["num_kv_heads"], c["head_dim"], c["rope_dim"]
    eps, base = c["rms_eps"], c["rope_theta"]
    T = xn.shape[0]
    qg = linear(xn, W(slot, Q_PROJ, (nq * 2 * D, H))).reshape(T, nq, 2 * D)
    q, gate = qg[..., :D], qg[..., D:]
    k = linear(xn, W(slot, K_PROJ, (nkv * D, H))).reshape(T, nkv, D)
    v = linear(xn, W(slot, V_PROJ, (nkv * D, H))).reshape(T, nkv, D)
    pos = pos0 + np.arange(T)
    qw, kw = W(slot, Q_NORM), W(slot, K_NORM)
    qn = q / np.sqrt(np.mean(q * q, axis=-1, keepdims=True) + eps) * (qw + 1.0)
    qr = bf(rope(qn, pos, R, base))
    kr = bf(rope(rmsnorm(k, kw, eps), pos, R, base))
    cache["k"].extend(list(kr))
    cache["v"].extend(list(v))
    K = np.stack(cache["k"])  # [L, nkv, D]
    V = np.stack(cache["v"])
    group = nq // nkv
    out = np.zeros((T, nq, D))
    for t in range(T):
        L = pos0 + t + 1
        for h in range(nq):
            s = K[:L, h // group, :] @ qr[t, h] / np.sqrt(D)
            p = np.exp(s - s.max())
            o = (p @ V[:L, h // group, :]) / p.sum()
            out[t, h] = o * sigmoid(gate[t, h])
    return linear(bf(out).reshape(T, nq * D), W(slot, O_PROJ, (H, nq * D)))


def deltanet_layer(W, slot, xn, state):
    """qwen_deltanet_reference (qwen_reference.cc:205-258): in_proj qkv / z /
    a / b; grouped causal conv over flat [Q|K|V] channels with SiLU
    (hip_kernels.hip:871-912); gated delta rule per value head
    (hip_kernels.hip:985-1095): q, k L2-normalised (eps 1e-6 in the sqrt), q
    also by 1/sqrt(dk); decay = exp(-exp(A_log) softplus(dt_bias + a)),
    beta = sigmoid(b); S *= decay; S += beta k (v - k.S); o = q.S; then
    bf16(bf16(o) * rsqrt(mean(o^2) + eps) * w * silu(z)); out_proj.
    state = dict(conv [C, Kc-1], S [nv, dk, dv]), updated."""
    c = W.cfg
    H, nk, nv, dk, dv, Kc = (c["hidden"], c["lin_qk_heads"], c["lin_v_heads"], c["lin_k_dim"], c["lin_v_dim"],
                             c["conv_kernel"])
    eps = c["rms_eps"]
    kw, vw = nk * dk, nv * dv
    C = 2 * kw + vw
    T = xn.shape[0]
    qkv = linear(xn, W(slot, IN_QKV, (C, H)))
    z = linear(xn, W(slot, IN_Z, (vw, H))).reshape(T, nv, dv)
    a = linear(xn, W(slot, IN_A, (nv, H)))
    b = linear(xn, W(slot, IN_B, (nv, H)))
    cw = W(slot, CONV, (C, Kc))
    conv = state["conv"]
    act = np.zeros((T, C))
    for t in range(T):
        window = np.concatenate([conv, qkv[t][:, None]], axis=1)  # [C, Kc], oldest first
        act[t] = bf(silu(np.sum(window * cw, axis=1)))
        conv = window[:, 1:]
    state["conv"] = conv
    q = act[:, :kw].reshape(T, nk, dk)
    k = act[:, kw:2 * kw].reshape(T, nk, dk)
    v = act[:, 2 * kw:].reshape(T, nv, dv)
    a_log, dt_bias, nw = W(slot, A_LOG), W(slot, DT_BIAS), W(slot, LIN_NORM)
    S = state["S"]
    out = np.zeros((T, nv, dv))
    for t in range(T):
        for h in range(nv):
            g = h // (nv // nk)
            qn = q[t, g] / np.sqrt(np.sum(q[t, g] ** 2) + 1e-6) / np.sqrt(dk)
            kn = k[t, g] / np.sqrt(np.sum(k[t, g] ** 2) + 1e-6)
            x = dt_bias[h] + a[t, h]
            decay = np.exp(-np.exp(a_log[h]) * (max(x, 0.0) + np.log1p(np.exp(-abs(x)))))
            beta = sigmoid(b[t, h])
            S[h] *= decay
            S[h] += beta * np.outer(kn, v[t, h] - kn @ S[h])
            o = qn @ S[h]
            rms = 1.0 / np.sqrt(np.mean(o * o) + eps)
            out[t, h] = bf(bf(o) * rms * nw * silu(z[t, h]))
    return linear(out.reshape(T, vw), W(slot, OUT_PROJ, (H, vw)))


def mlp(W, slot, xn):
    """qwen_mlp_reference (qwen_reference.cc:146-175)."""
    c = W.cfg
    H, F = c["hidden"], c["ffn"]
    g = linear(xn, W(slot, GATE, (F, H)))
    u = linear(xn, W(slot, UP, (F, H)))
    return linear(bf(silu(g) * u), W(slot, DOWN, (H, F)))


def decoder_layer(W, slot, h, attn, cache=None, state=None, pos0=0):
    """One layer of target_forward (generator.cc:550-634): pre-norm mixer,
    residual, post-norm MLP, residual."""
    eps = W.cfg["rms_eps"]
    xn = rmsnorm(h, W(slot, IN_LN), eps)
    mixed = attention_layer(W, slot, xn, cache, pos0) if attn else deltanet_layer(W, slot, xn, state)
    h = bf(h + mixed)
    xn = rmsnorm(h, W(slot, POST_LN), eps)
    return bf(h + mlp(W, slot, xn))


def embed(W, ids):
    c = W.cfg
    return W(0, EMBED, (c["vocab"], c["hidden"]))[np.asarray(ids)]


def fresh_state(cfg, n_layers):
    nk, nv, dk, dv, Kc = (cfg["lin_qk_heads"], cfg["lin_v_heads"], cfg["lin_k_dim"], cfg["lin_v_dim"],
                          cfg["conv_kernel"])
    C = 2 * nk * dk + nv * dv
    return ([dict(k=[], v=[]) for _ in range(n_layers)],
            [dict(conv=np.zeros((C, Kc - 1)), S=np.zeros((nv, dk, dv))) for _ in range(n_layers)])


def target_forward(W, ids):
    """target_forward (generator.cc:550-634) from empty caches: embedding,
    the decoder layers (layer i is attention iff (i+1) % interval == 0,
    qwen3_config.cc:166-176), final RMSNorm(+1), lm_head.  Returns the
    post-final-norm hidden [T, H] and the logits [T, V]."""
    c = W.cfg
    caches, states = fresh_state(c, c["num_layers"])
    h = embed(W, ids)
    for i in range(c["num_layers"]):
        attn = (i + 1) % c["full_attention_interval"] == 0
        h = decoder_layer(W, 2 + i, h, attn, caches[i], states[i], 0)
    hidden = rmsnorm(h, W(0, FINAL_NORM), c["rms_eps"])
    return hidden, linear(hidden, W(0, LM_HEAD, (c["vocab"], c["hidden"])))


def mtp_inputs(W, emb, hid):
    """qwen_mtp_forward_reference up to fc (generator.cc:139-166) with
    concat_mtp_inputs (generator.cc:24-66): each row is
    [RMSNorm(+1)(emb; pre_fc_norm_embedding) | RMSNorm(+1)(hid;
    pre_fc_norm_hidden)], then fc."""
    c = W.cfg
    H, eps = c["hidden"], c["rms_eps"]
    en = rmsnorm(emb, W(1, PRE_EMB), eps)
    hn = rmsnorm(hid, W(1, PRE_HID), eps)
    return linear(np.concatenate([en, hn], axis=1), W(1, FC, (H, 2 * H)))


def mtp_forward(W, emb, hid, cache, pos0):
    """qwen_mtp_forward_reference (generator.cc:139-183): fc of the
    normalised concat, one attention decoder layer on the MTP cache (RoPE
    position = cache length), RMSNorm(+1)(mtp.norm)."""
    x = mtp_inputs(W, emb, hid)
    x = decoder_layer(W, 1024, x, True, cache, None, pos0)
    return rmsnorm(x, W(1, MTP_NORM), W.cfg["rms_eps"])


def mtp_kv_row(W, emb_row, hid_row, pos):
    """The K and V rows [nkv, D] the MTP attention layer appends for one
    input (emb_row, hid_row) at RoPE position pos (attention.cc:459-464,
    hip_kernels.hip:295-308)."""
    c = W.cfg
    H, nkv, D, R = c["hidden"], c["num_kv_heads"], c["head_dim"], c["rope_dim"]
    x = mtp_inputs(W, emb_row[None], hid_row[None])
    xn = rmsnorm(x, W(1024, IN_LN), c["rms_eps"])
    k = linear(xn, W(1024, K_PROJ, (nkv * D, H))).reshape(1, nkv, D)
    v = linear(xn, W(1024, V_PROJ, (nkv * D, H))).reshape(nkv, D)
    kr = bf(rope(rmsnorm(k, W(1024, K_NORM), c["rms_eps"]), [pos], R, c["rope_theta"]))
    return kr[0], v
