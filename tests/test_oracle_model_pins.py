"""Pins the oracle's model-level functions with checks the oracle did not
write: its layer composition (target_forward, generator.cc:550-634), its MTP
forward (generator.cc:139-183) and its MTP cache protocol (prompt prefill
pairing, generator.cc:670-699; draft rows, :737-849; checkpoint restore and
the recovery row after a rejection, :934-1003) are compared with the
float64 restatement in npref.py, computed from the oracle's own weights.

Layers are isolated by zeroing the projections that write into the
residual stream (o_proj, out_proj, down), so each sub-layer's composition
is checked on its own as well as in the full stack.  Every comparison also
shows that it discriminates: the same numbers computed with a plausible
mistake (swapped concat halves, the previous hidden row, a RoPE position off
by one, a norm without its +1) fail it."""
import numpy as np
import pytest

import npref as R
from _hai import orc

P = 12


def agree(got, want):
    """(fraction of elements within one bf16 ulp, max |diff| / rms(want))."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    ulp = np.maximum(np.abs(want), 1e-30) * 2.0 ** -7
    frac = float(np.mean(np.abs(got - want) <= ulp))
    rel = float(np.abs(got - want).max() / max(np.sqrt(np.mean(want ** 2)), 1e-30))
    return frac, rel


def assert_agree(got, want, what, frac_min=0.99, rel_max=0.02):
    frac, rel = agree(got, want)
    assert frac >= frac_min and rel <= rel_max, f"{what}: {frac:.4f} within 1 ulp, max err {rel:.4f} of rms"


def assert_differs(got, want, what):
    frac, rel = agree(got, want)
    assert frac < 0.9 and rel > 0.1, f"{what}: a planted mistake was not detected ({frac:.4f} within 1 ulp, " \
                                     f"max err {rel:.4f} of rms)"


@pytest.fixture()
def model():
    m = orc.Model(orc.TINY, seed=0)
    yield m
    m.close()


def zero(m, *tids):
    for t in tids:
        m.set_tensor(t, np.zeros(m.tensor(t).size, np.float32))


def residual_writers(cfg):
    out = []
    for i in range(cfg["num_layers"]):
        attn = (i + 1) % cfg["full_attention_interval"] == 0
        out.append(R.tid(2 + i, R.O_PROJ if attn else R.OUT_PROJ))
        out.append(R.tid(2 + i, R.DOWN))
    return out


def prompt():
    return orc.synthetic_prompt(3, P, orc.TINY["vocab"]).astype(np.int32)


# ---------------------------------------------------------------- composition
def test_composition_closed_form_without_residual_writers(model):
    """Every o_proj / out_proj / down zeroed: each residual add is h + 0, so
    the final hidden is RMSNorm(+1)(final_norm) of the embedding rows and
    the logits are lm_head of it."""
    cfg = model.cfg
    zero(model, *residual_writers(cfg))
    ids = prompt()
    hid, lg = model.forward(ids)
    W = R.Weights(model)
    want_h = R.rmsnorm(R.embed(W, ids), W(0, R.FINAL_NORM), cfg["rms_eps"])
    assert_agree(hid, want_h, "final hidden")
    assert_agree(lg, R.linear(want_h, W(0, R.LM_HEAD, (cfg["vocab"], cfg["hidden"]))), "logits")
    # the final norm's +1 and its position are what the check sees
    assert_differs(hid, R.rmsnorm(R.embed(W, ids), W(0, R.FINAL_NORM), cfg["rms_eps"], off=0.0), "final norm +1")


@pytest.mark.parametrize("live", ["mlp1", "deltanet0", "deltanet2", "attention3"])
def test_composition_one_live_sublayer(model, live):
    """One sub-layer writes into the residual stream, the others add zero:
    the closed form is h + sublayer(RMSNorm(+1)(h)) followed by the final
    norm (MLP: down(silu(gate) * up), DeltaNet: conv + gated delta rule +
    gated norm + out_proj, attention: gated GQA + o_proj).  The DeltaNet
    gated-norm weight (no +1 in that norm) is set near 1 so that the
    layer's output is of the order of the residual stream."""
    cfg = model.cfg
    writers = residual_writers(cfg)
    keep = {"mlp1": R.tid(3, R.DOWN), "deltanet0": R.tid(2, R.OUT_PROJ), "deltanet2": R.tid(4, R.OUT_PROJ),
            "attention3": R.tid(5, R.O_PROJ)}[live]
    zero(model, *[t for t in writers if t != keep])
    if live.startswith("deltanet"):
        rng = np.random.default_rng(5)
        nw = orc.round_bf16((1.0 + 0.1 * rng.standard_normal(cfg["lin_v_dim"])).astype(np.float32))
        model.set_tensor(keep - R.OUT_PROJ + R.LIN_NORM, nw)
    ids = prompt()
    hid, lg = model.forward(ids)
    W = R.Weights(model)
    want_h, want_lg = R.target_forward(W, ids)
    assert_agree(hid, want_h, f"{live}: final hidden")
    assert_agree(lg, want_lg, f"{live}: logits")
    # the live sub-layer changes the result: the check is not vacuous
    assert_differs(hid, R.rmsnorm(R.embed(W, ids), W(0, R.FINAL_NORM), cfg["rms_eps"]), f"{live} contributes")


def test_composition_full_stack(model):
    """All weights live: the oracle's prefill forward (4 layers D,D,D,G,
    final norm, lm_head) agrees with the float64 restatement to bf16
    rounding, and so do its greedy argmaxes."""
    ids = prompt()
    hid, lg = model.forward(ids)
    W = R.Weights(model)
    want_h, want_lg = R.target_forward(W, ids)
    assert_agree(hid, want_h, "final hidden")
    assert_agree(lg, want_lg, "logits")
    top2 = np.sort(want_lg, axis=1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 1e-2  # rows whose argmax is not a near-tie
    assert np.array_equal(np.argmax(lg, axis=1)[clear], np.argmax(want_lg, axis=1)[clear])


# ---------------------------------------------------------------- MTP forward
def target_hidden(model, ids):
    return model.forward(ids)[0]


def test_mtp_forward_closed_form(model):
    """MTP o_proj and down zeroed: the MTP output is
    RMSNorm(+1)(mtp.norm)(fc([RMSNorm(+1)(emb; pre_fc_norm_embedding) |
    RMSNorm(+1)(h; pre_fc_norm_hidden)])) -- embedding half first."""
    cfg = model.cfg
    zero(model, R.tid(1024, R.O_PROJ), R.tid(1024, R.DOWN))
    ids = prompt()
    h = target_hidden(model, ids)
    out, _, _ = model.mtp_forward(ids, h)
    W = R.Weights(model)
    emb = R.embed(W, ids)
    want = R.rmsnorm(R.mtp_inputs(W, emb, h), W(1, R.MTP_NORM), cfg["rms_eps"])
    assert_agree(out, want, "MTP output")
    # planted mistakes: swapped concat halves; norms swapped between halves
    H = cfg["hidden"]
    en = R.rmsnorm(emb, W(1, R.PRE_EMB), cfg["rms_eps"])
    hn = R.rmsnorm(h, W(1, R.PRE_HID), cfg["rms_eps"])
    swapped = R.linear(np.concatenate([hn, en], axis=1), W(1, R.FC, (H, 2 * H)))
    assert_differs(out, R.rmsnorm(swapped, W(1, R.MTP_NORM), cfg["rms_eps"]), "swapped concat")
    en2 = R.rmsnorm(emb, W(1, R.PRE_HID), cfg["rms_eps"])
    hn2 = R.rmsnorm(h, W(1, R.PRE_EMB), cfg["rms_eps"])
    crossed = R.linear(np.concatenate([en2, hn2], axis=1), W(1, R.FC, (H, 2 * H)))
    assert_differs(out, R.rmsnorm(crossed, W(1, R.MTP_NORM), cfg["rms_eps"]), "pre-fc norms crossed")


def test_mtp_forward_full_layer(model):
    """All MTP weights live over the prompt rows (the MTP prompt prefill):
    output and the appended K / V rows agree with the float64 MTP forward
    (attention over the MTP cache, causal, RoPE position = cache length)."""
    ids = prompt()
    h = target_hidden(model, ids)
    out, k, v = model.mtp_forward(ids, h)
    W = R.Weights(model)
    cache = dict(k=[], v=[])
    want = R.mtp_forward(W, R.embed(W, ids), h, cache, 0)
    assert_agree(out, want, "MTP output")
    assert_agree(k, np.stack(cache["k"]), "MTP K rows")
    assert_agree(v, np.stack(cache["v"]), "MTP V rows")


# ---------------------------------------------------------------- cache protocol
def test_mtp_prefill_pairs_each_token_with_its_own_hidden(model):
    """After the prompt prefill (max_new = 1: no round runs) the MTP cache
    holds P rows and row i pairs emb(t_i) with the target's post-norm hidden
    h_i at RoPE position i (unshifted, generator.cc:670-699)."""
    ids = prompt()
    toks, st, _ = model.speculative(ids, 1, width=1)
    assert st["rounds"] == 0 and len(toks) == 1
    k, v = model.last_mtp_cache()
    assert k.shape[0] == P
    h = target_hidden(model, ids)
    W = R.Weights(model)
    emb = R.embed(W, ids)
    want = [R.mtp_kv_row(W, emb[i], h[i], i) for i in range(P)]
    assert_agree(k, np.stack([w[0] for w in want]), "K rows")
    assert_agree(v, np.stack([w[1] for w in want]), "V rows")
    shifted = [R.mtp_kv_row(W, emb[i], h[i - 1], i)[0] for i in range(1, P)]
    assert_differs(k[1:], np.stack(shifted), "hidden of the previous token")
    moved = [R.mtp_kv_row(W, emb[i], h[i], i + 1)[0] for i in range(P)]
    rd = model.cfg["rope_dim"]  # the rotated dims of each head
    assert_differs(k[..., :rd], np.stack(moved)[..., :rd], "RoPE position + 1")


def greedy_tokens(model, ids, n):
    return [int(t) for t in model.greedy(ids, n)]


def test_mtp_cache_after_a_rejection(model):
    """Width 2, first candidate forced correct, second forced wrong (a = 1):
    the MTP cache is restored to checkpoint[1] (prompt rows + the first draft
    row) and one recovery row is appended (generator.cc:970-1003) that pairs
    emb(correction) with the replay's hidden of the row before it (the
    accepted candidate's position), at RoPE position = cache length."""
    ids = prompt()
    V = model.cfg["vocab"]
    g = greedy_tokens(model, ids, 4)  # s_P, s_P+1, s_P+2, ...
    ov = np.array([g[0], g[1], (g[2] + 1) % V, 0], np.int32)  # ov[e]: candidate emitted at e
    toks, st, log = model.speculative(ids, 4, width=2, draft_override=ov)
    assert [int(t) for t in toks] == g[:4]
    assert st["rounds"] == 1 and st["accepted"] == 1 and st["corrections"] == 1
    assert st["mtp_recovery_tokens"] == 1
    k, v = model.last_mtp_cache()
    assert k.shape[0] == P + 2 == int(log[0][6])  # P prompt rows + draft row 0 + recovery row
    seq = np.concatenate([ids, np.array(g[:2], np.int32)])  # ..., s_P, s_P+1 (accepted)
    hs = target_hidden(model, seq)
    W = R.Weights(model)
    emb_next, emb_corr = R.embed(W, [g[0]])[0], R.embed(W, [g[2]])[0]
    draft0 = R.mtp_kv_row(W, emb_next, hs[P - 1], P)            # (emb(s_P), h_P-1) at P
    recovery = R.mtp_kv_row(W, emb_corr, hs[P + 1], P + 1)      # (emb(corr), h_P+1) at P+1
    assert_agree(k[P], draft0[0], "draft row K")
    assert_agree(v[P], draft0[1], "draft row V")
    assert_agree(k[P + 1], recovery[0], "recovery row K")
    assert_agree(v[P + 1], recovery[1], "recovery row V")
    assert_differs(k[P + 1], R.mtp_kv_row(W, emb_corr, hs[P], P + 1)[0], "recovery paired with h_P")
    rd = model.cfg["rope_dim"]
    assert_differs(k[P + 1][:, :rd], R.mtp_kv_row(W, emb_corr, hs[P + 1], P + 2)[0][:, :rd], "recovery at P+2")


def test_mtp_cache_after_full_acceptance(model):
    """Width 2, both candidates forced correct: the scratch cache becomes
    the MTP history (generator.cc:917-934): after the prompt rows, row P
    pairs emb(s_P) with h_P-1 and row P+1 pairs the first candidate's
    embedding with the MTP output of row P (the chained draft,
    generator.cc:826-832), at positions P and P+1."""
    ids = prompt()
    g = greedy_tokens(model, ids, 4)
    ov = np.array([g[0], g[1], g[2], 0], np.int32)
    toks, st, log = model.speculative(ids, 4, width=2, draft_override=ov)
    assert [int(t) for t in toks] == g[:4]
    assert st["rounds"] == 1 and st["accepted"] == 2 and st["corrections"] == 0
    k, v = model.last_mtp_cache()
    assert k.shape[0] == P + 2 == int(log[0][6])
    h = target_hidden(model, ids)
    W = R.Weights(model)
    cache = dict(k=[], v=[])
    R.mtp_forward(W, R.embed(W, ids), h, cache, 0)
    out0 = R.mtp_forward(W, R.embed(W, [g[0]]), h[P - 1:P], cache, P)
    assert_agree(k[:P + 1], np.stack(cache["k"]), "prompt rows + draft row 0, K")
    want1 = R.mtp_kv_row(W, R.embed(W, [g[1]])[0], out0[0], P + 1)
    assert_agree(k[P + 1], want1[0], "chained draft row K")
    assert_agree(v[P + 1], want1[1], "chained draft row V")
    hs = target_hidden(model, np.concatenate([ids, np.array(g[:1], np.int32)]))
    assert_differs(k[P + 1], R.mtp_kv_row(W, R.embed(W, [g[1]])[0], hs[P], P + 1)[0],
                   "chained row paired with the target hidden")


# ---------------------------------------------------------------- state machine
@pytest.mark.parametrize("width", [1, 2, 3, 4])
def test_state_machine_bookkeeping(model, width):
    """Random per-candidate acceptance (forced through draft overrides): the
    emitted tokens are the greedy continuation, every round's accepted count
    is the longest prefix of candidates equal to it, and the counters and
    lengths follow the reference's bookkeeping (generator.cc:720-1071):
    MTP clones = 2 per round + 1 per draft, one target clone per round,
    replay = next + accepted + correction per rejected round, the MTP cache
    grows by the drafts on full acceptance and by accepted + 1 (checkpoint +
    recovery row) otherwise, the target cache by k + 1 or accepted + 2."""
    ids = prompt()
    V = model.cfg["vocab"]
    NEW = 24
    g = greedy_tokens(model, ids, NEW + 1)
    rng = np.random.default_rng(width)
    ov = np.array([t if rng.random() < 0.7 else (t + 1 + int(rng.integers(V - 1))) % V for t in g], np.int32)
    toks, st, log = model.speculative(ids, NEW, width=width, draft_override=ov)
    assert [int(t) for t in toks] == g[:NEW]
    assert st["rounds"] == len(log)
    mtp_len, tgt_len, emitted, recov = P, P, 0, 0
    for r in log:
        k, a, full = int(r[0]), int(r[1]), int(r[2])
        assert int(r[5]) == emitted and int(r[4]) == g[emitted]
        cands = [int(c) for c in r[8:8 + k]]
        assert cands == [int(ov[emitted + 1 + i]) for i in range(k)]
        want_a = 0
        while want_a < k and cands[want_a] == g[emitted + 1 + want_a]:
            want_a += 1
        assert a == want_a and full == int(a == k)
        if full:
            mtp_len += k
            tgt_len += k + 1
            emitted += k + 1
            assert int(r[3]) == -1
        else:
            assert int(r[3]) == g[emitted + 1 + a]
            tgt_len += a + 2
            emitted += a + 2
            if emitted < NEW:
                mtp_len += a + 1
                recov += 1
        assert int(r[6]) == mtp_len and int(r[7]) == tgt_len
    rej = [r for r in log if int(r[2]) == 0]
    assert st["proposed"] == sum(int(r[0]) for r in log)
    assert st["accepted"] == sum(int(r[1]) for r in log)
    assert st["rejected"] == sum(int(r[0]) - int(r[1]) for r in rej)
    assert st["corrections"] == len(rej)
    assert st["replay_tokens"] == sum(int(r[1]) + 2 for r in rej)
    assert st["mtp_recovery_tokens"] == recov
    assert st["mtp_cache_clones"] == 2 * st["rounds"] + st["proposed"]
    assert st["target_cache_clones"] == st["rounds"]
    assert st["max_proposal_width"] == max(int(r[0]) for r in log)
