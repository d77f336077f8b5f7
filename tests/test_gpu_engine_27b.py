"""Parity at the 27B shape of the benchmark configurations (C3 bf16, the C5
weight format), where the CPU oracle is too slow to run the model, through
size-independent properties of the path:

* speculative decoding is lossless: the tokens of the speculative rounds
  (widths 1, 3, 8 and 16 -- 17 verify rows, two DeltaNet launches per
  layer -- every draft accepted, some drafts rejected, none accepted)
  equal greedy decoding of the same model, token by token;
* greedy decoding's tokens equal the argmax of the last row of a fresh
  forward over the whole sequence (prefill path, 16-row chunks): a verify row,
  a correction row and a prefill row of the same position agree;
* the round records add up (proposed = accepted + rejected, one correction
  per rejected round).

Random N(0, 0.02) weights give almost no natural acceptance, so acceptance
patterns are forced with draft overrides (the reference path takes the same
decisions for any draft source)."""
import numpy as np
import pytest

from _hai import hai

pytestmark = pytest.mark.gpu

P, NEW = 40, 24


def _refeed_greedy(eng, prompt, tokens):
    """argmax of the last row of a fresh forward over prompt + tokens[:i]."""
    seq = list(prompt)
    got = []
    for i in range(len(tokens)):
        _, lg = eng.forward(np.array(seq, np.int32))
        got.append(int(np.argmax(hai.bf16_to_f32(lg[-1]))))
        seq.append(int(tokens[i]))
    return got


def _check_lossless(eng, prompt, vocab):
    g = eng.greedy(prompt, NEW)
    assert len(g) == NEW
    assert list(g) == _refeed_greedy(eng, prompt, g)
    rng = np.random.default_rng(5)
    perturbed = g.copy()
    for i in (2, 3, 7):
        perturbed[i] = (perturbed[i] + 1) % vocab
    cases = [(1, None), (3, None), (3, g), (1, perturbed), (3, perturbed),
             (2, rng.integers(0, vocab, NEW).astype(np.int32)), (8, None), (16, g), (16, perturbed)]
    for width, ov in cases:
        toks, st, log = eng.speculative(prompt, NEW, width, draft_override=ov)
        assert list(toks) == list(g), (width, None if ov is None else list(ov))
        assert st["proposed"] == st["accepted"] + st["rejected"]
        assert st["corrections"] <= st["rounds"]
        if ov is not None and ov is g:
            assert st["accepted"] > 0 and st["corrections"] == 0


def test_27b_bf16_speculative_is_lossless():
    from hybridai_amd import engine as E
    eng = E.Engine(E.QWEN27B, max_context=P + 5 * NEW + 32, max_verify_tokens=17)
    try:
        eng.init_synthetic(seed=0, std=0.02)
        _check_lossless(eng, E.synthetic_prompt(1, P, E.QWEN27B["vocab"]), E.QWEN27B["vocab"])
    finally:
        eng.close()


def test_27b_fp8_speculative_is_lossless():
    from hybridai_amd import engine as E
    eng = E.Engine(E.QWEN27B, max_context=P + 5 * NEW + 32, max_verify_tokens=17, fp8=True)
    try:
        eng.init_synthetic(seed=0, std=0.02)
        _check_lossless(eng, E.synthetic_prompt(2, P, E.QWEN27B["vocab"]), E.QWEN27B["vocab"])
    finally:
        eng.close()


def test_27b_batch_equals_single_sequences():
    """Two sequences in lockstep (the C4 round structure, bit-exact GEMMs)
    give each sequence's single-sequence tokens and round records."""
    from hybridai_amd import engine as E
    B = 2
    prompts = np.stack([E.synthetic_prompt(10 + b, P, E.QWEN27B["vocab"]) for b in range(B)])
    single = E.Engine(E.QWEN27B, max_context=P + 5 * NEW + 32, max_verify_tokens=16)
    rand = np.random.default_rng(3).integers(0, E.QWEN27B["vocab"], NEW).astype(np.int32)
    try:
        single.init_synthetic(seed=0, std=0.02)
        g = [single.greedy(prompts[b], NEW) for b in range(B)]
        ov = np.stack([g[0], rand])  # sequence 0 accepts every draft, sequence 1 almost none
        want = [single.speculative(prompts[b], NEW, 3, draft_override=ov[b]) for b in range(B)]
    finally:
        single.close()
    eng = E.Engine(E.QWEN27B, max_context=P + 5 * NEW + 32, max_verify_tokens=16, batch=B)
    try:
        eng.init_synthetic(seed=0, std=0.02)
        got = eng.speculative_batch(prompts, NEW, 3, draft_override=ov)
    finally:
        eng.close()
    for b in range(B):
        assert list(got[b][0]) == list(want[b][0]) == list(g[b]), b
        assert np.array_equal(got[b][2], want[b][2]), b


@pytest.mark.parametrize("fp8", [False, True], ids=["bf16", "fp8"])
def test_27b_mfma_batch_logits_within_rounding_sensitivity(fp8):
    """The C4 / C5 tolerance mode at the 27B shape: a batch forward whose
    GEMMs run on the matrix cores (32 rows per launch, narrow layers split K
    and finish inside the next RMSNorm) against the bit-exact engine.

    64 layers of random weights amplify any rounding-level change: scaling
    every weight by (1 + 2^-8), half a bf16 ulp, moves the logits by ~0.1 on
    average (measured on MI355X: 0.108 bf16, 0.339 FP8), so the 2e-2 / 1e-2
    logit bound, met at the tiny depth (tests/test_gpu_engine_batch.py), is
    not a property any differently-rounded path can have here.  The bound
    checked is that the matrix-core path moves the logits no more than that
    half-ulp weight change does (measured: 0.060 / 0.056 mean)."""
    from hybridai_amd import engine as E
    B, T = 2, 16
    prompts = np.stack([E.synthetic_prompt(30 + b, T, E.QWEN27B["vocab"]) for b in range(B)])

    def exact_logits(std):
        eng = E.Engine(E.QWEN27B, max_context=T + 32, max_verify_tokens=16, fp8=fp8)
        try:
            eng.init_synthetic(seed=0, std=std)
            return np.stack([hai.bf16_to_f32(eng.forward(prompts[b])[1]) for b in range(B)])
        finally:
            eng.close()

    want = exact_logits(0.02)
    nudged = exact_logits(0.02 * (1 + 2 ** -8))
    eng = E.Engine(E.QWEN27B, max_context=T + 32, max_verify_tokens=16, fp8=fp8, batch=B, mfma=True)
    try:
        eng.init_synthetic(seed=0, std=0.02)
        got = hai.bf16_to_f32(eng.forward_batch(prompts)[1])
    finally:
        eng.close()
    d_mfma, d_nudge = np.abs(got - want), np.abs(nudged - want)
    assert np.isfinite(got).all()
    assert d_mfma.mean() <= d_nudge.mean(), (float(d_mfma.mean()), float(d_nudge.mean()))
    assert np.percentile(d_mfma, 99) <= np.percentile(d_nudge, 99)
    assert np.mean(got.argmax(-1) == want.argmax(-1)) >= np.mean(nudged.argmax(-1) == want.argmax(-1))


def test_c3_workload_full_decode():
    """C3 as BASELINE.json configures it: a 1024-token prompt through the fast
    prefill (1024-row chunks), then 256 new tokens at MTP depth 1.  Greedy
    decoding gives the reference continuation; the speculative decode with
    that continuation perturbed at 5 % of positions as drafts (the bench's
    headline leg: partial acceptance, corrections and rollbacks across the
    whole 1024 -> 1280 context) equals it token for token with the round
    bookkeeping adding up, and so does the speculative decode with the MTP
    head's own proposals."""
    from hybridai_amd import engine as E
    P, NEW = 1024, 256
    V = E.QWEN27B["vocab"]
    eng = E.Engine(E.QWEN27B, max_context=P + NEW + 32, max_verify_tokens=16, prefill_rows=1024)
    try:
        eng.init_synthetic(seed=0, std=0.02)
        prompt = E.synthetic_prompt(0, P, V)
        g = eng.greedy(prompt, NEW)
        assert len(g) == NEW
        rng = np.random.default_rng(7)
        drafts = g.copy()
        flip = rng.random(NEW) < 0.05
        flip[0] = False
        drafts[flip] = (drafts[flip] + 1) % V
        toks, st, log = eng.speculative(prompt, NEW, 1, draft_override=drafts)
        assert list(toks) == list(g)
        assert st["proposed"] == st["accepted"] + st["rejected"]
        assert st["corrections"] == st["rejected"] > 0
        assert st["accepted"] >= 0.85 * st["proposed"], st
        toks, st, _ = eng.speculative(prompt, NEW, 1)
        assert list(toks) == list(g)
        assert st["proposed"] == st["accepted"] + st["rejected"]
    finally:
        eng.close()
