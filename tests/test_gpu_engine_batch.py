"""Batched decode (several sequences in lockstep rounds) against the CPU
oracle's single-sequence restatement of the reference state machine: on the
bit-exact GEMMs every sequence's tokens, round records and counters equal its
own single-sequence decode; with the MFMA GEMMs (tolerance mode, launches of
4 or more rows) the batch's logits stay within the 2e-2 abs / 1e-2 rel
bound of the oracle's."""
import numpy as np
import pytest

from _hai import hai, orc

pytestmark = pytest.mark.gpu

B, P, NEW = 3, 24, 40
ROUND_KEYS = ("rounds", "proposed", "accepted", "rejected", "corrections", "mtp_recovery_tokens")


@pytest.fixture(scope="module")
def setup():
    from hybridai_amd import engine as E
    prompts = np.stack([orc.synthetic_prompt(10 + b, P, orc.TINY["vocab"]) for b in range(B)])
    ref = orc.Model(orc.TINY, seed=0)
    eng = E.Engine(E.TINY, max_context=P + 6 * NEW + 32, max_verify_tokens=16, batch=B)
    eng.init_synthetic(seed=0, std=0.02)
    yield eng, ref, prompts
    eng.close()
    ref.close()


def _check_against_oracle(results, ref, prompts, width, overrides=None, eos=()):
    for b in range(B):
        toks, st, log = results[b]
        ov = None if overrides is None else overrides[b]
        rtoks, rst, rlog = ref.speculative(prompts[b], NEW, width, eos=eos, draft_override=ov)
        assert list(toks) == list(rtoks), f"sequence {b}"
        assert np.array_equal(log, rlog), f"sequence {b} round log"
        for key in ROUND_KEYS:
            assert st[key] == rst[key], (b, key)


def test_batched_prefill_logits_bit_exact(setup):
    eng, ref, prompts = setup
    hid, lg = eng.forward_batch(prompts)
    for b in range(B):
        rh, rl = ref.forward(prompts[b])
        assert np.array_equal(hai.bf16_to_f32(hid[b]), rh)
        assert np.array_equal(hai.bf16_to_f32(lg[b]), rl)


@pytest.mark.parametrize("width", [1, 3])
def test_batched_speculative_equals_each_sequence(setup, width):
    eng, ref, prompts = setup
    _check_against_oracle(eng.speculative_batch(prompts, NEW, width), ref, prompts, width)


def test_batched_mixed_acceptance(setup):
    """Sequence 0 drafts its greedy continuation (every draft accepted),
    sequence 1 the same with a few positions perturbed, sequence 2 random
    tokens (almost every draft rejected): full acceptance, partial
    acceptance and corrections in the same rounds."""
    eng, ref, prompts = setup
    rng = np.random.default_rng(4)
    ov = []
    for b in range(B):
        g = ref.greedy(prompts[b], NEW)
        if b == 1:
            g = g.copy()
            for i in (3, 4, 17, 30):
                g[i] = (g[i] + 11) % orc.TINY["vocab"]
        if b == 2:
            g = rng.integers(0, orc.TINY["vocab"], NEW).astype(np.int32)
        ov.append(g)
    ov = np.stack(ov)
    res = eng.speculative_batch(prompts, NEW, 3, draft_override=ov)
    _check_against_oracle(res, ref, prompts, 3, overrides=ov)
    assert res[0][1]["corrections"] == 0 and res[0][1]["accepted"] > 0
    assert res[2][1]["corrections"] > res[1][1]["corrections"]


def test_batched_eos_ends_sequences_at_different_rounds(setup):
    eng, ref, prompts = setup
    g0 = ref.greedy(prompts[0], NEW)
    eos = [int(g0[12])]
    res = eng.speculative_batch(prompts, NEW, 2, eos=eos)
    _check_against_oracle(res, ref, prompts, 2, eos=eos)
    assert len(res[0][0]) <= 13


def test_mfma_batch_logits_within_tolerance():
    from hybridai_amd import engine as E
    prompts = np.stack([orc.synthetic_prompt(20 + b, P, orc.TINY["vocab"]) for b in range(B)])
    ref = orc.Model(orc.TINY, seed=0)
    eng = E.Engine(E.TINY, max_context=P + 32, max_verify_tokens=16, batch=B, mfma=True)
    eng.init_synthetic(seed=0, std=0.02)
    try:
        _, lg = eng.forward_batch(prompts)
        for b in range(B):
            _, rl = ref.forward(prompts[b])
            got = hai.bf16_to_f32(lg[b])
            assert np.allclose(got, rl, atol=2e-2, rtol=1e-2), float(np.abs(got - rl).max())
            # most rows keep their argmax (the tolerance is far below the top-2 gaps)
            assert np.mean(got.argmax(1) == rl.argmax(1)) > 0.9
    finally:
        eng.close()
        ref.close()


def test_mfma_fp8_batch_logits_within_tolerance():
    """FP8 weights on the MFMA path (codes decoded exactly, per-block scale in
    fp32) against the oracle's FP8 model."""
    from hybridai_amd import engine as E
    prompts = np.stack([orc.synthetic_prompt(30 + b, P, orc.TINY["vocab"]) for b in range(B)])
    ref = orc.Model(orc.TINY, seed=3, fp8=True)
    eng = E.Engine(E.TINY, max_context=P + 32, max_verify_tokens=16, batch=B, mfma=True, fp8=True)
    eng.init_synthetic(seed=3, std=0.02)
    try:
        _, lg = eng.forward_batch(prompts)
        for b in range(B):
            _, rl = ref.forward(prompts[b])
            got = hai.bf16_to_f32(lg[b])
            assert np.allclose(got, rl, atol=2e-2, rtol=1e-2), float(np.abs(got - rl).max())
            assert np.mean(got.argmax(1) == rl.argmax(1)) > 0.9
    finally:
        eng.close()
        ref.close()
