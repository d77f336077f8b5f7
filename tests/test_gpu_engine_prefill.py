"""Fast prefill (hai_engine_options::prefill_rows): prompts in chunks of
that many rows per sequence, every GEMM of the chunk tiled on the matrix
cores, matrix-core attention, DeltaNet as chained 16-token launches inside
one call, lm_head on the last row only.  Tolerance mode for the prompt, so
checked as the other matrix-core paths are:

* tiny config against the CPU oracle: logits within 2e-2 + 1e-2 |logit|
  (the matrix-core engine's bound), argmax agreement above 90 %; FP8
  against the oracle's FP8 model; a decode after a fast prefill, on the
  bit-exact or the matrix-core decode path, teacher-forced against the
  oracle's forward of the emitted prefix;
* the 27B shape, where the oracle cannot run: the fast prefill moves the
  logits no more than scaling every weight by (1 + 2^-8) moves the exact
  engine's (the rounding sensitivity of 64 random layers), and a greedy
  decode after it is teacher-forced against the same engine's forward
  (each token within the 99.9th percentile of that sensitivity of the
  forward's argmax)."""
import numpy as np
import pytest

from _hai import hai, orc
from test_gpu_engine_mfma_decode import teacher_forced

pytestmark = pytest.mark.gpu


def tol(top):
    return 2 * (2e-2 + 1e-2 * abs(top))


@pytest.mark.parametrize("B,P,rows,mfma,fp8", [(1, 200, 64, False, False), (3, 150, 48, False, False),
                                               (2, 130, 64, True, False), (2, 100, 32, True, True)])
def test_tiny_fast_prefill_logits(B, P, rows, mfma, fp8):
    from hybridai_amd import engine as E
    seed = 3 if fp8 else 0
    prompts = np.stack([orc.synthetic_prompt(60 + b, P, orc.TINY["vocab"]) for b in range(B)])
    ref = orc.Model(orc.TINY, seed=seed, fp8=fp8)
    eng = E.Engine(E.TINY, max_context=P + 32, max_verify_tokens=16, batch=B, mfma=mfma, fp8=fp8,
                   prefill_rows=rows)
    try:
        eng.init_synthetic(seed=seed, std=0.02)
        _, lg = eng.forward_batch(prompts) if B > 1 else (None, eng.forward(prompts[0])[1][None])
        for b in range(B):
            _, rl = ref.forward(prompts[b])
            got = hai.bf16_to_f32(lg[b])
            assert np.allclose(got, rl, atol=2e-2, rtol=1e-2), float(np.abs(got - rl).max())
            assert np.mean(got.argmax(1) == rl.argmax(1)) > 0.9
    finally:
        eng.close()
        ref.close()


@pytest.mark.parametrize("mfma", [False, True], ids=["exact_decode", "mfma_decode"])
def test_tiny_decode_after_fast_prefill(mfma):
    """Speculative decode at depth 3 of three sequences after a fast prefill
    of 150-token prompts in 64-row chunks: every emitted token within the
    tolerance of the oracle's argmax over the emitted prefix."""
    from hybridai_amd import engine as E
    B, P, NEW, W = 3, 150, 40, 3
    V = orc.TINY["vocab"]
    prompts = np.stack([orc.synthetic_prompt(80 + b, P, V) for b in range(B)])
    ref = orc.Model(orc.TINY, seed=0)
    eng = E.Engine(E.TINY, max_context=P + (W + 2) * (NEW + W + 1) + 32, max_verify_tokens=16, batch=B, mfma=mfma,
                   prefill_rows=64)
    try:
        eng.init_synthetic(seed=0, std=0.02)
        res = eng.speculative_batch(prompts, NEW, W)
        for b in range(B):
            toks = res[b][0]
            assert len(toks) == NEW
            seq = np.concatenate([prompts[b], toks[:-1]]).astype(np.int32)
            _, lg = ref.forward(seq)
            teacher_forced(toks, lg[P - 1:], tol, f"sequence {b}", 0.9)
    finally:
        eng.close()
        ref.close()


def test_27b_fast_prefill_within_rounding_sensitivity():
    from hybridai_amd import engine as E
    P = 600
    prompt = E.synthetic_prompt(7, P, E.QWEN27B["vocab"])

    def exact_logits(std):
        eng = E.Engine(E.QWEN27B, max_context=P + 32, max_verify_tokens=16)
        try:
            eng.init_synthetic(seed=0, std=std)
            return hai.bf16_to_f32(eng.forward(prompt)[1])
        finally:
            eng.close()

    want = exact_logits(0.02)
    nudged = exact_logits(0.02 * (1 + 2 ** -8))
    eng = E.Engine(E.QWEN27B, max_context=P + 64, max_verify_tokens=16, prefill_rows=256)
    try:
        eng.init_synthetic(seed=0, std=0.02)
        got = hai.bf16_to_f32(eng.forward(prompt)[1])
        toks = eng.greedy(prompt, 8)
        seq = np.concatenate([prompt, toks[:-1]]).astype(np.int32)
        lg = hai.bf16_to_f32(eng.forward(seq)[1])
    finally:
        eng.close()
    d_fast, d_nudge = np.abs(got - want), np.abs(nudged - want)
    assert np.isfinite(got).all()
    assert d_fast.mean() <= d_nudge.mean(), (float(d_fast.mean()), float(d_nudge.mean()))
    assert np.percentile(d_fast, 99) <= np.percentile(d_nudge, 99)
    # the decode after a fast prefill (lm_head of the last row only) follows
    # the same engine's full forward of the emitted prefix
    sens = float(np.percentile(d_nudge, 99.9))
    teacher_forced(toks, lg[P - 1:], lambda top: sens, "27B greedy after fast prefill", 0.5)
