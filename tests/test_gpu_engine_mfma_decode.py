"""Speculative decode of the matrix-core engine (tolerance mode: MFMA GEMMs
for launches of 4 or more rows and MFMA attention), the path of the C4 / C5
benchmark configurations, with forced full, partial and no acceptance per
sequence (draft overrides).

The matrix-core kernels choose their split plans from the launch's row
count, so a verify row, a correction row and a prefill row of one position
may round differently and an argmax may flip where the top two logits are
within rounding of each other.  Token streams are therefore checked
teacher-forced: every emitted token must be the argmax, or within a stated
logit tolerance of the argmax, of a forward over the emitted prefix -- the
CPU oracle's (tiny config, tolerance 2 x (2e-2 + 1e-2 |logit|), the logit
bound of the verify path) or, at the 27B shape where the oracle cannot run,
the same engine's batch prefill forward.  A cache or rollback mistake gives
tokens whose logits sit several units below the maximum.  The state
machine's bookkeeping (accepted prefixes, corrections, cache lengths,
counters) is checked exactly from each decode's outputs (specmath.py)."""
import numpy as np
import pytest

from _hai import hai, orc
from specmath import check_rounds

pytestmark = pytest.mark.gpu


def forced_overrides(ref_tokens, kinds, vocab, seed):
    """One override row per sequence: "full" drafts the reference
    continuation, "partial" perturbs a few positions of it, "none" drafts
    random tokens."""
    rng = np.random.default_rng(seed)
    rows = []
    for toks, kind in zip(ref_tokens, kinds):
        t = np.array(toks, np.int32).copy()
        if kind == "partial":
            for i in range(2, len(t), 5):
                t[i] = (t[i] + 1 + int(rng.integers(vocab - 1))) % vocab
        elif kind == "none":
            t = rng.integers(0, vocab, len(t)).astype(np.int32)
        rows.append(t)
    return np.stack(rows)


def teacher_forced(tokens, logits_rows, delta_fn, what, min_agree):
    """logits_rows[i] is the forward's prediction for tokens[i]."""
    agree = 0
    for i, t in enumerate(tokens):
        row = logits_rows[i]
        top = float(row.max())
        gap = top - float(row[int(t)])
        assert gap <= delta_fn(top), f"{what}: token {i} = {int(t)} is {gap:.3f} below the argmax logit {top:.3f}"
        agree += int(int(np.argmax(row)) == int(t))
    assert agree >= min_agree * len(tokens), f"{what}: argmax agreement {agree}/{len(tokens)}"


# ---------------------------------------------------------------- tiny config vs the CPU oracle
def test_tiny_mfma_speculative_against_oracle():
    """Three sequences at depth 3 on the matrix-core engine, drafts forced
    from the engine's own continuation (the oracle's may differ from it at a
    near-tie, after which none of its drafts would match)."""
    from hybridai_amd import engine as E
    B, P, NEW, W = 3, 24, 40, 3
    V = orc.TINY["vocab"]
    prompts = np.stack([orc.synthetic_prompt(40 + b, P, V) for b in range(B)])
    ref = orc.Model(orc.TINY, seed=0)
    eng = E.Engine(E.TINY, max_context=P + (W + 2) * (NEW + W + 1) + 32, max_verify_tokens=16, batch=B, mfma=True)
    try:
        eng.init_synthetic(seed=0, std=0.02)
        rng = np.random.default_rng(2)
        first = eng.speculative_batch(prompts, NEW + W + 1, W,
                                      draft_override=rng.integers(0, V, (B, NEW + W + 1)).astype(np.int32))
        ov = forced_overrides([r[0] for r in first], ["full", "partial", "none"], V, 1)
        res = eng.speculative_batch(prompts, NEW, W, draft_override=ov)
        for b in range(B):
            toks, st, log = res[b]
            assert len(toks) == NEW
            check_rounds(toks, log, st, P, NEW)
            seq = np.concatenate([prompts[b], toks[:-1]]).astype(np.int32)
            _, lg = ref.forward(seq)
            teacher_forced(toks, lg[P - 1:], lambda top: 2 * (2e-2 + 1e-2 * abs(top)), f"sequence {b}", 0.9)
        assert res[0][1]["accepted"] >= 0.5 * res[0][1]["proposed"]
        assert 0 < res[1][1]["accepted"] < res[1][1]["proposed"]
        assert res[2][1]["accepted"] <= 1
    finally:
        eng.close()
        ref.close()


# ---------------------------------------------------------------- 27B shape (C4 / C5 structure)
def run_forced(E, fp8, B, P, NEW, W, kinds, seed, max_context=None):
    """The C4 / C5 round structure at the 27B shape: a first decode with
    random drafts gives each sequence's own continuation, the second forces
    the acceptance pattern of `kinds` with it.  Returns the engine (open),
    the prompts and the second decode's results."""
    V = E.QWEN27B["vocab"]
    prompts = np.stack([E.synthetic_prompt(seed + b, P, V) for b in range(B)])
    cap = max_context or P + (W + 2) * (NEW + W + 1) + 64
    eng = E.Engine(E.QWEN27B, max_context=cap, max_verify_tokens=16, fp8=fp8, batch=B, mfma=True)
    eng.init_synthetic(seed=0, std=0.02)
    rng = np.random.default_rng(seed)
    first = eng.speculative_batch(prompts, NEW + W + 1, W,
                                  draft_override=rng.integers(0, V, (B, NEW + W + 1)).astype(np.int32))
    for b in range(B):
        check_rounds(first[b][0], first[b][2], first[b][1], P, NEW + W + 1)
    ov = forced_overrides([r[0] for r in first], kinds, V, seed + 1)
    res = eng.speculative_batch(prompts, NEW, W, draft_override=ov)
    return eng, prompts, res


def check_27b(eng, prompts, res, kinds, NEW):
    B, P = prompts.shape
    for b in range(B):
        toks, st, log = res[b]
        assert len(toks) == NEW
        check_rounds(toks, log, st, P, NEW)
        if kinds[b] == "full":
            assert st["accepted"] >= 0.5 * st["proposed"], (b, st)
        elif kinds[b] == "none":
            assert st["accepted"] == 0 and st["corrections"] == st["rounds"], (b, st)
    assert any(0 < r[1]["accepted"] < r[1]["proposed"] for r, k in zip(res, kinds) if k == "partial")
    seq = np.stack([np.concatenate([prompts[b], res[b][0][:-1]]) for b in range(B)]).astype(np.int32)
    _, lg = eng.forward_batch(seq)
    for b in range(B):
        rows = hai.bf16_to_f32(lg[b, P - 1:])
        # every token within 0.5 of the argmax logit (a wrong cache gives
        # gaps of several units: the logits' spread is ~1.4 at this shape);
        # the argmax itself flips at near-ties -- the top two of 248320
        # random logits are ~0.3 apart on average and the two paths differ
        # by ~0.06 -- so agreement is only bounded from below
        teacher_forced(res[b][0], rows, lambda top: 0.5, f"sequence {b}", 0.5)


def test_c4_shape_mfma_bf16_decode():
    """27B bf16, 8 sequences, chained depth 3 (verify of 32 rows)."""
    from hybridai_amd import engine as E
    kinds = ["full", "full", "partial", "partial", "partial", "none", "none", "full"]
    eng, prompts, res = run_forced(E, False, 8, 64, 20, 3, kinds, 100)
    try:
        check_27b(eng, prompts, res, kinds, 20)
    finally:
        eng.close()


def test_c5_shape_mfma_fp8_decode():
    """27B FP8 weights, 32 sequences, depth 1 (verify of 64 rows)."""
    from hybridai_amd import engine as E
    kinds = (["full", "partial", "none", "full"] * 8)
    eng, prompts, res = run_forced(E, True, 32, 48, 12, 1, kinds, 200)
    try:
        check_27b(eng, prompts, res, kinds, 12)
    finally:
        eng.close()


def test_c4_long_prompt_rollback_bookkeeping():
    """The C4 workload's 8 x 8192-token prompts: forced full, partial and no
    acceptance at depth 3, the DeltaNet state and KV rolled back by length
    at every partial acceptance; every round's bookkeeping exact and the
    forced-full sequences accepted."""
    from hybridai_amd import engine as E
    kinds = ["full", "partial", "none", "full", "partial", "none", "full", "partial"]
    P, NEW, W = 8192, 12, 3
    eng, prompts, res = run_forced(E, False, 8, P, NEW, W, kinds, 300)
    try:
        for b in range(8):
            toks, st, log = res[b]
            assert len(toks) == NEW
            check_rounds(toks, log, st, P, NEW)
            if kinds[b] == "full":
                assert st["accepted"] >= 0.5 * st["proposed"], (b, st)
            if kinds[b] == "none":
                assert st["accepted"] == 0, (b, st)
        assert any(0 < r[1]["accepted"] < r[1]["proposed"] for r, k in zip(res, kinds) if k == "partial")
    finally:
        eng.close()


def test_c5_workload_prompts_mfma_fp8_decode():
    """C5's 32 x 512-token prompts with FP8 weights at depth 1 (verify of 64
    rows): forced full, partial and no acceptance per sequence, every round's
    bookkeeping exact, and every emitted token within 0.5 of the argmax of a
    fresh forward over the sequence."""
    from hybridai_amd import engine as E
    kinds = (["full", "partial", "none", "full"] * 8)
    eng, prompts, res = run_forced(E, True, 32, 512, 12, 1, kinds, 400)
    try:
        check_27b(eng, prompts, res, kinds, 12)
    finally:
        eng.close()
