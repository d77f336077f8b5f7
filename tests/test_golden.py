"""Golden vectors of the tiny C1 configuration (tests/golden/tiny_c1.json,
written by tests/golden/make_golden.py): the CPU oracle must reproduce them
exactly, and so must the GPU engine (marked gpu).  Speculative decoding must
also emit exactly the plain greedy continuation."""
import hashlib
import json

import numpy as np
import pytest

from _hai import ROOT, hai, orc

GOLD = json.loads((ROOT / "tests" / "golden" / "tiny_c1.json").read_text())
P, NEW = 32, 64


def digest(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()[:32]


@pytest.fixture(scope="module")
def oracle_model():
    m = orc.Model(orc.TINY, seed=0)
    yield m
    m.close()


def test_prompt_stream(oracle_model):
    assert [int(t) for t in orc.synthetic_prompt(0, P, orc.TINY["vocab"])] == GOLD["prompt"]


def test_oracle_weights(oracle_model):
    for tid, want in GOLD["weights_sha256_32"].items():
        assert digest(orc.f32_to_bf16_bits(oracle_model.tensor(int(tid)))) == want, tid


def test_oracle_prefill(oracle_model):
    hid, lg = oracle_model.forward(np.array(GOLD["prompt"], np.int64))
    assert digest(orc.f32_to_bf16_bits(hid)) == GOLD["prefill_hidden_sha256_32"]
    assert digest(orc.f32_to_bf16_bits(lg)) == GOLD["prefill_logits_sha256_32"]


def test_oracle_greedy_and_speculative(oracle_model):
    prompt = np.array(GOLD["prompt"], np.int64)
    assert [int(t) for t in oracle_model.greedy(prompt, NEW)] == GOLD["greedy"]
    for width, g in GOLD["speculative"].items():
        toks, st, log = oracle_model.speculative(prompt, NEW, int(width))
        assert [int(t) for t in toks] == g["tokens"] == GOLD["greedy"]
        assert np.asarray(log).astype(int).tolist() == g["round_log"]
        for k, v in g["stats"].items():
            assert int(st[k]) == v, (width, k)


@pytest.mark.gpu
def test_engine_reproduces_golden():
    from hybridai_amd import engine as E
    eng = E.Engine(E.TINY, max_context=P + NEW + 32, max_verify_tokens=16)
    try:
        eng.init_synthetic(seed=0, std=0.02)
        prompt = np.array(GOLD["prompt"], np.int64)
        hid, lg = eng.forward(prompt)
        assert digest(hid) == GOLD["prefill_hidden_sha256_32"]
        assert digest(lg) == GOLD["prefill_logits_sha256_32"]
        assert [int(t) for t in eng.greedy(prompt, NEW)] == GOLD["greedy"]
        for width, g in GOLD["speculative"].items():
            toks, st, log = eng.speculative(prompt, NEW, int(width))
            assert [int(t) for t in toks] == g["tokens"]
            assert np.asarray(log).astype(int).tolist() == g["round_log"]
    finally:
        eng.close()
