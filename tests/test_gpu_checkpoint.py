"""Checkpoints on the GPU: the tiny C1 model written as a Qwen checkpoint
(oracle weights under the reference's names, tests/ckpt.py) and loaded by
hai_engine_load_checkpoint must give the engine the oracle's weights bit
for bit, and so the oracle's tokens and round logs; with FP8 Linears
(F8_E4M3 + weight_scale_inv, sharded, F32 or BF16-widened scales) the
oracle's FP8 model.  Through hybridai::Generator, a checkpoint directory
takes text prompts through its tokenizer, decodes the oracle's tokens and
stops at the stop ids of its config.json and generation_config.json."""
import json
import os
import subprocess

import numpy as np
import pytest
import torch

import ckpt
import tok
from _hai import ROOT, hai, orc

pytestmark = pytest.mark.gpu

P, NEW = 32, 64
GOLD = json.loads((ROOT / "tests" / "golden" / "tiny_c1.json").read_text())


@pytest.fixture(scope="module")
def dirs(tmp_path_factory):
    base = tmp_path_factory.mktemp("ckpt")
    return {"bf16": ckpt.write_tiny_checkpoint(base / "bf16"),
            "fp8": ckpt.write_tiny_checkpoint(base / "fp8", fp8=True, shards=3)}


def _engine(E, d, fp8):
    cfg, eos, fmt = E.model_config_load(d)
    assert fmt == (E.WEIGHTS_FP8_BLOCK128 if fp8 else E.WEIGHTS_BF16)
    eng = E.Engine(cfg, max_context=P + NEW + 32, max_verify_tokens=17, fp8=fp8)
    eng.load_checkpoint(d)
    return eng


def test_bf16_checkpoint_weights_and_decode(dirs):
    from hybridai_amd import engine as E
    eng = _engine(E, dirs["bf16"], False)
    ref = orc.Model(orc.TINY, seed=0)
    try:
        for tid, name, _ in ckpt.tensor_list(orc.TINY):
            got = hai.bf16_to_f32(eng.read_tensor(tid))
            assert np.array_equal(got.view(np.uint32), ref.tensor(tid).astype(np.float32).view(np.uint32)), name
        prompt = orc.synthetic_prompt(0, P, orc.TINY["vocab"])
        toks, st, log = eng.speculative(prompt, NEW, 1)
        rtoks, rst, rlog = ref.speculative(prompt, NEW, 1)
        assert list(toks) == list(rtoks)
        assert np.array_equal(log, rlog)
        toks3, _, _ = eng.speculative(prompt, NEW, 3)
        assert list(toks3) == list(ref.greedy(prompt, NEW))
    finally:
        eng.close()
        ref.close()


def test_fp8_checkpoint_equals_the_oracle_fp8_model(dirs):
    from hybridai_amd import engine as E
    eng = _engine(E, dirs["fp8"], True)
    ref = orc.Model(orc.TINY, seed=0, fp8=True)
    try:
        prompt = orc.synthetic_prompt(0, P, orc.TINY["vocab"])
        _, lg = eng.forward(prompt)
        _, rlg = ref.forward(prompt)
        assert np.array_equal(hai.bf16_to_f32(lg).view(np.uint32), rlg.astype(np.float32).view(np.uint32))
        toks, _, log = eng.speculative(prompt, NEW, 2)
        rtoks, _, rlog = ref.speculative(prompt, NEW, 2)
        assert list(toks) == list(rtoks) and np.array_equal(log, rlog)
    finally:
        eng.close()
        ref.close()


def test_format_mismatch_and_bf16_scales(dirs, tmp_path):
    """An engine created for the other weight format refuses the checkpoint;
    BF16 scale grids are widened exactly (scales chosen as bf16 numbers)."""
    from hybridai_amd import engine as E
    cfg, _, _ = E.model_config_load(dirs["fp8"])
    eng = E.Engine(cfg, max_context=P + NEW + 32, max_verify_tokens=16, fp8=False)
    try:
        with pytest.raises(RuntimeError, match="FP8"):
            eng.load_checkpoint(dirs["fp8"])
    finally:
        eng.close()
    d = ckpt.write_tiny_checkpoint(tmp_path / "bs", fp8=True, scale_dtype=torch.bfloat16)
    eng = _engine(E, d, True)
    try:
        prompt = orc.synthetic_prompt(0, P, orc.TINY["vocab"])
        toks = eng.greedy(prompt, 16)
        assert len(toks) == 16
    finally:
        eng.close()


def _generator_run(model_dir, mode, prompt, max_new, width=1, layout="plain", **env_extra):
    subprocess.run(["make", "-s", "-C", str(ROOT / "tests" / "backend")], check=True, capture_output=True)
    env = dict(os.environ, HYBRIDAI_SPECULATIVE_WIDTH=str(width), **env_extra)
    return subprocess.run([str(ROOT / "tests" / "backend" / "_build" / "generator_run"), str(model_dir), mode, prompt,
                           str(max_new), layout], capture_output=True, text=True, timeout=300, env=env)


def _generator(model_dir, mode, prompt, max_new, width=1, layout="plain"):
    """(tokens, stats, text) of hybridai::Generator through tests/backend/generator_run."""
    r = _generator_run(model_dir, mode, prompt, max_new, width, layout)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = dict(line.split(" ", 1) for line in r.stdout.strip().splitlines())
    stats = dict(kv.split("=") for kv in lines["stats"].split())
    text = b"" if lines["text_hex"] == "-" else bytes.fromhex(lines["text_hex"])
    return [int(t) for t in lines["tokens"].split()], stats, text.decode(errors="replace")


TEXT = "The quick brown fox can't wait: 你好, мир! 12 apples.\n"


def test_generator_encodes_text_and_decodes_the_result(dirs):
    """A text prompt through the public API: encoded by the checkpoint's
    tokenizer.json (the ids the HF library gives), plain or in the chat
    layout (generator.cc:468-474); the tokens equal the oracle's greedy
    decode of those ids at widths 1 and 3, and result.text is their decoding
    without special tokens (generator.cc:1032, 1275)."""
    hf = tok.hf(dirs["bf16"])
    ref = orc.Model(orc.TINY, seed=0)
    try:
        for layout, text in (("plain", TEXT), ("chat", f"<|im_start|>user\n{TEXT}<|im_end|>\n"
                                                       "<|im_start|>assistant\n<think>\n\n</think>\n\n"),
                             ("chat-think", f"<|im_start|>user\n{TEXT}<|im_end|>\n<|im_start|>assistant\n<think>\n")):
            ids = hf.encode(text).ids
            want = [int(t) for t in ref.greedy(ids, NEW)]
            for width in (1, 3):
                toks, stats, out = _generator(dirs["bf16"], "spec", TEXT, NEW, width=width, layout=layout)
                assert toks == want, (layout, width)
                assert int(stats["prompt_tokens"]) == len(ids)
                assert out == hf.decode(want, skip_special_tokens=True)
    finally:
        ref.close()


def test_generator_stop_ids_from_config_and_generation_config(tmp_path):
    """Stop ids are config.json's eos_token_id joined with
    generation_config.json's (generator.cc:476-480): greedy and speculative
    decoding stop at the first one emitted, whichever file names it."""
    d0 = ckpt.write_tiny_checkpoint(tmp_path / "plain")
    ids = tok.hf(d0).encode(TEXT).ids
    ref = orc.Model(orc.TINY, seed=0)
    g = [int(t) for t in ref.greedy(ids, NEW)]
    ref.close()
    firsts = [k for k in range(3, NEW) if g[k] not in g[:k]]  # positions where a token first appears
    b = g[firsts[0]]
    a = g[next(k for k in firsts if k >= firsts[0] + 3)]
    d = ckpt.write_tiny_checkpoint(tmp_path / "eos", eos=[orc.TINY["vocab"] - 1, a], generation_eos=[b])
    for mode in ("spec", "greedy"):
        assert _generator(d, mode, TEXT, NEW)[0] == g[:g.index(b) + 1]
    d = ckpt.write_tiny_checkpoint(tmp_path / "eos2", eos=a, generation_eos=orc.TINY["vocab"] - 2)
    assert _generator(d, "spec", TEXT, NEW)[0] == g[:g.index(a) + 1]


def test_generator_context_bound_is_max_position_embeddings(dirs):
    """A checkpoint engine takes prompt + max_new_tokens up to
    max_position_embeddings (4096 in the test config), with the reference's
    check and message (generator.cc:481-485); HYBRIDAI_MAX_CONTEXT caps the
    positions (the KV memory) and a request above the cap names it."""
    d = dirs["bf16"]
    n = len(tok.hf(d).encode(TEXT).ids)
    r = _generator_run(d, "greedy", TEXT, 4097 - n)
    assert r.returncode == 1 and "generate failed" in r.stdout and "prompt exceeds model context" in r.stdout, r.stdout
    r = _generator_run(d, "spec", TEXT, 64 - n, width=3, HYBRIDAI_MAX_CONTEXT="64")
    assert r.returncode == 0, r.stdout + r.stderr
    r = _generator_run(d, "spec", TEXT, 65 - n, width=3, HYBRIDAI_MAX_CONTEXT="64")
    assert r.returncode == 1 and "exceed HYBRIDAI_MAX_CONTEXT (64 positions)" in r.stdout, r.stdout
