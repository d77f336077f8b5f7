"""Checkpoints on the GPU: the tiny C1 model written as a Qwen checkpoint
(oracle weights under the reference's names, tests/ckpt.py) and loaded by
hai_engine_load_checkpoint must give the engine the oracle's weights bit
for bit, and so the oracle's tokens and round logs; with FP8 Linears
(F8_E4M3 + weight_scale_inv, sharded, F32 or BF16-widened scales) the
oracle's FP8 model.  Through hybridai::Generator, a checkpoint directory
decodes the golden tokens and stops at the EOS ids of its config.json."""
import json
import os
import subprocess

import numpy as np
import pytest
import torch

import ckpt
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


def _generator(model_dir, mode, prompt, max_new, width=1):
    subprocess.run(["make", "-s", "-C", str(ROOT / "tests" / "backend")], check=True, capture_output=True)
    env = dict(os.environ, HYBRIDAI_SPECULATIVE_WIDTH=str(width))
    r = subprocess.run([str(ROOT / "tests" / "backend" / "_build" / "generator_run"), str(model_dir), mode, prompt,
                        str(max_new)], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    return [int(t) for t in r.stdout.split("\n")[0].split()[1:]]


def test_generator_loads_a_checkpoint_directory(dirs, tmp_path):
    """The golden C1 decode (tests/golden/tiny_c1.json) from a checkpoint
    directory through the public API, at widths 1 and 3; then EOS ids read
    from config.json stop greedy and speculative decoding at the first one
    emitted."""
    g = list(GOLD["greedy"])
    prompt = "ids:" + ",".join(str(int(t)) for t in GOLD["prompt"])
    assert _generator(dirs["bf16"], "spec", prompt, NEW, width=1) == g[:NEW]
    assert _generator(dirs["bf16"], "spec", prompt, NEW, width=3) == g[:NEW]
    stop = g[5]
    d = ckpt.write_tiny_checkpoint(tmp_path / "eos", eos=[orc.TINY["vocab"] - 1, stop])
    assert _generator(d, "spec", prompt, NEW) == g[:g.index(stop) + 1]
    assert _generator(d, "greedy", prompt, NEW) == g[:g.index(stop) + 1]
