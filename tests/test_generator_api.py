"""hybridai::Generator (include/hybrid.h) served by this library: the error
paths on the CPU, a compile of the implementation against the reference's
own hybrid.h, the declared struct members compared with it, and (GPU) the
tiny C1 decode through the public API against the golden vectors."""
import json
import os
import re
import subprocess
from pathlib import Path

import pytest

from _hai import ROOT, orc

DRIVER = ROOT / "tests" / "backend" / "_build" / "generator_run"
REF = Path("/root/reference")
MIRROR = ROOT / "vicold.hybridai_amd" / "host" / "refabi" / "hybrid_api.h"
GOLD = json.loads((ROOT / "tests" / "golden" / "tiny_c1.json").read_text())
needs_reference = pytest.mark.skipif(not REF.is_dir(), reason="reference tree not mounted")


def _driver():
    subprocess.run(["make", "-s", "-C", str(ROOT / "tests" / "backend")], check=True, capture_output=True)
    return str(DRIVER)


def test_error_paths_without_device():
    r = subprocess.run([_driver(), "--cpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr


@needs_reference
def test_generator_compiles_against_reference_header():
    cmd = ["g++", "-std=c++20", "-fsyntax-only", "-Wall", "-DHAI_WITH_REFERENCE_TREE", f"-I{REF / 'include'}",
           f"-I{REF / 'src'}", f"-I{ROOT / 'include'}", f"-I{ROOT / 'vicold.hybridai_amd' / 'host'}",
           str(ROOT / "vicold.hybridai_amd" / "host" / "generator.cc")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def _members(text, struct):
    body = re.search(r"struct HYBRIDAI_API " + struct + r"\s*\{(.*?)\n\};", text, re.S).group(1)
    return re.findall(r"^\s*[\w:<>]+\s+(\w+)\s*(?:=[^;]*)?;", body, re.M)


@needs_reference
@pytest.mark.parametrize("struct", ["GeneratorOptions", "GenerationOptions", "GenerationResult"])
def test_struct_members_match_reference(struct):
    ref = (REF / "include" / "hybrid.h").read_text()
    got = _members(MIRROR.read_text(), struct)
    assert got and got == _members(ref, struct)


def _run(mode, max_new=64, model="synthetic:tiny?seed=0&std=0.02&context=256", prompt_ids=None, width=None):
    prompt = "ids:" + ",".join(str(t) for t in (GOLD["prompt"] if prompt_ids is None else prompt_ids))
    env = {k: v for k, v in os.environ.items() if k != "HYBRIDAI_SPECULATIVE_WIDTH"}
    if width is not None:
        env["HYBRIDAI_SPECULATIVE_WIDTH"] = str(width)
    r = subprocess.run([_driver(), model, mode, prompt, str(max_new)],
                       capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = dict(line.split(" ", 1) for line in r.stdout.strip().splitlines())
    toks = [int(t) for t in lines["tokens"].split()]
    stats = dict(kv.split("=") for kv in lines["stats"].split())
    return toks, stats


@pytest.mark.gpu
def test_greedy_through_public_api():
    toks, stats = _run("greedy")
    assert toks == GOLD["greedy"]
    assert stats["prompt_tokens"] == str(len(GOLD["prompt"])) and stats["text_ok"] == "1"


@pytest.mark.gpu
@pytest.mark.parametrize("width", [1, 2, 3])
def test_speculative_through_public_api(width):
    """HYBRIDAI_SPECULATIVE_WIDTH selects the proposal width
    (generator.cc:124-137); tokens and counters equal the golden vectors."""
    toks, stats = _run("spec", width=width)
    g = GOLD["speculative"][str(width)]
    assert toks == g["tokens"] == GOLD["greedy"]
    for key, name in (("rounds", "rounds"), ("proposed", "proposed"), ("accepted", "accepted"),
                      ("rejected", "rejected"), ("corrections", "corrections"),
                      ("mtp_recovery_tokens", "mtp_recovery_tokens"), ("max_proposal_width", "max_width")):
        assert int(stats[name]) == g["stats"][key], key


@pytest.mark.gpu
@pytest.mark.parametrize("env,width", [(None, 8), ("", 8), ("16", 16), ("0", 8), ("17", 8), ("4x", 8)])
def test_speculative_width_from_environment(env, width):
    """Unset, empty or invalid values give the reference's default width
    8; 16, the largest, verifies 17 rows.  Tokens and counters equal the
    oracle's restatement of the state machine at that width."""
    toks, stats = _run("spec", 40, width=env)
    ref = orc.Model(orc.TINY, seed=0)
    rt, rs, _ = ref.speculative(GOLD["prompt"], 40, width)
    ref.close()
    assert toks == [int(t) for t in rt] == GOLD["greedy"][:40]
    assert int(stats["max_width"]) == rs["max_proposal_width"] == width
    for key in ("rounds", "proposed", "accepted", "rejected", "corrections", "mtp_recovery_tokens"):
        assert int(stats[key]) == rs[key], key


@pytest.mark.gpu
def test_fp8_weights_through_public_api():
    """model_dir "...&weights=fp8": the C5 weight format; the speculative
    decode equals the oracle's greedy decode of its FP8 model."""
    prompt = orc.synthetic_prompt(3, 24, orc.TINY["vocab"])
    toks, stats = _run("spec", 40, "synthetic:tiny?seed=3&std=0.02&context=256&weights=fp8", list(prompt))
    ref = orc.Model(orc.TINY, seed=3, fp8=True)
    assert toks == list(ref.greedy(prompt, 40))
    ref.close()


def test_unknown_weight_format_is_rejected():
    r = subprocess.run([_driver(), "synthetic:tiny?weights=int4", "greedy", "ids:1,2", "4"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode != 0 and "weights=int4" in (r.stdout + r.stderr)
