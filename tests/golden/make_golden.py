"""Writes tests/golden/tiny_c1.json: the CPU oracle's outputs on the tiny C1
configuration (4 layers D,D,D,G, hidden 256, vocab 4096, 1 MTP layer, bf16
N(0, 0.02) synthetic weights, seed 0, 32-token prompt, 64 new tokens).

The reference's own implementation cannot run here (its CPU backend cannot
execute the path and its HIP kernels do not build on ROCm 7.2), so these are
regression vectors of the pinned oracle: any change to the oracle's numerics
or to the speculative state machine shows up as a difference.  Run from the
repository root:  python tests/golden/make_golden.py
"""
import hashlib
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import oracle as orc  # noqa: E402

P, NEW = 32, 64


def digest(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()[:32]


def main():
    cfg = orc.TINY
    m = orc.Model(cfg, seed=0)
    prompt = orc.synthetic_prompt(0, P, cfg["vocab"])
    out = {"config": "tiny C1", "seed": 0, "prompt": [int(t) for t in prompt]}
    out["weights_sha256_32"] = {str(t): digest(orc.f32_to_bf16_bits(m.tensor(t)))
                               for t in (0, 1, 2, 64, 65, 66, 67, 128, 130, 132, 138, 141, 322, 327, 329, 1024 * 64 + 11)
                               if _has(m, t)}
    hid, lg = m.forward(prompt)
    out["prefill_hidden_sha256_32"] = digest(orc.f32_to_bf16_bits(hid))
    out["prefill_logits_sha256_32"] = digest(orc.f32_to_bf16_bits(lg))
    out["prefill_last_argmax"] = int(np.argmax(lg[-1]))
    greedy = m.greedy(prompt, NEW)
    out["greedy"] = [int(t) for t in greedy]
    out["speculative"] = {}
    for width in (1, 2, 3):
        toks, st, log = m.speculative(prompt, NEW, width)
        out["speculative"][str(width)] = {
            "tokens": [int(t) for t in toks],
            "stats": {k: int(v) for k, v in st.items() if isinstance(v, (int, np.integer))},
            "round_log": np.asarray(log).astype(int).tolist(),
        }
    m.close()
    path = Path(__file__).with_name("tiny_c1.json")
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {path}")


def _has(m, t):
    try:
        m.tensor(t)
        return True
    except KeyError:
        return False


if __name__ == "__main__":
    main()
