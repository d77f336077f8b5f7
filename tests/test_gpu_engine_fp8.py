"""End-to-end parity of the verify engine with FP8 E4M3 weights (128x128
block scales, the C5 weight format) against the CPU oracle's FP8 model: the
synthetic bf16 model quantised with synthetic U(0.5,2)/448 scales, every
QuantizedWeight Linear of the reference then computing with decode(q) * s.
Logits, greedy tokens and every speculative round must be bit-identical.

Two configurations: the tiny config, where every checkpoint tensor starts on
a 128-row block of its stored matrix, and an odd one (hidden 320, one KV head
of 64, DeltaNet qkv of 320 rows, ffn 448) where tensors stacked into one
matrix start mid-block and K ends in a partial block, so the per-row scale
maps are exercised."""
import numpy as np
import pytest

from _hai import hai, orc

pytestmark = pytest.mark.gpu

P, NEW = 32, 48
ODD = dict(hidden=320, num_layers=4, full_attention_interval=4, num_q_heads=3, num_kv_heads=1, head_dim=64,
           rope_dim=16, lin_qk_heads=1, lin_v_heads=3, lin_k_dim=64, lin_v_dim=64, conv_kernel=4, ffn=448,
           vocab=1000, mtp_layers=1, rms_eps=1e-6, rope_theta=1e7)
QUANTIZED_KINDS = {2, 3, 10, 11, 12, 13, 14, 17, 18, 19}


@pytest.fixture(scope="module", params=["tiny", "odd"])
def engines(request):
    from hybridai_amd import engine as E
    cfg = orc.TINY if request.param == "tiny" else ODD
    eng = E.Engine(cfg, max_context=P + NEW + 32, max_verify_tokens=16, fp8=True)
    eng.init_synthetic(seed=3, std=0.02)
    ref = orc.Model(cfg, seed=3, fp8=True)
    prompt = orc.synthetic_prompt(3, P, cfg["vocab"])
    yield eng, ref, prompt, cfg
    eng.close()
    ref.close()


def test_bf16_tensors_match_and_fp8_tensors_are_not_exposed(engines):
    eng, ref, _, _ = engines
    for slot in (0, 1, 2, 5, 1024):
        for kind in range(20):
            tid = slot * 64 + kind
            try:
                want = ref.tensor(tid)
            except KeyError:
                continue
            if slot >= 2 and kind in QUANTIZED_KINDS:
                with pytest.raises(KeyError):
                    eng.read_tensor(tid)
                continue
            assert np.array_equal(hai.bf16_to_f32(eng.read_tensor(tid)), want), f"tensor {tid}"


def test_prefill_logits_bit_exact(engines):
    eng, ref, prompt, _ = engines
    hid, lg = eng.forward(prompt)
    rh, rl = ref.forward(prompt)
    assert np.array_equal(hai.bf16_to_f32(hid), rh)
    assert np.array_equal(hai.bf16_to_f32(lg), rl)


@pytest.mark.parametrize("width", [1, 3])
def test_speculative_matches_reference_state_machine(engines, width):
    eng, ref, prompt, _ = engines
    toks, st, log = eng.speculative(prompt, NEW, width)
    rtoks, rst, rlog = ref.speculative(prompt, NEW, width)
    assert list(toks) == list(rtoks)
    assert np.array_equal(log, rlog)
    assert st["accepted"] == rst["accepted"] and st["corrections"] == rst["corrections"]
    assert list(toks) == list(ref.greedy(prompt, NEW))


def test_forced_partial_acceptance(engines):
    eng, ref, prompt, cfg = engines
    g = ref.greedy(prompt, NEW)
    ov = g.copy()
    for i in (4, 17, 18, 30):
        ov[i] = (ov[i] + 5) % cfg["vocab"]
    toks, st, log = eng.speculative(prompt, NEW, 3, draft_override=ov)
    rtoks, rst, rlog = ref.speculative(prompt, NEW, 3, draft_override=ov)
    assert list(toks) == list(rtoks) == list(g)
    assert np.array_equal(log, rlog)
    assert st["accepted"] == rst["accepted"] > 0
