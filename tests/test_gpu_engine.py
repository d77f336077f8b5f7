"""End-to-end parity of the verify engine with the CPU oracle on the tiny
config of BASELINE.json (4 layers D,D,D,G, hidden 256, vocab 4096, 1 MTP
layer, bf16 ~ N(0, 0.02) synthetic weights seed 0, 32-token prompt, 64 new
tokens, MTP width 1): token ids and every round's candidates / accepted
count must be bit-identical, logits bit-identical."""
import numpy as np
import pytest

from _hai import hai, orc

pytestmark = pytest.mark.gpu

P, NEW = 32, 64


@pytest.fixture(scope="module", params=[False, True], ids=["launches", "graphs"])
def engines(request):
    """The engine with plain launches and with captured HIP graphs (every
    round replays the draft/verify/correction graphs with host
    synchronisations in between; each replay is checked through the round
    logs)."""
    from hybridai_amd import engine as E
    eng = E.Engine(E.TINY, max_context=P + NEW + 32, max_verify_tokens=17, use_graphs=request.param)
    eng.init_synthetic(seed=0, std=0.02)
    ref = orc.Model(orc.TINY, seed=0)
    prompt = orc.synthetic_prompt(0, P, orc.TINY["vocab"])
    yield eng, ref, prompt
    eng.close()
    ref.close()


def test_weights_match_oracle(engines):
    eng, ref, _ = engines
    for slot in (0, 1, 2, 3, 4, 5, 1024):
        for kind in range(20):
            tid = slot * 64 + kind
            try:
                want = ref.tensor(tid)
            except KeyError:
                continue
            got = eng.read_tensor(tid)
            assert np.array_equal(hai.bf16_to_f32(got), want), f"tensor {tid}"


def test_prefill_logits_bit_exact(engines):
    eng, ref, prompt = engines
    hid, lg = eng.forward(prompt)
    rh, rl = ref.forward(prompt)
    assert np.array_equal(hai.bf16_to_f32(hid), rh)
    assert np.array_equal(hai.bf16_to_f32(lg), rl)


def test_greedy_tokens_bit_exact(engines):
    eng, ref, prompt = engines
    assert list(eng.greedy(prompt, NEW)) == list(ref.greedy(prompt, NEW))


@pytest.mark.parametrize("width", [1, 2, 3])
def test_speculative_matches_reference_state_machine(engines, width):
    eng, ref, prompt = engines
    toks, st, log = eng.speculative(prompt, NEW, width)
    rtoks, rst, rlog = ref.speculative(prompt, NEW, width)
    assert list(toks) == list(rtoks)
    assert st["rounds"] == rst["rounds"] and st["accepted"] == rst["accepted"]
    assert st["proposed"] == rst["proposed"] and st["corrections"] == rst["corrections"]
    assert st["mtp_recovery_tokens"] == rst["mtp_recovery_tokens"]
    assert st["replay_tokens"] == rst["replay_tokens"] and st["rejected"] == rst["rejected"]
    assert np.array_equal(log, rlog)
    # speculative decoding emits exactly the greedy continuation
    assert list(toks) == list(ref.greedy(prompt, NEW))


@pytest.mark.parametrize("width,perturb", [(1, ()), (3, ()), (3, (5, 20, 21, 40)), (2, (1, 2, 3, 30)),
                                           (8, (9, 10, 33)), (16, ()), (16, (4, 22, 23, 45))])
def test_forced_acceptance_patterns(engines, width, perturb):
    """Draft override: candidates taken from the greedy continuation (full
    acceptance) with some positions perturbed (partial acceptance)."""
    eng, ref, prompt = engines
    g = ref.greedy(prompt, NEW)
    ov = g.copy()
    for i in perturb:
        ov[i] = (ov[i] + 7) % orc.TINY["vocab"]
    toks, st, log = eng.speculative(prompt, NEW, width, draft_override=ov)
    rtoks, rst, rlog = ref.speculative(prompt, NEW, width, draft_override=ov)
    assert list(toks) == list(rtoks) == list(g)
    assert np.array_equal(log, rlog)
    assert st["accepted"] == rst["accepted"] > 0


@pytest.mark.parametrize("width,perturb", [(1, (3, 9, 10, 27)), (3, (5, 20, 21, 40))])
def test_device_draft_override_in_spec_rounds(engines, width, perturb):
    """The benchmark hook: prefill + spec_rounds with the overrides uploaded
    once (set_draft_override) emit the tokens and counts of
    generate_speculative with the same overrides, and leave later rounds on
    the MTP proposals once cleared."""
    eng, ref, prompt = engines
    g = ref.greedy(prompt, NEW)
    ov = g.copy()
    for i in perturb:
        ov[i] = (ov[i] + 7) % orc.TINY["vocab"]
    want, wst, _ = ref.speculative(prompt, NEW, width, draft_override=ov)
    eng.prefill(prompt, NEW)
    eng.set_draft_override(ov)
    out = np.zeros(NEW, np.int32)
    try:
        n, st = eng.spec_rounds(4096, width, out)
    finally:
        eng.set_draft_override(None)
    assert n == NEW and list(out) == list(want) == list(g)
    for key in ("rounds", "proposed", "accepted", "rejected", "corrections"):
        assert st[key] == wst[key], key
    # cleared: the MTP head proposes again (random weights: nothing accepted)
    eng.prefill(prompt, NEW)
    n, st = eng.spec_rounds(4096, width, out)
    assert list(out[:n]) == list(g[:n]) and st["accepted"] < wst["accepted"]


def test_width_beyond_the_verify_rows_is_rejected(engines):
    """Width 16 (17 verify rows, the largest the reference allows) runs;
    a wider proposal than the engine verifies is an argument error, not a
    silent clamp."""
    eng, ref, prompt = engines
    with pytest.raises(RuntimeError, match="max_verify_tokens"):
        eng.speculative(prompt, NEW, 17)
    toks, st, _ = eng.speculative(prompt, NEW, 16)
    assert list(toks) == list(ref.greedy(prompt, NEW)) and st["max_proposal_width"] == 16


def test_eos_stops_like_reference(engines):
    eng, ref, prompt = engines
    g = ref.greedy(prompt, NEW)
    eos = [int(g[10]), int(g[37])]
    toks, st, log = eng.speculative(prompt, NEW, 2, eos=eos, draft_override=g)
    rtoks, rst, rlog = ref.speculative(prompt, NEW, 2, eos=eos, draft_override=g)
    assert list(toks) == list(rtoks)
    assert toks[-1] in eos
    assert np.array_equal(log, rlog)


def test_eos_draft_ends_the_chain_on_the_device(engines):
    """Width 3 with drafts forced to the greedy continuation: every round
    emits next_target and three accepted drafts, so output position j with
    j % 4 == 2 is the second draft of a chain.  With that token as the only
    EOS id the chain stops after it (generator.cc:845-847): the last round
    proposes 2, not 3, its second candidate is the EOS id, and tokens and
    round logs equal the oracle's.  The chain is counted on the device, so a
    round waits on the stream once (no correction happens)."""
    eng, ref, prompt = engines
    g = ref.greedy(prompt, NEW)
    j = next(j for j in range(6, NEW - 4) if j % 4 == 2 and g[j] not in g[:j])
    eos = [int(g[j])]
    toks, st, log = eng.speculative(prompt, NEW, 3, eos=eos, draft_override=g)
    rtoks, rst, rlog = ref.speculative(prompt, NEW, 3, eos=eos, draft_override=g)
    assert list(toks) == list(rtoks) == list(g[:j + 1])
    assert np.array_equal(log, rlog)
    assert log[-1][0] == 2 and log[-1][9] == eos[0] and log[-1][2] == 1
    assert st["corrections"] == 0 and st["host_syncs"] == st["rounds"] == (j + 2) // 4
    for key in ("rounds", "proposed", "accepted", "rejected"):
        assert st[key] == rst[key], key


def test_eos_set_with_natural_drafts_matches_reference(engines):
    """The MTP head's own proposals (random weights: mostly rejected) with an
    EOS set that holds a draft seen mid-chain in an EOS-free run: tokens and
    round logs equal the oracle's, and the host waits once per round plus
    once per correction."""
    eng, ref, prompt = engines
    _, _, free_log = ref.speculative(prompt, NEW, 3)
    mids = [int(r[8 + 1]) for r in free_log if r[0] == 3]
    eos = [mids[len(mids) // 2]]
    toks, st, log = eng.speculative(prompt, NEW, 3, eos=eos)
    rtoks, rst, rlog = ref.speculative(prompt, NEW, 3, eos=eos)
    assert any(r[0] == 2 and r[9] == eos[0] for r in log[:-1]), "no chain ended on the EOS draft"
    assert list(toks) == list(rtoks)
    assert np.array_equal(log, rlog)
    # a correction that ends the generation runs no correction step
    assert st["rounds"] + st["corrections"] - 1 <= st["host_syncs"] <= st["rounds"] + st["corrections"]


def test_token_ids_outside_vocabulary_are_rejected(engines):
    """Prompt and draft-override ids index the embedding table: ids outside
    [0, vocab) are an argument error before anything runs, and the engine
    decodes normally afterwards."""
    eng, ref, prompt = engines
    bad = prompt.copy()
    bad[3] = orc.TINY["vocab"]
    with pytest.raises(RuntimeError, match="outside the vocabulary"):
        eng.speculative(bad, NEW, 1)
    ov = ref.greedy(prompt, NEW).copy()
    ov[5] = -1
    with pytest.raises(RuntimeError, match="outside the vocabulary"):
        eng.speculative(prompt, NEW, 2, draft_override=ov)
    with pytest.raises(RuntimeError, match="outside the vocabulary"):
        eng.forward(bad)
    toks, _, _ = eng.speculative(prompt, NEW, 1)
    assert list(toks) == list(ref.greedy(prompt, NEW))
