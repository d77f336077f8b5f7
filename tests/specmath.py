"""The bookkeeping of the reference's speculative state machine
(generator.cc:720-1071), checked from a decode's own outputs: its emitted
tokens, its per-round records and its counters (TEST INFRASTRUCTURE ONLY).

Round record (int32 x 16): [proposal_count k, accepted a, full, correction
(-1 if none), next_target, emitted_before, mtp_len_after, target_len_after,
cand0..cand7].  For every round, with e = emitted_before:
  * next_target is the token emitted at e, and the candidates are the drafts;
  * a is the longest prefix of candidates equal to the tokens emitted after
    next_target, and full = (a == k);
  * full: k + 1 tokens are emitted, the target cache grows by k + 1 and the
    MTP cache by k (the scratch cache keeps every draft row);
  * otherwise the correction is the token emitted at e + a + 1 and differs
    from candidate a; a + 2 tokens are emitted, the target cache grows by
    a + 2 (the replay) and, unless the decode ends there, the MTP cache by
    a + 1 (checkpoint[a] plus the recovery row);
  * counters: proposed = sum k, accepted = sum a, rejected and replay tokens
    over the rejected rounds, one correction per rejected round.
"""
from __future__ import annotations


def check_rounds(tokens, log, stats, prompt_len, max_new, mtp_len0=None):
    """Asserts the relations above; returns the number of rejected rounds."""
    toks = [int(t) for t in tokens]
    mtp_len = prompt_len if mtp_len0 is None else mtp_len0
    tgt_len = prompt_len
    emitted = 0
    recov = 0
    rejected_rounds = 0
    for r in log:
        k, a, full, corr = int(r[0]), int(r[1]), int(r[2]), int(r[3])
        assert int(r[5]) == emitted, ("emitted_before", int(r[5]), emitted)
        assert int(r[4]) == toks[emitted], "next_target is the token emitted first"
        cands = [int(c) for c in r[8:8 + min(k, 8)]]
        want_a = 0
        while want_a < k and want_a < len(cands) and emitted + 1 + want_a < len(toks) \
                and cands[want_a] == toks[emitted + 1 + want_a]:
            want_a += 1
        assert 0 <= a <= k and full == int(a == k)
        if k <= 8 and full == 0:
            assert a == want_a, ("accepted prefix", a, want_a)
        if full:
            assert corr == -1
            emitted += k + 1
            mtp_len += k
            tgt_len += k + 1
        else:
            rejected_rounds += 1
            emitted += a + 1
            if emitted < len(toks):
                assert corr == toks[emitted], "the correction is emitted after the accepted prefix"
                if a < len(cands):
                    assert cands[a] != corr, "the rejected candidate differs from the correction"
                emitted += 1
            tgt_len += a + 2
            if emitted < max_new:
                mtp_len += a + 1
                recov += 1
        assert int(r[6]) == mtp_len, ("mtp_len_after", int(r[6]), mtp_len)
        assert int(r[7]) == tgt_len, ("target_len_after", int(r[7]), tgt_len)
    rej = [r for r in log if int(r[2]) == 0]
    assert stats["rounds"] == len(log)
    assert stats["proposed"] == sum(int(r[0]) for r in log)
    assert stats["accepted"] == sum(int(r[1]) for r in log)
    assert stats["rejected"] == sum(int(r[0]) - int(r[1]) for r in rej)
    assert stats["corrections"] == len(rej)
    assert stats["mtp_recovery_tokens"] == recov
    if "replay_tokens" in stats:
        assert stats["replay_tokens"] == sum(int(r[1]) + 2 for r in rej)
    return rejected_rounds
