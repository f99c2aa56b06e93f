"""The MTP loop's policy and accounting (turboqwenfare_amd/mtp_loop.py) on a
scripted engine: runtime/mtp.rs's own known answers, reached through the
loop rather than by calling MtpStatistics / MtpController directly."""
import pytest

from turboqwenfare_amd import mtp
from turboqwenfare_amd.mtp_loop import MtpLoop


class ScriptedEngine:
    """Accepted lengths from a script; emitted tokens are numbered so that the
    stream can be checked."""

    def __init__(self, accepted, k):
        self.accepted, self.k, self.next_token, self.calls = list(accepted), k, 100, []

    def _tok(self):
        self.next_token += 1
        return self.next_token

    def start(self, token):
        self.calls.append(("start", token))
        return self._tok(), {}

    def plain(self, step, boundary):
        self.calls.append(("plain", step, boundary))
        return self._tok(), {}

    def speculative(self, step, boundary):
        self.calls.append(("spec", step, boundary))
        a = self.accepted.pop(0)
        assert 0 <= a <= self.k
        return [self._tok() for _ in range(a + 1)], a, {}


def test_statistics_known_answer_through_the_loop():
    """mtp.rs statistics_track_acceptance_rate_and_emitted_per_pass: pair
    verifications accepted, rejected, accepted -> 3 drafted, 2 accepted,
    5 emitted over 3 target passes (k = 1 is verify_pair)."""
    loop = MtpLoop(ScriptedEngine([1, 0, 1], k=1), k=1, window=8)
    loop.run(5, 3)
    st = loop.stats
    assert (st.drafted_tokens, st.accepted_tokens, st.emitted_tokens,
            st.target_backbone_passes) == (3, 2, 5, 3)
    assert abs(st.acceptance_rate() - 2 / 3) < 1e-9
    assert abs(st.emitted_tokens_per_target_pass() - 5 / 3) < 1e-9


def test_controller_enables_after_a_full_positive_window():
    """mtp.rs controller_enables_only_after_a_sustained_positive_rolling_benefit
    (window 4, emitted 2 per pass): off until the window fills, then on, and
    speculation continues."""
    loop = MtpLoop(ScriptedEngine([1] * 10, k=1), k=1, window=4)
    recs = loop.run(0, 6)
    assert [r.enabled for r in recs[1:]] == [False, False, False, True, True, True]
    assert all(r.speculative for r in recs[1:])


def test_warm_up_without_benefit_leaves_speculation_off():
    """Every draft rejected: net benefit 0 over the full window is not above
    +0.10, so the controller stays off and later steps decode one token
    without drafts, feeding nothing more to the statistics."""
    k = 3
    eng = ScriptedEngine([0] * 4, k=k)
    loop = MtpLoop(eng, k=k, window=4)
    recs = loop.run(7, 9)
    assert [r.speculative for r in recs[1:]] == [True] * 4 + [False] * 5
    assert all(not r.enabled for r in recs)
    assert loop.stats.target_backbone_passes == 4 and loop.stats.drafted_tokens == 4 * k
    assert [c[0] for c in eng.calls] == ["start"] + ["spec"] * 4 + ["plain"] * 5


def test_token_stream_and_boundaries():
    """Each pass starts from the last emitted token; a k-draft pass emits
    accepted + 1 tokens."""
    k = 3
    eng = ScriptedEngine([3, 0, 2, 1], k=k)
    loop = MtpLoop(eng, k=k, window=8)
    recs = loop.run(42, 4)
    stream = [t for r in recs for t in r.emitted]
    assert stream == list(range(101, 101 + len(stream)))
    assert [len(r.emitted) for r in recs] == [1, 4, 1, 3, 2]
    boundaries = [c[2] for c in eng.calls[1:]]
    ends = [r.emitted[-1] for r in recs[:-1]]
    assert boundaries == ends
    st = loop.stats
    assert (st.drafted_tokens, st.accepted_tokens, st.emitted_tokens) == (12, 6, 10)


def test_disable_needs_outcomes_below_the_baseline():
    """mtp.rs controller_disables_after_a_sustained_negative_rolling_benefit
    feeds emitted 0; a verify pass emits at least one token, so only such
    outcomes switch an enabled controller off."""
    c = mtp.MtpController(4)
    for _ in range(4):
        c.record_and_decide(2)
    assert c.enabled
    for a in range(4):  # any accepted length keeps it on
        c.record_and_decide(a + 1)
    assert c.enabled
    for _ in range(4):
        c.record_and_decide(0)
    assert not c.enabled


def test_loop_rejects_bad_k_and_steps_before_start():
    with pytest.raises(ValueError):
        MtpLoop(ScriptedEngine([], k=1), k=0)
    loop = MtpLoop(ScriptedEngine([], k=1), k=1)
    with pytest.raises(RuntimeError):
        loop.step()
