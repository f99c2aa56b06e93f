"""GPU acceptance sampling (a22) against the CPU definition: accepted length
and token ids must be bit-exact for identical logits and uniforms."""
import numpy as np
import pytest

import cpu_oracle as orc
from turboqwenfare_amd import mtp, synth
from turboqwenfare_amd import _lib
from turboqwenfare_amd._lib import ERR_INVALID, HipError

pytestmark = pytest.mark.gpu

V = 151936


def case(seed: int, k: int = 3, vocab: int = V, noise: float = 1.0):
    """Target = draft + noise: small noise -> mostly accepted, large -> rejected.
    Draft tokens are drawn from the draft softmax at T = 0.7 (as a real
    drafter would) with the reference's own inverse-CDF draw."""
    rng = np.random.default_rng(seed)
    draft = (rng.standard_normal((k, vocab)) * 3).astype(np.float32)
    target = np.empty((k + 1, vocab), np.float32)
    target[:k] = draft + (rng.standard_normal((k, vocab)) * noise).astype(np.float32)
    target[k] = (rng.standard_normal(vocab) * 3).astype(np.float32)
    ud = synth.philox_uniforms(seed, 7, k)
    dtok = np.array([orc.softmax_draw(draft[i], 0.7, float(ud[i])) for i in range(k)], np.int32)
    u = synth.philox_uniforms(seed, 0, k)
    ur = synth.philox_uniforms(seed, 1, k + 1)
    return target, draft, dtok, u, ur


@pytest.mark.parametrize("noise", [0.05, 0.5, 3.0])
def test_stochastic_bit_exact_over_seeds(backend, noise):
    accepted = []
    for seed in range(0, 64, 4):
        target, draft, dtok, u, ur = case(seed, noise=noise)
        got = backend.accept(target, draft, dtok, 0.7, False, u, ur)
        want = orc.accept(target, draft, dtok, 0.7, False, u, ur)
        assert got == want, f"seed {seed}"
        accepted.append(got[0])
    print(f"noise {noise}: accepted lengths {accepted}")


def test_stochastic_exercises_every_accepted_length(backend):
    seen = set()
    for seed in range(64):
        target, draft, dtok, u, ur = case(seed, vocab=4096, noise=0.6)
        got = backend.accept(target, draft, dtok, 0.7, False, u, ur)
        assert got == orc.accept(target, draft, dtok, 0.7, False, u, ur), f"seed {seed}"
        seen.add(got[0])
    assert seen == {0, 1, 2, 3}


@pytest.mark.parametrize("seed", range(16))
def test_greedy_bit_exact(backend, seed):
    target, draft, dtok, _, _ = case(seed, noise=0.3)
    # make some drafts match the target argmax
    for i in range(3):
        if (seed >> i) & 1:
            dtok[i] = int(np.argmax(target[i]))
    got = backend.accept(target, None, dtok, 0.0, True)
    want = orc.accept(target, None, dtok, 0.0, True)
    assert got == want


def test_greedy_k1_is_verify_pair(backend):
    rng = np.random.default_rng(1)
    for seed in range(8):
        target = (rng.standard_normal((2, 1000)) * 3).astype(np.float32)
        a0 = int(np.argmax(target[0]))
        for d in (a0, (a0 + 1) % 1000):
            acc, toks = backend.accept(target, None, [d], 0.0, True)
            out = mtp.verify_pair(a0, d)
            assert out.accepted == (acc == 1)
            assert out.emitted_tokens == len(toks)
            assert toks[0] == a0


@pytest.mark.parametrize("k", [0, 1, 2, 5, 7])
def test_other_draft_lengths(backend, k):
    for seed in range(4):
        target, draft, dtok, u, ur = case(100 + seed, k=k, vocab=20000, noise=0.4)
        for greedy in (False, True):
            got = backend.accept(target, draft, dtok, 0.7, greedy, u, ur)
            assert got == orc.accept(target, draft, dtok, 0.7, greedy, u, ur)


def test_identical_distributions_always_accept(backend):
    rng = np.random.default_rng(3)
    draft = (rng.standard_normal((3, 5000)) * 3).astype(np.float32)
    target = np.concatenate([draft, draft[:1]])
    dtok = [17, 99, 4000]
    u = np.array([0.999999, 0.5, 0.0], np.float32)
    ur = synth.philox_uniforms(3, 1, 4)
    got = backend.accept(target, draft, dtok, 0.9, False, u, ur)
    assert got[0] == 3
    assert got == orc.accept(target, draft, dtok, 0.9, False, u, ur)


def test_zero_target_probability_always_rejects(backend):
    draft = np.zeros((1, 64), np.float32)
    target = np.zeros((2, 64), np.float32)
    target[0, 5] = -np.inf  # p(d) = 0 < q(d)
    got = backend.accept(target, draft, [5], 0.7, False, np.array([0.0], np.float32),
                         np.array([0.3, 0.3], np.float32))
    assert got[0] == 0 and got[1][0] != 5
    assert got == orc.accept(target, draft, [5], 0.7, False, np.array([0.0], np.float32),
                             np.array([0.3, 0.3], np.float32))


def test_one_hot_target_accepts(backend):
    rng = np.random.default_rng(4)
    draft = (rng.standard_normal((2, 3000)) * 3).astype(np.float32)
    target = np.full((3, 3000), -1e4, np.float32)
    target[0, 42] = 10.0
    target[1, 7] = 10.0
    target[2, 2999] = 10.0
    u = np.array([0.99, 0.99], np.float32)
    ur = np.array([0.5, 0.5, 0.5], np.float32)
    got = backend.accept(target, draft, [42, 7], 0.7, False, u, ur)
    assert got == (2, [42, 7, 2999])
    assert got == orc.accept(target, draft, [42, 7], 0.7, False, u, ur)


def test_nan_and_inf_logits(backend):
    rng = np.random.default_rng(5)
    target = (rng.standard_normal((4, 9000)) * 3).astype(np.float32)
    draft = (rng.standard_normal((3, 9000)) * 3).astype(np.float32)
    target[0, ::7] = np.nan
    draft[1, ::5] = np.nan
    target[2, 100] = np.inf
    draft[2, :] = -np.inf
    target[3, :] = np.nan
    dtok = [int(np.nanargmax(target[0])), 3, 100]
    u = np.array([0.2, 0.4, 0.6], np.float32)
    ur = np.array([0.1, 0.9, 0.5, 0.7], np.float32)
    for greedy in (False, True):
        got = backend.accept(target, draft, dtok, 0.7, greedy, u, ur)
        assert got == orc.accept(target, draft, dtok, 0.7, greedy, u, ur)


def test_ties_and_tiny_vocab(backend):
    for vocab in (1, 2, 3, 4097):
        target = np.zeros((3, vocab), np.float32)
        draft = np.zeros((2, vocab), np.float32)
        dtok = [0, vocab - 1]
        u = np.array([0.0, 0.75], np.float32)
        ur = np.array([0.999, 0.0, 0.5], np.float32)
        for greedy in (False, True):
            got = backend.accept(target, draft, dtok, 0.7, greedy, u, ur)
            assert got == orc.accept(target, draft, dtok, 0.7, greedy, u, ur), vocab


def test_rejects_invalid_arguments(backend):
    t = np.zeros((2, 10), np.float32)
    with pytest.raises(HipError) as e:
        backend.accept(t, t[:1], [10], 0.7, False, np.zeros(1, np.float32), np.zeros(2, np.float32))
    assert e.value.status == ERR_INVALID
    with pytest.raises(HipError):
        backend.accept(t, t[:1], [1], 0.7, False, np.ones(1, np.float32), np.zeros(2, np.float32))
    with pytest.raises(HipError):
        backend.accept(t, t[:1], [1], 0.0, False, np.zeros(1, np.float32), np.zeros(2, np.float32))


def test_device_entry_point_matches_host(backend):
    target, draft, dtok, u, ur = case(9)
    bufs = [backend.to_device(a) for a in (target, draft, dtok, u, ur)]
    acc = backend.alloc(4)
    toks = backend.alloc(16)
    for rep in range(2):
        backend.accept_device(bufs[0], bufs[1], bufs[2], 3, V, 0.7, False, bufs[3], bufs[4], acc,
                              toks)
        a = int(backend.read(acc, np.int32, (1,))[0])
        tk = [int(v) for v in backend.read(toks, np.int32, (4,))[: a + 1]]
        assert (a, tk) == orc.accept(target, draft, dtok, 0.7, False, u, ur)
    for b in bufs + [acc, toks]:
        backend.free(b)


@pytest.mark.parametrize("greedy", [False, True])
def test_poll_timeout_reports_failure_and_recovers(backend, monkeypatch, greedy):
    """An exchange that times out makes the one-launch acceptance write
    accepted = -1, and every workgroup still leaves (stochastic: the others
    time out on the first one's missing sums within 20 ms; greedy: only
    workgroup 0 gathers); the next call is bit-exact again.  The timeout is
    forced from the host (workgroup 0 takes its first exchange, or the greedy
    arg-max gather, as timed out), so the kernel exits normally."""
    target, draft, dtok, u, ur = case(17)
    bufs = [backend.to_device(a) for a in (target, draft, dtok, u, ur)]
    acc = backend.alloc(4)
    toks = backend.alloc(16)
    want = orc.accept(target, draft, dtok, 0.7, greedy, u, ur)

    def run():
        backend.accept_device(bufs[0], bufs[1], bufs[2], 3, V, 0.7, greedy, bufs[3], bufs[4], acc,
                              toks)
        a = int(backend.read(acc, np.int32, (1,))[0])
        return a, [int(v) for v in backend.read(toks, np.int32, (4,))[: a + 1]]

    with backend.variant(_lib.VARIANT_RECOVER, False):
        assert run() == want
        monkeypatch.setenv("TQF_HIP_ACCEPT_FAIL_POLL", "1")
        assert run()[0] == -1
        monkeypatch.delenv("TQF_HIP_ACCEPT_FAIL_POLL")
        for _ in range(2):
            assert run() == want
    # with recovery (the default) the timed-out launch is re-run through the
    # three-kernel path: the same bits, one re-run counted
    before = backend.recovery_counts()
    monkeypatch.setenv("TQF_HIP_ACCEPT_FAIL_POLL", "1")
    assert run() == want
    monkeypatch.delenv("TQF_HIP_ACCEPT_FAIL_POLL")
    assert backend.recovery_counts() == (before[0], before[1] + 1)
    assert run() == want and backend.recovery_counts() == (before[0], before[1] + 1)
    for b in bufs + [acc, toks]:
        backend.free(b)


def test_matches_committed_golden(backend):
    """The committed oracle outcomes (tests/golden/oracle_vectors.npz) for
    seeds 0..63, greedy and stochastic, at V = 1000, k = 3."""
    import sys
    from pathlib import Path

    golden = Path(__file__).resolve().parent / "golden"
    sys.path.insert(0, str(golden))
    from golden_inputs import accept_inputs

    g = np.load(golden / "oracle_vectors.npz")
    for gi, greedy in enumerate((True, False)):
        for seed in range(64):
            target, draft, dtok, u, ur = accept_inputs(seed)
            a, toks = backend.accept(target, draft, dtok, 0.7, greedy, u, ur)
            assert a == g["accept_len"][gi, seed], (greedy, seed)
            assert toks == list(g["accept_tokens"][gi, seed, : a + 1]), (greedy, seed)


def test_launch_paths_alternate_on_one_context(backend):
    """Calls that take the one-launch kernel (every chunk's workgroup resident
    at once) and calls whose vocab is beyond its grid (the three-kernel path)
    interleave on one context and its scratch, each equal to the oracle."""
    for k, vocab, seed in ((3, V, 21), (1, 1_100_000, 22), (3, V, 23), (7, 600_000, 24),
                           (7, 20_000, 25), (0, 1_100_000, 26), (3, 600_000, 27), (3, V, 21)):
        target, draft, dtok, u, ur = case(seed, k=k, vocab=vocab, noise=0.5)
        for greedy in (False, True):
            got = backend.accept(target, draft, dtok, 0.7, greedy, u, ur)
            assert got == orc.accept(target, draft, dtok, 0.7, greedy, u, ur), (k, vocab, greedy)


@pytest.mark.parametrize("vocab", [3000, 150_000])
def test_rejection_without_residual_mass(backend, vocab):
    """A rejected pair whose residual max(0, p - q) is zero everywhere (target
    row = draft row, the draft token impossible under both): the replacement
    is drawn from the target row itself; with no mass in that row either
    (every logit NaN), it is the row's arg-max (token 0 without candidates)."""
    rng = np.random.default_rng(31)
    k = 2
    draft = (rng.standard_normal((k, vocab)) * 3).astype(np.float32)
    target = np.concatenate([draft, (rng.standard_normal((1, vocab)) * 3).astype(np.float32)])
    bad = vocab // 2 + 7
    target[0, bad] = draft[0, bad] = -np.inf
    u = np.array([0.3, 0.3], np.float32)
    for ur0 in (0.0, 0.37, 0.999):
        ur = np.array([ur0, 0.5, 0.5], np.float32)
        got = backend.accept(target, draft, [bad, 1], 0.7, False, u, ur)
        assert got[0] == 0
        assert got == orc.accept(target, draft, [bad, 1], 0.7, False, u, ur), ur0
    target[0, :] = np.nan
    draft[0, :] = np.nan
    ur = np.array([0.6, 0.5, 0.5], np.float32)
    got = backend.accept(target, draft, [bad, 1], 0.7, False, u, ur)
    assert got == (0, [0]) == orc.accept(target, draft, [bad, 1], 0.7, False, u, ur)


@pytest.mark.parametrize("T", [2.0 ** -31, 2.0 ** -29, 0.01, 0.1, 0.37, 0.7, 1.0, 1.7, 3.3, 100.0,
                               2.0 ** 29, 2.0 ** 31])
def test_temperatures_across_the_division_paths(backend, T):
    """Temperatures inside [2^-30, 2^30] take the launch-wide reciprocal form
    of (l - M) / T, the others the per-element division; every one must match
    the oracle's IEEE division bit for bit."""
    for seed in range(3):
        target, draft, dtok, u, ur = case(200 + seed, k=3, vocab=20000, noise=0.5)
        scale = np.float32(min(max(T, 1e-3), 1e3))  # logit spreads comparable to T
        target = (target * scale).astype(np.float32)
        draft = (draft * scale).astype(np.float32)
        got = backend.accept(target, draft, dtok, T, False, u, ur)
        assert got == orc.accept(target, draft, dtok, T, False, u, ur), (T, seed)


def _softmax64(row, T):
    z = np.exp((row.astype(np.float64) - row.max()) / T)
    return z / z.sum()


def test_draw_frequencies_follow_p(backend):
    """The acceptance's own draw (k = 0: the bonus token, and the MTP loop's
    stochastic selection), whose definition departs from Sampler::select's
    sorted running-sum draw (sampling/mod.rs:166-190, 227-248): its
    frequencies over 20,000 uniforms follow p = softmax(l / T) (chi-square,
    5 degrees of freedom)."""
    V, T, n = 6, 0.7, 20_000
    target = np.array([[2.0, 1.0, 0.5, 0.0, -1.0, 1.5]], np.float32)
    p = _softmax64(target[0], T)
    ur = synth.philox_uniforms(77, 1, n)
    counts = np.zeros(V)
    empty = np.zeros((0, V), np.float32)
    for i in range(n):
        a, toks = backend.accept(target, empty, [], T, False, np.zeros(0, np.float32),
                                 ur[i:i + 1])
        counts[toks[0]] += 1
    chi2 = float(np.sum((counts - n * p) ** 2 / (n * p)))
    print(f"draw chi2 {chi2:.2f}, counts {counts.astype(int).tolist()}")
    assert chi2 < 25.0  # P(chi2 > 25) ~ 1e-4 at 5 degrees of freedom


def test_speculative_emission_follows_p(backend):
    """With d ~ q, the first emitted token is distributed as p: the
    speculative-sampling identity, on the device path."""
    V, T, n = 6, 0.7, 20_000
    target = np.array([[2.0, 1.0, 0.5, 0.0, -1.0, 1.5], [0, 0, 0, 0, 0, 0]], np.float32)
    draft = np.array([[0.0, 2.0, 1.0, 0.5, 0.0, -2.0]], np.float32)
    p, q = _softmax64(target[0], T), _softmax64(draft[0], T)
    uq = synth.philox_uniforms(78, 2, n)
    u = synth.philox_uniforms(78, 0, n)
    ur = synth.philox_uniforms(78, 1, 2 * n)
    cq = np.cumsum(q)
    counts = np.zeros(V)
    for i in range(n):
        d = int(min(np.searchsorted(cq, float(uq[i]), side="right"), V - 1))
        _, toks = backend.accept(target, draft, [d], T, False, u[i:i + 1], ur[2 * i:2 * i + 2])
        counts[toks[0]] += 1
    chi2 = float(np.sum((counts - n * p) ** 2 / (n * p)))
    print(f"speculative chi2 {chi2:.2f}, counts {counts.astype(int).tolist()}")
    assert chi2 < 25.0
