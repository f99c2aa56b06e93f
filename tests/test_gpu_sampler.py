"""The device's reference-exact Sampler::select (tqf_hip_sampler_select_device)
against the C oracle's restatement of the reference's draw (orc_softmax_draw:
softmax with f32::exp and the token-order total, the stable descending sort,
the inverse-CDF walk; sampling/mod.rs:166-190, 227-266), bit for bit: the same
token for the same logits, temperature and uniform, and the same two f32 sums
(the token-order total of the exponentials, the sorted-order total of the
probabilities: orc_softmax_draw_sums), which the device computes with its
exact parallel fold.  The uniforms come from the reference's own generator
(Xoshiro256PlusPlus::from_seed, next_f32)."""
import numpy as np
import pytest

import cpu_oracle as orc
from turboqwenfare_amd.sampling import Sampler, Xoshiro256PlusPlus

pytestmark = pytest.mark.gpu

V = 151_936


def logits_for(seed: int, scale: float = 3.0, vocab: int = V) -> np.ndarray:
    return (np.random.default_rng(seed).standard_normal(vocab) * scale).astype(np.float32)


def same_f32(a, b) -> bool:
    a, b = np.float32(a), np.float32(b)
    return (np.isnan(a) and np.isnan(b)) or a.tobytes() == b.tobytes()


def check_draws(backend, lg, T, us, what=None):
    """The device's tokens and sums for rows lg against the oracle's."""
    lg2 = np.atleast_2d(lg)
    toks, sums = backend.sampler_select(lg2, T, list(us), sums=True)
    for r in range(lg2.shape[0]):
        tok, total, psum = orc.softmax_draw_sums(lg2[r], T, float(np.float32(us[r])))
        assert toks[r] == tok, (what, r, toks[r], tok)
        assert same_f32(sums[r, 0], total), (what, r, "total", sums[r, 0], total)
        assert same_f32(sums[r, 1], psum), (what, r, "total2", sums[r, 1], psum)


@pytest.mark.parametrize("seed", range(64))
def test_select_equals_reference_draw(backend, seed):
    """The configuration's shape: V = 151,936, N(0, 9) logits, T = 0.7."""
    lg = logits_for(seed)
    u = Xoshiro256PlusPlus.from_seed(seed).next_f32()
    check_draws(backend, lg, 0.7, [u], seed)


@pytest.mark.parametrize("scale,T", [(1.0, 1.0), (0.1, 1.0), (3.0, 2.0), (3.0, 0.05), (30.0, 0.7)])
def test_select_flat_and_peaked_rows(backend, scale, T):
    """Flat rows fold all 151,936 terms in both sums; peaked ones few."""
    rng = Xoshiro256PlusPlus.from_seed(int(scale * 100 + T * 10))
    for s in range(3):
        lg = logits_for(1000 + s, scale)
        check_draws(backend, lg, T, [rng.next_f32()], (scale, T, s))


@pytest.mark.parametrize("T", [1.0, 0.5])
def test_select_subnormal_exponentials(backend, T):
    """Logits spread over 104 T below the maximum: about one exponential in
    six is subnormal, and the token-order sum climbs through every binade from
    the smallest subnormal's."""
    rng = np.random.default_rng(int(T * 10))
    lg = rng.uniform(-104.0 * T, 0.0, V).astype(np.float32)
    lg[rng.integers(0, V)] = 0.0
    us = Xoshiro256PlusPlus.from_seed(77)
    for _ in range(3):
        check_draws(backend, lg, T, [us.next_f32()], T)


def test_select_rows_side_by_side(backend):
    """Eight rows in one call, each its own row's draw."""
    lg = np.stack([logits_for(2000 + r, 1.0 + r) for r in range(8)])
    rng = Xoshiro256PlusPlus.from_seed(7)
    us = [rng.next_f32() for _ in range(8)]
    check_draws(backend, lg, 0.9, us)


@pytest.mark.parametrize("u", [0.0, 2.0 ** -24, 0.5, 1.0 - 2.0 ** -24])
def test_select_extreme_uniforms(backend, u):
    for seed in (11, 12):
        lg = logits_for(seed, 1.0)
        check_draws(backend, lg, 1.0, [u], (seed, u))


def test_select_ties_nan_and_infinities(backend):
    """Exact ties (equal probabilities: the lower token first), NaN logits (the
    total is NaN: the first sorted token), -inf logits (probability 0), an
    all-NaN row and an all--inf row, +inf (NaN probabilities)."""
    rng = Xoshiro256PlusPlus.from_seed(99)
    rows = []
    base = logits_for(31, 1.0, 4096)
    t = base.copy()
    t[100:140] = 2.5  # 40 equal logits
    rows.append(t)
    t = base.copy()
    t[[5, 900, 3000]] = np.nan
    rows.append(t)
    t = base.copy()
    t[::3] = -np.inf
    rows.append(t)
    rows.append(np.full(4096, np.nan, np.float32))
    rows.append(np.full(4096, -np.inf, np.float32))
    t = base.copy()
    t[77] = np.inf
    rows.append(t)
    t = np.zeros(4096, np.float32)  # a uniform row: every probability equal
    rows.append(t)
    for i, row in enumerate(rows):
        for _ in range(4):
            check_draws(backend, row, 0.8, [rng.next_f32()], i)


@pytest.mark.parametrize("vocab", [1, 2, 63, 64, 65, 4095, 4096, 4097, 70_000])
def test_select_small_and_ragged_vocabularies(backend, vocab):
    rng = Xoshiro256PlusPlus.from_seed(vocab)
    for s in range(3):
        lg = logits_for(vocab * 10 + s, 2.0, vocab)
        check_draws(backend, lg, 0.7, [rng.next_f32()], (vocab, s))


def test_greedy_is_the_argmax(backend):
    """Temperature 0 (Sampler::Greedy) returns top_logit_candidates' token 0."""
    lg = np.stack([logits_for(50 + r) for r in range(4)])
    lg[1, 10:20] = lg[1].max() + 1.0  # ties: the lowest index
    lg[2, :] = np.nan
    lg[2, 500] = 1.0  # NaN never wins
    got = backend.sampler_select(lg, 0.0, [0.0] * 4)
    assert got == [int(orc.top_logit_candidates(lg[r])[0][0]) for r in range(4)]


def test_seeded_sampler_reproduces_the_reference_stream(backend):
    """A seeded Sampler (Xoshiro256PlusPlus::seeded + select) over a sequence
    of logit rows gives the oracle's draws with the oracle's generator."""
    s = Sampler(backend, 0.7, seed=2024)
    ref = orc.Xoshiro(2024)
    d = backend.alloc(4 * V)
    try:
        for step in range(8):
            lg = logits_for(3000 + step)
            backend.write(d, lg)
            want = orc.softmax_draw(lg, 0.7, float(np.float32(ref.next_f32())))
            assert s.select_device(d, V, -1) == want, step
    finally:
        backend.free(d)
        s.free()


def test_bad_arguments_are_rejected(backend):
    from turboqwenfare_amd._lib import HipError

    d = backend.alloc(4 * 16)
    for rows, vocab, T in ((0, 16, 0.7), (9, 16, 0.7), (1, 0, 0.7), (1, 16, -1.0), (1, 16, float("nan")),
                           (1, 16, float("inf"))):
        with pytest.raises(HipError):
            backend.sampler_select_device(d, rows, vocab, T, d, d)
    backend.free(d)
