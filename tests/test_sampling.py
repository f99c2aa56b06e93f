"""turboqwenfare_amd.sampling (host side of Sampler, CPU):
- Xoshiro256PlusPlus against the reference's known answer
  (sampling/mod.rs:662-669: state [1, 1, 1, 1] -> 16,777,217, then a
  different value) and its unit-interval and mixing tests (:672-692);
- the same streams as the C oracle's generator (orc_xoshiro_*, pinned by the
  same known answer) over several seeds, including the SplitMix64 seeding;
- next_f32 is exactly (next_u64 >> 40) / 2^24."""
import numpy as np
import pytest

import cpu_oracle as orc
from turboqwenfare_amd.sampling import Sampler, Xoshiro256PlusPlus


def test_xoshiro_known_answer():
    rng = Xoshiro256PlusPlus([1, 1, 1, 1])
    assert rng.next_u64() == 16_777_217
    assert rng.next_u64() != 16_777_217


def test_next_f32_in_unit_interval_and_exact():
    rng = Xoshiro256PlusPlus.from_seed(12345)
    twin = Xoshiro256PlusPlus.from_seed(12345)
    for _ in range(20000):
        v = rng.next_f32()
        assert 0.0 <= v < 1.0
        assert v == np.float32((twin.next_u64() >> 40) * 2.0 ** -24)


def test_seeding_from_zero_is_well_mixed():
    rng = Xoshiro256PlusPlus.from_seed(0)
    first = [rng.next_u64() for _ in range(8)]
    assert all(v != 0 for v in first) and len(set(first)) == 8


@pytest.mark.parametrize("seed", [0, 1, 42, 2**63 + 5, 2**64 - 1])
def test_streams_equal_the_oracle(seed):
    mine = Xoshiro256PlusPlus.from_seed(seed)
    ref = orc.Xoshiro(seed)
    for _ in range(1000):
        assert mine.next_u64() == ref.next_u64()
    for _ in range(1000):
        assert mine.next_f32() == np.float32(ref.next_f32())


def test_greedy_sampler_returns_the_callers_token():
    s = Sampler(None, 0.0)
    assert s.is_greedy() and s.select_device(None, 10, 7) == 7
