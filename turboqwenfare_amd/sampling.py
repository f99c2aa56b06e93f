"""Token selection as the reference's ``Sampler`` does it
(``src/sampling/mod.rs:31-74``), on the HIP backend.

- ``Xoshiro256PlusPlus`` restates the reference's generator
  (``sampling/mod.rs:274-331``): SplitMix64 seeding of the four state words,
  ``next_u64`` (xoshiro256++), and ``next_f32`` = the top 24 bits / 2^24. It
  is host code, as in the reference, where the generator lives in the
  sampler object that the decode loop owns.
- ``Sampler`` mirrors ``Sampler::new`` / ``Sampler::select``: temperature 0
  is the greedy identity (the caller's argmax, returned verbatim); otherwise
  each ``select`` draws one ``next_f32`` and runs the device's
  reference-exact stochastic path (``tqf_hip_sampler_select_device``:
  softmax with f32::exp and the token-order f32 total, the stable descending
  sort, the inverse-CDF walk). With the default filters (no penalties,
  top_k, top_p or min_p) a seeded ``Sampler`` over the same logits returns
  the reference's token stream.
"""
from __future__ import annotations

import time

import numpy as np

_MASK = (1 << 64) - 1


def _rotl(x: int, k: int) -> int:
    return ((x << k) | (x >> (64 - k))) & _MASK


class Xoshiro256PlusPlus:
    """xoshiro256++ with SplitMix64 seeding (sampling/mod.rs:274-331)."""

    def __init__(self, state):
        if len(state) != 4:
            raise ValueError("four state words")
        self.state = [int(s) & _MASK for s in state]

    @classmethod
    def from_seed(cls, seed: int) -> "Xoshiro256PlusPlus":
        """Xoshiro256PlusPlus::from_seed (:283-298): four SplitMix64 outputs."""
        z = int(seed) & _MASK
        words = []
        for _ in range(4):
            z = (z + 0x9E3779B97F4A7C15) & _MASK
            x = z
            x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & _MASK
            x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & _MASK
            words.append(x ^ (x >> 31))
        return cls(words)

    @classmethod
    def seeded(cls, seed: int | None) -> "Xoshiro256PlusPlus":
        """Xoshiro256PlusPlus::seeded (:302-309): the seed, or the wall clock
        in nanoseconds when there is none."""
        return cls.from_seed(seed if seed is not None else time.time_ns() & _MASK)

    def next_u64(self) -> int:
        """:311-326."""
        s = self.state
        result = (_rotl((s[0] + s[3]) & _MASK, 23) + s[0]) & _MASK
        t = (s[1] << 17) & _MASK
        s[2] ^= s[0]
        s[3] ^= s[1]
        s[1] ^= s[2]
        s[0] ^= s[3]
        s[2] ^= t
        s[3] = _rotl(s[3], 45)
        return result

    def next_f32(self) -> np.float32:
        """:328-330: (next_u64 >> 40) / 2^24, exact in binary32, in [0, 1)."""
        return np.float32((self.next_u64() >> 40) / float(1 << 24))


class Sampler:
    """Sampler::new / Sampler::select (sampling/mod.rs:31-74) with the
    stochastic draw on the device.

    ``temperature == 0.0`` (an exact comparison, as ``Sampler::new`` makes
    it) selects greedy, which returns ``greedy_token`` untouched."""

    def __init__(self, be, temperature: float, seed: int | None = None):
        self.be = be
        self.temperature = float(temperature)
        self.greedy = self.temperature == 0.0
        self.rng = None if self.greedy else Xoshiro256PlusPlus.seeded(seed)
        self._d_u = None if self.greedy else be.alloc(4)
        self._d_tok = None if self.greedy else be.alloc(4)

    def is_greedy(self) -> bool:
        return self.greedy

    def select_device(self, d_logits, vocab: int, greedy_token: int) -> int:
        """One token from a device row of `vocab` logits (Sampler::select)."""
        if self.greedy:
            return int(greedy_token)
        u = self.rng.next_f32()
        self.be.write(self._d_u, np.array([u], np.float32))
        self.be.sampler_select_device(d_logits, 1, vocab, self.temperature, self._d_u, self._d_tok)
        return int(self.be.read(self._d_tok, np.int32, (1,))[0])

    def free(self) -> None:
        for b in (self._d_u, self._d_tok):
            if b is not None:
                self.be.free(b)
        self._d_u = self._d_tok = None
