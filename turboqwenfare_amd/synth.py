"""Seeded synthetic workloads (host side), byte-identical to the device
generator in ``csrc/tqf_synth.hip``.

No reference counterpart: the reference benchmarks real checkpoints; the
MI355X configurations are defined on synthetic data from a seeded Philox
stream.  Philox4x32-10 follows Salmon, Moraes, Dror & Shaw, "Parallel random
numbers: as easy as 1, 2, 3" (SC'11).
"""
from __future__ import annotations

import numpy as np

_M32 = np.uint64(0xFFFFFFFF)
PHILOX_M0 = 0xD2511F53
PHILOX_M1 = 0xCD9E8D57
PHILOX_W0 = 0x9E3779B9
PHILOX_W1 = 0xBB67AE85
UNIFORM_KEY1 = 0x243F6A88


def philox4x32_10(ctr: np.ndarray, key: tuple[int, int]) -> np.ndarray:
    """Philox4x32-10 of counters ``ctr`` [N, 4] (uint32) under ``key``."""
    c = np.asarray(ctr, dtype=np.uint32).astype(np.uint64)
    c0, c1, c2, c3 = c[:, 0], c[:, 1], c[:, 2], c[:, 3]
    k0, k1 = int(key[0]) & 0xFFFFFFFF, int(key[1]) & 0xFFFFFFFF
    for rnd in range(10):
        if rnd:
            k0 = (k0 + PHILOX_W0) & 0xFFFFFFFF
            k1 = (k1 + PHILOX_W1) & 0xFFFFFFFF
        p0 = np.uint64(PHILOX_M0) * c0
        p1 = np.uint64(PHILOX_M1) * c2
        n0 = (p1 >> np.uint64(32)) ^ c1 ^ np.uint64(k0)
        n2 = (p0 >> np.uint64(32)) ^ c3 ^ np.uint64(k1)
        c0, c1, c2, c3 = n0, p1 & _M32, n2, p0 & _M32
    return np.stack([c0, c1, c2, c3], axis=1).astype(np.uint32)


RECIPE_UNIFORM = 0
RECIPE_ZERO_MEAN = 1
RECIPES = {"uniform": RECIPE_UNIFORM, "zero_mean": RECIPE_ZERO_MEAN}


def zero_mean_nibbles(words: np.ndarray) -> np.ndarray:
    """Every nibble 0 of the uint32 ``words`` becomes 8, so that q - 8 is
    symmetric on [-7, 7] (mean 0) instead of uniform on [-8, 7] (mean -0.5).
    Bit 4j of t is the OR of nibble j's four bits; no bit of another nibble
    reaches it."""
    w = np.asarray(words, dtype=np.uint32)
    t = w | (w >> np.uint32(1))
    t = t | (t >> np.uint32(2))
    z = ~t & np.uint32(0x11111111)
    return w | (z << np.uint32(3))


def q4_0_synthetic(rows: int, cols: int, tensor_id: int, seed: int,
                   recipe: int | str = RECIPE_UNIFORM) -> np.ndarray:
    """GGML Q4_0 bytes [rows * cols/32 * 18] of (tensor_id, seed).

    Block b (row-major): Philox(ctr=(b_lo, b_hi, 0, 0)) gives the 16 nibble
    bytes (little-endian words); Philox(ctr=(b_lo, b_hi, 1, 0)) word 0 gives
    u = (w >> 8) 2^-24 and the scale d = 0.005 + 0.015 u (binary32, no fused
    multiply-add), stored as binary16 rounded to nearest even.

    ``recipe`` "uniform" (0) keeps the nibbles uniform on 0..15, the literal
    configuration text, whose weights carry E[q - 8] = -0.5 and so a common
    rank-one component in every matrix; "zero_mean" (1) maps nibble 0 to 8
    (``zero_mean_nibbles``), still packed Q4_0 with zero-point 8.
    """
    recipe = RECIPES.get(recipe, recipe) if isinstance(recipe, str) else int(recipe)
    if recipe not in (RECIPE_UNIFORM, RECIPE_ZERO_MEAN):
        raise ValueError(f"unknown recipe {recipe}")
    if cols % 32:
        raise ValueError("cols must be a multiple of 32")
    n = rows * (cols // 32)
    idx = np.arange(n, dtype=np.uint64)
    lo = (idx & _M32).astype(np.uint32)
    hi = (idx >> np.uint64(32)).astype(np.uint32)
    zeros = np.zeros(n, dtype=np.uint32)
    q = philox4x32_10(np.stack([lo, hi, zeros, zeros], axis=1), (tensor_id, seed))
    if recipe == RECIPE_ZERO_MEAN:
        q = zero_mean_nibbles(q)
    s = philox4x32_10(np.stack([lo, hi, np.ones(n, dtype=np.uint32), zeros], axis=1),
                      (tensor_id, seed))
    u = (s[:, 0] >> np.uint32(8)).astype(np.float32) * np.float32(2.0 ** -24)
    d = np.float32(0.005) + np.float32(0.015) * u
    d16 = d.astype(np.float16).view(np.uint16)
    out = np.empty((n, 18), dtype=np.uint8)
    out[:, 0:2] = d16.view(np.uint8).reshape(n, 2)
    out[:, 2:18] = q.view(np.uint8).reshape(n, 16)
    return out.reshape(-1)


def philox_uniforms(seed: int, stream: int, count: int) -> np.ndarray:
    """``count`` uniforms in [0, 1) with 24 bits: (word0 >> 8) 2^-24 of
    Philox(ctr=(i, stream, 0, 0), key=(seed, 0x243F6A88))."""
    i = np.arange(count, dtype=np.uint32)
    ctr = np.stack([i, np.full(count, stream, np.uint32), np.zeros(count, np.uint32),
                    np.zeros(count, np.uint32)], axis=1)
    w = philox4x32_10(ctr, (seed, UNIFORM_KEY1))[:, 0]
    return (w >> np.uint32(8)).astype(np.float32) * np.float32(2.0 ** -24)


def normal(shape, seed: int, std: float = 1.0) -> np.ndarray:
    """Seeded N(0, std^2) float32 activations / router weights (host only)."""
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def zipf_routes(tokens: int, n_experts: int = 256, top_k: int = 8, s: float = 1.1,
                seed: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """Skewed prefill routes: per token, top_k distinct experts drawn without
    replacement from a Zipf(s) popularity by Gumbel-top-k (argmax of
    log p_e + Gumbel noise), with weights softmax-renormalised over the chosen
    scores (summing to 1 like RouterResult::from_logits).  Expert ranks are a
    seeded permutation, so the head expert is not expert 0.
    Returns ids [tokens, top_k] u16 (descending score) and w [tokens, top_k] f32."""
    rng = np.random.default_rng(seed)
    rank = rng.permutation(n_experts)
    logp = -s * np.log(rank.astype(np.float64) + 1.0)
    scores = logp[None, :] + rng.gumbel(size=(tokens, n_experts))
    ids = np.argsort(-scores, axis=1, kind="stable")[:, :top_k]
    sel = np.take_along_axis(scores, ids, axis=1)
    p = np.exp(sel - sel[:, :1])
    w = (p / p.sum(axis=1, keepdims=True)).astype(np.float32)
    return ids.astype(np.uint16), w


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (u16), round to nearest even."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (b + np.uint64(0x7FFF) + ((b >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    return r.astype(np.uint16)


def bf16_to_f32(x: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(x, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def pack_q4_k_scales(sc, mn) -> np.ndarray:
    """The 12 packed bytes holding eight 6-bit (scale, min) pairs, the
    inverse of get_scale_min_k4 (dequant.rs:139-148): pairs 0-3 in the low
    six bits of bytes 0-3 / 4-7; pairs 4-7 split into a low nibble (bytes
    8-11) and two high bits (the top bits of bytes 0-3 / 4-7)."""
    sc, mn = np.asarray(sc, np.int64), np.asarray(mn, np.int64)  # [..., 8]
    b = np.zeros(sc.shape[:-1] + (12,), np.int64)
    for j in range(4):
        b[..., j] = sc[..., j] | ((sc[..., j + 4] >> 4) << 6)
        b[..., j + 4] = mn[..., j] | ((mn[..., j + 4] >> 4) << 6)
        b[..., j + 8] = (sc[..., j + 4] & 15) | ((mn[..., j + 4] & 15) << 4)
    return b.astype(np.uint8)


def centered_q4_k(rows: int, cols: int, seed: int, d_range=(1e-4, 4e-4)) -> np.ndarray:
    """Random Q4_K bytes shaped like trained weights: per sub-block min equal
    to its scale and dmin = 7.5 d, so the values d sc (q - 7.5) are centred
    (up to the f16 rounding of dmin) with spread ~d sc."""
    rng = np.random.default_rng(seed)
    n = rows * (cols // 256)
    blk = np.empty((n, 144), np.uint8)
    d = rng.uniform(*d_range, size=n).astype(np.float16)
    blk[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    blk[:, 2:4] = (d.astype(np.float32) * 7.5).astype(np.float16).view(np.uint8).reshape(n, 2)
    sc = rng.integers(1, 64, size=(n, 8))
    blk[:, 4:16] = pack_q4_k_scales(sc, sc)
    blk[:, 16:] = rng.integers(0, 256, size=(n, 128), dtype=np.uint8)
    return blk.reshape(-1)
