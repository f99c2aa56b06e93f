"""CPU tests that pin the oracle (oracle/tqf_oracle.c) to something other than
itself: the reference crate's own known-answer tests (file:line cited on each),
library routines (numpy's IEEE binary16 conversion, float64 arithmetic),
closed forms and invariants, and statistical checks.  A plausible mistake in
the restatement (a dropped term, a wrong sign or index, a transposed operand,
the wrong tie order) fails at least one of them."""
from __future__ import annotations

import math
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

import cpu_oracle as orc
from turboqwenfare_amd import mtp, synth
from turboqwenfare_amd.synth import centered_q4_k, pack_q4_k_scales

GOLDEN = Path(__file__).resolve().parent / "golden"


def q4_block(scale_bits: int, qs: bytes) -> np.ndarray:
    return np.frombuffer(scale_bits.to_bytes(2, "little") + qs, dtype=np.uint8)


def np_dequant(w: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Independent numpy decode of GGML Q4_0 (library f16 conversion)."""
    b = w.reshape(rows, cols // 32, 18)
    d = b[:, :, 0:2].copy().view(np.float16).astype(np.float64)  # [rows, B, 1]
    qs = b[:, :, 2:].astype(np.int64)
    lo = (qs & 15) - 8
    hi = (qs >> 4) - 8
    vals = np.concatenate([lo, hi], axis=2).astype(np.float64) * d
    return vals.reshape(rows, cols)


# ---- a1: f16 ----------------------------------------------------------------
def test_f16_known_values():
    # dequant.rs:243-251
    assert orc.f16_to_f32(0x3C00) == 1.0
    assert orc.f16_to_f32(0x4000) == 2.0
    assert orc.f16_to_f32(0x0000) == 0.0
    assert orc.f16_to_f32(0xBC00) == -1.0


def test_f16_exhaustive_against_numpy_and_the_independent_decoder():
    # every binary16 pattern: numpy's conversion is a library routine, the
    # independent decoder restates validate.rs:48-69 (arithmetic, not bits)
    want = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    for bits in range(65536):
        a = orc.f16_to_f32(bits)
        b = orc.f16_to_f32_indep(bits)
        w = want[bits]
        if np.isnan(w):
            assert math.isnan(a) and math.isnan(b), hex(bits)
        else:
            assert np.float32(a).view(np.uint32) == w.view(np.uint32), hex(bits)
            assert np.float32(b).view(np.uint32) == w.view(np.uint32), hex(bits)


def test_f16_round_trip_set_and_rounding_against_numpy():
    # dequant.rs:279-284
    for bits in (0x0000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0xC100, 0x7C00):
        assert orc.f32_to_f16(orc.f16_to_f32(bits)) == bits
    assert math.isnan(orc.f16_to_f32(orc.f32_to_f16(float("nan"))))
    rng = np.random.default_rng(1)
    vals = np.concatenate([rng.standard_normal(4000).astype(np.float32) * 10,
                           rng.uniform(0.005, 0.02, 4000).astype(np.float32),
                           np.float32([6e-8, 3e-5, 65504, 65520, 1e6, -1e-9])])
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    got = np.array([orc.f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, want)


# ---- a2: Q4_0 block decode -----------------------------------------------------
def test_dequantize_q4_0_known_block():
    # dequant.rs:253-264: qs[0] = 0x18 -> low 8 (0.0), high 1 (-7.0), rest -8.0
    block = q4_block(0x3C00, bytes([0x18]) + bytes(15))
    out = orc.dequantize_q4_0(block)
    assert out[0] == 0.0 and out[16] == -7.0 and out[1] == -8.0 and out[17] == -8.0


def test_dequantize_i37_pattern_agrees_with_independent_and_numpy():
    # validate.rs:270-283: byte i = i*37 + 11 (mod 256)
    block = np.array([(i * 37 + 11) & 0xFF for i in range(18)], dtype=np.uint8)
    a = orc.dequantize_q4_0(block)
    b = orc.dequantize_q4_0(block, independent=True)
    assert np.array_equal(a, b)
    assert np.array_equal(a.astype(np.float64), np_dequant(block, 1, 32)[0])


def test_dequantize_matches_numpy_on_random_blocks():
    rng = np.random.default_rng(2)
    for _ in range(200):
        block = rng.integers(0, 256, 18, dtype=np.uint8)
        block[1] &= 0x7B  # finite scales
        assert np.array_equal(orc.dequantize_q4_0(block).astype(np.float64),
                              np_dequant(block, 1, 32)[0])


# ---- a3: GEMV ----------------------------------------------------------------
def test_matvec_canonical_q4_zero_block_kat():
    # weights.rs:2500-2508: scale 1.0, nibbles 15 -> 7 x 32 ones = 224
    w = q4_block(0x3C00, b"\xff" * 16)
    assert orc.q4_0_matvec(w, 1, 32, np.ones(32, np.float32))[0] == 224.0


def test_matvec_rows_and_expert_planes_kat():
    # weights.rs:2458-2480 (row decode 7.0 x 32 / 0.0 x 32) and 2511-2530
    # (expert plane 0 -> 224, plane 1 -> 0)
    first = q4_block(0x3C00, b"\xff" * 16)
    second = np.zeros(18, np.uint8)
    assert np.array_equal(orc.dequantize_q4_0(first), np.full(32, 7.0, np.float32))
    assert np.all(orc.dequantize_q4_0(second) == 0.0)
    w = np.concatenate([first, second])
    assert list(orc.q4_0_matvec(w, 2, 32, np.ones(32, np.float32))) == [224.0, 0.0]


def test_matvec_rejects_bad_shapes():
    with pytest.raises(ValueError):
        orc.q4_0_matvec(np.zeros(18, np.uint8), 1, 48, np.ones(48, np.float32))
    with pytest.raises(ValueError):
        orc.q4_0_matvec(np.zeros(17, np.uint8), 1, 32, np.ones(32, np.float32))


def test_matvec_one_hot_probe_recovers_columns():
    # kernels.rs:1168-1196 technique: x = e_j returns column j exactly
    rows, cols = 16, 96
    w = synth.q4_0_synthetic(rows, cols, 77, 1)
    dense = np_dequant(w, rows, cols)
    for j in range(cols):
        x = np.zeros(cols, np.float32)
        x[j] = 1.0
        assert np.array_equal(orc.q4_0_matvec(w, rows, cols, x).astype(np.float64), dense[:, j])


def test_matvec_all_ff_closed_form():
    # an all-0xFF nibble row gives 7 d sum(x) per block
    rng = np.random.default_rng(3)
    x = rng.standard_normal(64).astype(np.float32)
    w = np.concatenate([q4_block(0x2E66, b"\xff" * 16), q4_block(0x3800, b"\xff" * 16)])
    d0, d1 = np.float16(np.uint16(0x2E66).view(np.float16)), 0.5
    want = 7 * float(d0) * float(np.sum(x[:32], dtype=np.float64)) + 7 * d1 * float(
        np.sum(x[32:], dtype=np.float64))
    assert abs(orc.q4_0_matvec(w, 1, 64, x)[0] - want) < 1e-5 * max(1.0, abs(want))


@pytest.mark.parametrize("rows,cols", [(1, 32), (7, 96), (33, 512), (64, 2048)])
def test_matvec_against_float64_brute_force(rows, cols):
    w = synth.q4_0_synthetic(rows, cols, rows + cols, 2)
    x = np.random.default_rng(rows).standard_normal(cols).astype(np.float32)
    want = np_dequant(w, rows, cols) @ x.astype(np.float64)
    got = orc.q4_0_matvec(w, rows, cols, x)
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1.0)) < 1e-5


def test_f32_matvec_against_float64():
    rng = np.random.default_rng(4)
    w = rng.standard_normal((9, 300)).astype(np.float32)
    x = rng.standard_normal(300).astype(np.float32)
    assert np.allclose(orc.f32_matvec(w, x), w.astype(np.float64) @ x, rtol=1e-5, atol=1e-5)


# ---- a6: router ----------------------------------------------------------------
def test_router_stable_renormalised_kat():
    # experts/mod.rs:1639-1650
    logits = np.full(256, -10.0, np.float32)
    logits[21] = 4.0
    logits[3] = 4.0
    logits[8] = 3.0
    ids, w = orc.router_from_logits(logits)
    assert ids[0] == 3 and ids[1] == 21
    assert abs(float(np.sum(w, dtype=np.float32)) - 1.0) < 1e-6
    assert w[0] > w[2]


def test_router_rejects_wrong_length_nan_and_duplicates():
    # experts/mod.rs:1652-1673
    with pytest.raises(ValueError):
        orc.router_from_logits(np.zeros(255, np.float32))
    bad = np.zeros(256, np.float32)
    bad[7] = np.nan
    with pytest.raises(ValueError):
        orc.router_from_logits(bad)
    assert not orc.router_validate(np.full(8, 3, np.uint16), np.full(8, 0.125, np.float32))
    assert orc.router_validate(np.arange(8, dtype=np.uint16), np.full(8, 0.125, np.float32))


def test_router_matches_float64_softmax_and_stable_order():
    rng = np.random.default_rng(5)
    for trial in range(50):
        logits = (rng.standard_normal(256) * 2).astype(np.float32)
        if trial % 5 == 0:  # exact ties: ties go to the lower id
            logits[rng.integers(0, 256, 40)] = logits.max()
        ids, w = orc.router_from_logits(logits)
        p = np.exp(logits.astype(np.float64) - logits.max())
        p /= p.sum()
        order = sorted(range(256), key=lambda i: (-np.float32(p[i]), i))[:8]
        assert list(ids) == order
        want = p[order] / p[order].sum()
        assert np.allclose(w, want, rtol=1e-5, atol=1e-7)
        assert all(w[i] >= w[i + 1] for i in range(7))


# ---- a7/a8/a21 -----------------------------------------------------------------
def test_silu_sigmoid_rmsnorm_kats_and_closed_forms():
    # reference.rs:124-146 and weights.rs:2483-2497
    assert orc.sigmoid(0.0) == 0.5
    assert orc.silu_mul(np.zeros(3), np.array([1.0, -2.0, 5.0]))[0] == 0.0
    out = orc.qwen_rmsnorm(np.array([3.0, 4.0]), np.array([1.0, 1.0]))
    assert abs(math.sqrt(float(np.mean(out.astype(np.float64) ** 2))) - 1.0) < 1e-5
    rng = np.random.default_rng(6)
    g = rng.standard_normal(100).astype(np.float32) * 4
    u = rng.standard_normal(100).astype(np.float32)
    gd = g.astype(np.float64)
    assert np.allclose(orc.silu_mul(g, u), gd / (1 + np.exp(-gd)) * u, rtol=1e-6, atol=1e-7)
    x = rng.standard_normal(2048).astype(np.float32)
    wn = rng.standard_normal(2048).astype(np.float32)
    xd = x.astype(np.float64)
    want = xd / np.sqrt(np.mean(xd ** 2) + 1e-6) * wn
    assert np.allclose(orc.qwen_rmsnorm(x, wn), want, rtol=1e-5, atol=1e-6)
    for v in (-30.0, -1.5, 0.25, 7.0):
        assert abs(orc.sigmoid(v) - 1 / (1 + math.exp(-v))) < 1e-7


# ---- a10/a12: expert and MoE layer -------------------------------------------
def np_expert(g, u, d, H, F, x):
    gv = np_dequant(g, F, H) @ x.astype(np.float64)
    uv = np_dequant(u, F, H) @ x.astype(np.float64)
    h = gv / (1 + np.exp(-gv)) * uv
    return np_dequant(d, H, F) @ h


def test_expert_forward_against_float64():
    H, F = 512, 256
    g, u, d = (synth.q4_0_synthetic(F, H, 900, 0), synth.q4_0_synthetic(F, H, 901, 0),
               synth.q4_0_synthetic(H, F, 902, 0))
    x = np.random.default_rng(7).standard_normal(H).astype(np.float32)
    want = np_expert(g, u, d, H, F, x)
    got = orc.expert_forward(g, u, d, H, F, x)
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1.0)) < 1e-5


@pytest.fixture(scope="module")
def small_layer():
    import sys
    sys.path.insert(0, str(GOLDEN))
    from golden_inputs import SMALL, small_layer_inputs

    router, gate, x, mats = small_layer_inputs()
    E, H, F = SMALL["experts"], SMALL["hidden"], SMALL["width"]
    host = orc.MoeLayerHost(router, gate, *mats[E], [m[0] for m in mats[:E]],
                            [m[1] for m in mats[:E]], [m[2] for m in mats[:E]], hidden=H, width=F)
    return host, router, gate, x, mats


def test_moe_layer_is_the_composition_of_its_pinned_parts(small_layer):
    # experts/mod.rs:1540-1634: shared expert scaled by sigmoid(gate . x),
    # then the routed experts in route order with the renormalised weights;
    # checked in float64 against independently decoded weights
    host, router, gate, x, mats = small_layer
    H, F = 256, 256
    y, ids, w = host.forward_batch(x)
    for t in range(4):
        lid, lw = orc.router_from_logits(orc.f32_matvec(router, x[t]))
        assert np.array_equal(ids[t], lid) and np.array_equal(w[t], lw)
        sg = 1 / (1 + math.exp(-float(gate.astype(np.float64) @ x[t].astype(np.float64))))
        want = np_expert(*mats[256], H, F, x[t]) * sg
        for k in range(8):
            want = want + float(w[t, k]) * np_expert(*mats[int(ids[t, k])], H, F, x[t])
        assert np.max(np.abs(y[t] - want) / np.maximum(np.abs(want), 1.0)) < 1e-5
    assert mtp.routes_union(ids) == orc.batch_union(ids)


def test_moe_layer_matches_golden(small_layer):
    host, _, _, x, _ = small_layer
    g = np.load(GOLDEN / "oracle_vectors.npz")
    for m in (1, 4):
        y, ids, w = host.forward_batch(x[:m])
        assert np.array_equal(ids, g[f"moe_ids{m}"]) and np.array_equal(w, g[f"moe_w{m}"])
        assert np.array_equal(y, g[f"moe_y{m}"])


def test_moe_layer_threaded_equals_serial(small_layer):
    host, _, _, x, _ = small_layer
    a = host.forward_batch(x, nthreads=1)
    b = host.forward_batch(x, nthreads=4)
    for u, v in zip(a, b):
        assert np.array_equal(u, v)


def test_routed_combine_against_float64_and_its_invariants(small_layer):
    # experts/mod.rs:1562-1566 for given routes: y = sum_k w_k expert_k(x) in
    # route order, checked in float64 against independently decoded weights
    host, _, _, x, mats = small_layer
    H, F = 256, 256
    rng = np.random.default_rng(3)
    t = 5
    xs = rng.standard_normal((t, H)).astype(np.float32)
    ids = rng.integers(0, 256, size=(t, 8)).astype(np.uint16)
    ids[0, 3] = ids[0, 1]  # a repeated expert is computed twice
    w = rng.random((t, 8)).astype(np.float32)
    y = host.routed_combine(xs, ids, w)
    for r in range(t):
        want = np.zeros(H)
        for k in range(8):
            want = want + float(w[r, k]) * np_expert(*mats[int(ids[r, k])], H, F, xs[r])
        assert np.max(np.abs(y[r] - want) / np.maximum(np.abs(want), 1.0)) < 1e-5
    # one-hot routes reproduce a single expert exactly
    oh = np.zeros_like(w)
    oh[:, 0] = 1.0
    y1 = host.routed_combine(xs, ids, oh)
    for r in range(t):
        e = int(ids[r, 0])
        assert np.array_equal(y1[r], orc.expert_forward(*mats[e], H, F, xs[r]))
    # threads do not change a bit; an out-of-range id is an error
    assert np.array_equal(host.routed_combine(xs, ids, w, nthreads=4), y)
    bad = ids.copy()
    bad[2, 2] = 256
    with pytest.raises(ValueError):
        host.routed_combine(xs, bad, w)


def test_routed_combine_is_the_routed_part_of_the_layer(small_layer):
    # forward_batch = shared * sigmoid(gate . x) + routed part, with the layer's
    # own routes (the two differ only in where the fp32 sums start)
    host, _, gate, x, mats = small_layer
    y, ids, w = host.forward_batch(x)
    routed = host.routed_combine(x, ids, w)
    for t in range(4):
        sg = orc.sigmoid(float(np.dot(gate.astype(np.float64), x[t].astype(np.float64))))
        shared = orc.expert_forward(*mats[256], 256, 256, x[t]) * np.float32(sg)
        want = y[t].astype(np.float64) - shared
        assert np.max(np.abs(routed[t] - want) / np.maximum(np.abs(want), 1.0)) < 1e-5


def test_config1_gemv_matches_golden():
    import sys
    sys.path.insert(0, str(GOLDEN))
    from golden_inputs import gemv_inputs

    w, x = gemv_inputs()
    g = np.load(GOLDEN / "oracle_vectors.npz")
    assert np.array_equal(orc.q4_0_matvec(w, 512, 2048, x), g["gemv_y"])


# ---- a16/a17/a18: greedy, draw, xoshiro --------------------------------------
def test_top_logit_candidates_ties_and_nan():
    # sampling/mod.rs:412-415 and 444-452
    toks, _ = orc.top_logit_candidates(np.array([1.0, 5.0, 5.0, 5.0, 2.0]))
    assert toks[0] == 1 and list(toks[:3]) == [1, 2, 3]
    toks, _ = orc.top_logit_candidates(np.array([1.0, np.nan, 3.0, np.nan]))
    assert toks[0] == 2
    big = np.arange(4096, dtype=np.float32) * 0.001
    big[2000] = np.nan
    assert orc.top_logit_candidates(big)[0][0] == 4095


def test_top_logit_candidates_against_numpy():
    rng = np.random.default_rng(8)
    for _ in range(100):
        lg = rng.integers(-5, 5, 300).astype(np.float32)  # many ties
        toks, vals = orc.top_logit_candidates(lg)
        want = np.argsort(-lg, kind="stable")[:4]
        assert list(toks) == list(want) and np.array_equal(vals, lg[want])


def test_xoshiro_reference_definition():
    # sampling/mod.rs:662-669
    rng = orc.Xoshiro(state=[1, 1, 1, 1])
    assert rng.next_u64() == 16_777_217
    assert rng.next_u64() != 16_777_217
    r = orc.Xoshiro(seed=3)
    assert all(0.0 <= r.next_f32() < 1.0 for _ in range(1000))


def test_softmax_draw_frequencies_track_the_softmax():
    # sampling/mod.rs:476-499: softmax [3,2,1,0] at T = 1
    values = np.array([3.0, 2.0, 1.0, 0.0], np.float32)
    p = np.exp(values.astype(np.float64))
    p /= p.sum()
    rng = orc.Xoshiro(seed=20260819)
    n = 60_000
    counts = np.zeros(4)
    for _ in range(n):
        counts[orc.softmax_draw(values, 1.0, rng.next_f32())] += 1
    assert np.all(np.abs(counts / n - p) < 0.01)


def test_softmax_draw_inverse_cdf_boundaries():
    values = np.array([0.0, 0.0, 0.0, 0.0], np.float32)  # uniform: quarters
    assert orc.softmax_draw(values, 1.0, 0.0) == 0
    assert orc.softmax_draw(values, 1.0, 0.2499) == 0
    assert orc.softmax_draw(values, 1.0, 0.2501) == 1
    assert orc.softmax_draw(values, 1.0, 0.9999) == 3


def _host_expf():
    import ctypes
    import ctypes.util

    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    return libm.expf


def test_softmax_draw_sums_are_the_sequential_f32_sums():
    """The draw's two sums (orc_softmax_draw_sums) against numpy's float32
    accumulate, which adds left to right in float32 (checked on a case where
    a pairwise order would differ): the token-order total of the host C
    library's expf((l - max) / T), then p = e / total and the sum of p in a
    stable descending order.  Rows: the configuration's N(0, 9) logits,
    flat ones, and one whose exponentials span the subnormal range."""
    assert np.add.accumulate(np.float32([1.0, 2.0 ** -24, 2.0 ** -24]))[-1] == np.float32(1.0)
    expf = _host_expf()
    rng = np.random.default_rng(5)
    rows = [((rng.standard_normal(151_936) * 3).astype(np.float32), 0.7),
            ((rng.standard_normal(151_936) * 0.1).astype(np.float32), 1.0),
            (rng.uniform(-104.0, 0.0, 20_000).astype(np.float32), 1.0)]
    for lg, T in rows:
        z = (lg - lg.max()) / np.float32(T)
        e = np.array([expf(float(v)) for v in z], np.float32)
        total = np.add.accumulate(e)[-1]
        p = e / total
        psum = np.add.accumulate(p[np.argsort(-p, kind="stable")])[-1]
        tok, t_orc, p_orc = orc.softmax_draw_sums(lg, T, 0.37)
        assert t_orc.tobytes() == total.tobytes() and p_orc.tobytes() == psum.tobytes()
        assert tok == orc.softmax_draw(lg, T, 0.37)
    assert np.count_nonzero((e > 0) & (e < np.finfo(np.float32).tiny)) > 1000  # subnormal terms


# ---- Philox -------------------------------------------------------------------
def philox_vectors():
    out = []
    for line in (GOLDEN / "philox_vectors.txt").read_text().splitlines():
        a, b = line.split("->")
        out.append(([int(v, 16) for v in a.split()], [int(v, 16) for v in b.split()]))
    return out


def test_philox_against_rocrand_and_random123_vectors():
    vecs = philox_vectors()
    # the first three are Random123's published kat_vectors for philox4x32_10
    assert vecs[0][1] == [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]
    assert vecs[1][1] == [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]
    assert vecs[2][1] == [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]
    for inp, want in vecs:
        assert list(orc.philox4x32_10(inp[:4], inp[4:])) == want
        assert list(synth.philox4x32_10(np.array([inp[:4]], np.uint32), inp[4:])[0]) == want


# ---- a22: acceptance ------------------------------------------------------------
def test_accept_exp_is_within_two_ulp_of_exp():
    zs = np.concatenate([np.linspace(-87, 0, 20001, dtype=np.float32),
                         np.float32([-1e-8, -0.0, 0.0, -86.99, -0.5])])
    for z in zs:
        got = np.float32(orc.accept_exp(float(z)))
        want = math.exp(float(z))
        ulp = np.spacing(np.float32(want))
        assert abs(float(got) - want) <= 2 * float(ulp), z
    assert orc.accept_exp(-87.5) == 0.0 and orc.accept_exp(float("-inf")) == 0.0
    assert orc.accept_exp(float("nan")) == 0.0


def test_fixed_point_helpers_are_exact():
    rng = np.random.default_rng(9)
    vals = np.concatenate([rng.random(2000).astype(np.float32), np.float32([0, 1, 1e-30, 0.5])])
    for v in vals:
        f = Fraction(float(v))
        assert orc.fix40(float(v)) == math.floor(f * 2 ** 40)
        assert orc.fix62(float(v)) == math.floor(f * 2 ** 62)
    for _ in range(2000):
        total = int(rng.integers(1, 2 ** 63, dtype=np.uint64))
        u = float(np.float32(rng.random()))
        assert orc.scale_floor(total, u) == math.floor(total * Fraction(u))
        v = int(rng.integers(0, 2 ** 63, dtype=np.uint64)) >> int(rng.integers(0, 60))
        assert np.float32(orc.u64_to_f32(v)) == np.float32(float(Fraction(v)))


def softmax64(row, T):
    z = row.astype(np.float64) / T
    e = np.exp(z - z.max())
    return e / e.sum()


def test_accept_closed_forms():
    rng = np.random.default_rng(10)
    V, k = 50, 3
    draft = (rng.standard_normal((k, V)) * 2).astype(np.float32)
    target = np.vstack([draft, (rng.standard_normal(V) * 2).astype(np.float32)[None]])
    dtok = rng.integers(0, V, k).astype(np.int32)
    u = rng.random(k).astype(np.float32)
    ur = rng.random(k + 1).astype(np.float32)
    # p == q: every draft is accepted, the bonus comes from the last target row
    a, toks = orc.accept(target, draft, dtok, 0.7, False, u, ur)
    assert a == k and toks[:k] == list(dtok)
    # p(d) = 0 < q(d): rejected at position 0, the replacement is not d
    t2 = target.copy()
    t2[0, dtok[0]] = -np.inf
    a, toks = orc.accept(t2, draft, dtok, 0.7, False, u, ur)
    assert a == 0 and toks[0] != dtok[0]
    # one-hot p on d: accepted whatever the uniform
    t3 = target.copy()
    t3[0] = -1e4
    t3[0, dtok[0]] = 0.0
    a, toks = orc.accept(t3, draft, dtok, 0.7, False, np.float32([0.999999, 0, 0]), ur)
    assert a >= 1 and toks[0] == dtok[0]


def test_accept_greedy_k1_is_verify_pair():
    rng = np.random.default_rng(11)
    for _ in range(200):
        target = rng.integers(-3, 3, (2, 20)).astype(np.float32)
        d = int(rng.integers(0, 20))
        a, toks = orc.accept(target, None, [d], 0.7, True)
        top = int(orc.top_logit_candidates(target[0])[0][0])
        vp = mtp.verify_pair(top, d)
        assert (a == 1) == vp.accepted and len(toks) == vp.emitted_tokens
        assert toks[0] == (d if vp.accepted else top)


def test_accept_emits_tokens_distributed_as_the_target():
    # speculative sampling: with d ~ q, the first emitted token ~ p (chi-square)
    V, T = 6, 0.7
    target = np.array([[2.0, 1.0, 0.5, 0.0, -1.0, 1.5], [0, 0, 0, 0, 0, 0]], np.float32)
    draft = np.array([[0.0, 2.0, 1.0, 0.5, 0.0, -2.0]], np.float32)
    p = softmax64(target[0], T)
    q = softmax64(draft[0], T)
    rng = np.random.default_rng(12)
    n = 40_000
    counts = np.zeros(V)
    cq = np.cumsum(q)
    for _ in range(n):
        d = int(min(np.searchsorted(cq, rng.random(), side="right"), V - 1))
        _, toks = orc.accept(target, draft, [d], T, False, rng.random(1).astype(np.float32),
                             rng.random(2).astype(np.float32))
        counts[toks[0]] += 1
    chi2 = float(np.sum((counts - n * p) ** 2 / (n * p)))
    assert chi2 < 25.0  # 5 degrees of freedom: P(chi2 > 25) ~ 1e-4


def test_accept_matches_golden():
    import sys
    sys.path.insert(0, str(GOLDEN))
    from golden_inputs import accept_inputs

    g = np.load(GOLDEN / "oracle_vectors.npz")
    for gi, greedy in enumerate((True, False)):
        for seed in range(64):
            target, draft, dtok, u, ur = accept_inputs(seed)
            a, toks = orc.accept(target, draft, dtok, 0.7, greedy, u, ur)
            assert a == g["accept_len"][gi, seed]
            assert toks == list(g["accept_tokens"][gi, seed, : a + 1])
    assert set(g["accept_len"][0]) == {0, 1, 2, 3} and set(g["accept_len"][1]) == {0, 1, 2, 3}


# ---- f1 / a4 / a20: Q4_K ------------------------------------------------------
def lcg_q4_k_weights(rows: int, cols: int) -> np.ndarray:
    """The reference's Q4_K fixture (backend/metal/kernels.rs:1118-1132):
    d = 1.0, dmin = 0.25, every other byte from the LCG
    counter = counter * 1103515245 + 12345 (u32), byte = counter >> 16."""
    n_blocks = rows * (cols // 256)
    out = np.zeros((n_blocks, 144), np.uint8)
    counter = 1
    for b in range(n_blocks):
        out[b, 0:2] = (0x00, 0x3C)
        out[b, 2:4] = (0x00, 0x34)
        for i in range(4, 144):
            counter = (counter * 1_103_515_245 + 12_345) & 0xFFFFFFFF
            out[b, i] = (counter >> 16) & 0xFF
    return out.reshape(-1)


def lcg_vector(cols: int) -> np.ndarray:
    """kernels.rs:1134-1138: ((i % 11) * 0.3 - 1.5) in f32."""
    return np.array([np.float32(i % 11) * np.float32(0.3) - np.float32(1.5) for i in range(cols)], np.float32)


def q4_k_exact(block: np.ndarray) -> np.ndarray:
    """The decoded values as exact rationals in float64: d sc q - dmin m with
    d, dmin the f16 fields (numpy binary16) and the 6-bit (sc, m) of each
    sub-block from the 12 packed bytes."""
    b = np.asarray(block, np.uint8)
    d = float(b[0:2].view(np.float16)[0])
    dmin = float(b[2:4].view(np.float16)[0])
    s = [int(v) for v in b[4:16]]
    out = np.zeros(256)
    for j in range(8):
        if j < 4:
            sc, m = s[j] & 63, s[j + 4] & 63
        else:
            sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4)
            m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4)
        qs = b[16 + 32 * (j // 2): 16 + 32 * (j // 2) + 32].astype(np.int64)
        q = (qs & 0xF) if j % 2 == 0 else (qs >> 4)
        out[64 * (j // 2) + 32 * (j % 2): 64 * (j // 2) + 32 * (j % 2) + 32] = d * sc * q - dmin * m
    return out


def test_q4_k_dequant_kat():
    # dequant.rs:287-306: d = 1, dmin = 0, every sub-block scale 1, qs[0] = 0x12
    b = np.zeros(144, np.uint8)
    b[0:2] = (0x00, 0x3C)
    b[4:8] = 1
    b[8:12] = 1
    b[16] = 0x12
    for indep in (False, True):
        out = orc.dequantize_q4_k(b, independent=indep)
        assert out[0] == 2.0 and out[32] == 1.0 and out[1] == 0.0


def test_q4_k_primary_equals_independent():
    # validate.rs:289-298: the byte pattern i * 19 + 3, then random blocks
    blk = np.array([(i * 19 + 3) & 0xFF for i in range(144)], np.uint8)
    assert np.array_equal(orc.dequantize_q4_k(blk), orc.dequantize_q4_k(blk, independent=True))
    rng = np.random.default_rng(41)
    for _ in range(300):
        blk = rng.integers(0, 256, 144).astype(np.uint8)
        blk[1] &= 0x7B  # finite f16 d and dmin (exponent below all-ones)
        blk[3] &= 0x7B
        a, b = orc.dequantize_q4_k(blk), orc.dequantize_q4_k(blk, independent=True)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_q4_k_dequant_is_the_once_rounded_exact_value():
    # every fp32 step before the final subtraction is exact (d sc needs 17
    # bits, (d sc) q 21, dmin m 17), so each value is the exact decode
    # rounded once to f32
    rng = np.random.default_rng(42)
    blocks = [lcg_q4_k_weights(1, 256)] + [rng.integers(0, 256, 144).astype(np.uint8) for _ in range(200)]
    for blk in blocks:
        blk = blk.copy()
        blk[1] &= 0x7B
        blk[3] &= 0x7B
        assert np.array_equal(orc.dequantize_q4_k(blk), q4_k_exact(blk).astype(np.float32))


def test_q4k_gemv_reference_fixture_against_float64():
    # kernels.rs:1140-1165 shape (17 x 512) and fixture; float64 brute force
    rows, cols = 17, 512
    w = lcg_q4_k_weights(rows, cols)
    x = lcg_vector(cols)
    y = orc.q4k_gemv(w, rows, cols, x)
    dq = np.concatenate([q4_k_exact(w[i * 144:(i + 1) * 144]) for i in range(rows * 2)]).reshape(rows, cols)
    want = dq @ x.astype(np.float64)
    assert np.max(np.abs(y - want) / np.maximum(np.abs(want), 1.0)) < 1e-5
    # the reference's own test bound against its Metal kernel is 1e-2 absolute
    assert np.max(np.abs(y - want)) < 1e-2


def test_q4k_gemv_one_hot_columns_recover_the_decode():
    # kernels.rs:1168-1196: a one-hot input selects one decoded element
    w = lcg_q4_k_weights(1, 256)
    dq = orc.dequantize_q4_k(w)
    for k in range(256):
        x = np.zeros(256, np.float32)
        x[k] = 1.0
        assert orc.q4k_gemv(w, 1, 256, x)[0] == dq[k]
    with pytest.raises(ValueError):
        orc.q4k_gemv(w, 1, 200, np.zeros(200, np.float32))


def test_quantize_q8_k_closed_forms():
    q, sums, scale = orc.quantize_q8_k(np.zeros(256, np.float32))
    assert scale == 0.0 and not q.any() and not sums.any()
    rng = np.random.default_rng(43)
    v = rng.standard_normal(256).astype(np.float32)
    i_max = int(np.argmax(np.abs(v)))
    q, sums, scale = orc.quantize_q8_k(v)
    assert q[i_max] == -127  # the largest magnitude maps to -127 (sign folded into the scale)
    assert np.array_equal(sums, q.astype(np.int64).reshape(16, 16).sum(axis=1).astype(np.int16))
    assert np.max(np.abs(q.astype(np.float64) * scale - v)) <= abs(scale) / 2 * (1 + 1e-6)
    # signed maximum -127 -> inverse scale exactly 1: ties round to even
    t = np.zeros(256, np.float32)
    t[0] = -127.0
    t[1:7] = (2.5, 3.5, -2.5, -3.5, 0.5, 126.5)
    q, _, scale = orc.quantize_q8_k(t)
    assert scale == 1.0
    assert list(q[:7]) == [-127, 2, 4, -2, -4, 0, 126]


def test_q4_k_dot_pre_against_float64_of_its_integer_terms():
    rng = np.random.default_rng(44)
    nb = 3
    row = rng.integers(0, 256, nb * 144).astype(np.uint8)
    for b in range(nb):
        row[b * 144 + 1] &= 0x3B  # modest finite d, dmin
        row[b * 144 + 3] &= 0x3B
    x = rng.standard_normal(nb * 256).astype(np.float32)
    qs, ss, scs = zip(*(orc.quantize_q8_k(x[b * 256:(b + 1) * 256]) for b in range(nb)))
    q8, sums, scales = np.concatenate(qs), np.concatenate(ss), np.array(scs, np.float32)
    got = orc.q4_k_dot_pre(row, q8, sums, scales)
    want = 0.0
    for b in range(nb):
        blk = row[b * 144:(b + 1) * 144]
        d = float(blk[0:2].view(np.float16)[0])
        dmin = float(blk[2:4].view(np.float16)[0])
        # d sc q - dmin m summed against q8, times the Q8_K scale, exactly
        dq_over = q4_k_exact(blk)  # d sc q - dmin m
        want += float(scales[b]) * float(np.dot(dq_over, q8[b * 256:(b + 1) * 256].astype(np.float64)))
    assert abs(got - want) <= 1e-5 * max(abs(want), 1.0)


def test_q4_k_matvec_within_the_q8_k_rounding_bound():
    # each activation moves by at most half its chunk's Q8_K step, so the
    # integer path sits within sum_b |scale_b|/2 * sum_i |w_i| of the fp32 GEMV
    rng = np.random.default_rng(45)
    rows, cols = 8, 512
    w = lcg_q4_k_weights(rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    a = orc.q4_k_matvec(w, rows, cols, x)
    b = orc.q4k_gemv(w, rows, cols, x)
    steps = np.array([orc.quantize_q8_k(x[c * 256:(c + 1) * 256])[2] for c in range(cols // 256)])
    for r in range(rows):
        dq = np.concatenate([q4_k_exact(w[(r * 2 + c) * 144:(r * 2 + c + 1) * 144]) for c in range(2)])
        bound = sum(abs(steps[c]) / 2 * np.abs(dq[c * 256:(c + 1) * 256]).sum() for c in range(2))
        assert abs(float(a[r]) - float(b[r])) <= bound * 1.001 + 1e-3


def random_q4_k(rows: int, cols: int, seed: int, d_range=(0.002, 0.05)) -> np.ndarray:
    """Random GGML Q4_K bytes whose f16 d and dmin are finite and modest."""
    rng = np.random.default_rng(seed)
    n = rows * (cols // 256)
    blk = rng.integers(0, 256, size=(n, 144), dtype=np.uint8)
    blk[:, 0:2] = rng.uniform(*d_range, size=n).astype(np.float16).view(np.uint8).reshape(n, 2)
    blk[:, 2:4] = rng.uniform(*d_range, size=n).astype(np.float16).view(np.uint8).reshape(n, 2)
    return blk.reshape(-1)


def test_pack_q4_k_scales_inverts_the_decoder():
    # every 6-bit scale and min lands where the oracle's decoder (and the
    # independent float64 decode) reads it
    rng = np.random.default_rng(3)
    for _ in range(20):
        sc, mn = rng.integers(0, 64, size=8), rng.integers(0, 64, size=8)
        b = np.zeros(144, np.uint8)
        b[0:2] = (0x00, 0x3C)  # d = 1
        b[2:4] = (0x00, 0x3C)  # dmin = 1
        b[4:16] = pack_q4_k_scales(sc, mn)
        b[16:] = 0x35  # q = 5 (low nibble) and 3 (high nibble)
        want = np.concatenate([np.full(32, sc[j] * (5 if j % 2 == 0 else 3) - mn[j]) for j in range(8)])
        assert np.array_equal(orc.dequantize_q4_k(b), want.astype(np.float32))
        assert np.array_equal(q4_k_exact(b), want.astype(np.float64))
    w = centered_q4_k(4, 512, 9)
    v = q4_k_dense(w, 4, 512)
    assert abs(v.mean()) < 0.05 * v.std()


def q4_k_dense(w: np.ndarray, rows: int, cols: int) -> np.ndarray:
    nb = rows * (cols // 256)
    return np.concatenate([q4_k_exact(w[i * 144:(i + 1) * 144]) for i in range(nb)]).reshape(rows, cols)


@pytest.fixture(scope="module")
def q4k_small_layer():
    E, H, F = 256, 256, 256
    rng = np.random.default_rng(61)
    router = (rng.standard_normal((E, H)) / 16).astype(np.float32)
    gate = (rng.standard_normal(H) / 16).astype(np.float32)
    shapes = ((F, H), (F, H), (H, F))
    mats = [tuple(random_q4_k(r, c, 5000 + 3 * e + i) for i, (r, c) in enumerate(shapes))
            for e in range(E + 1)]
    host = orc.MoeLayerHost(router, gate, *mats[E], [m[0] for m in mats[:E]],
                            [m[1] for m in mats[:E]], [m[2] for m in mats[:E]], hidden=H,
                            width=F, fmt="q4_k")
    x = rng.standard_normal((4, H)).astype(np.float32)
    return host, router, gate, x, mats


def test_q4_k_moe_layer_is_the_composition_of_its_pinned_parts(q4k_small_layer):
    # experts/mod.rs:1600-1634 with matvec_payload's Q4_K arm: bit-identical
    # to the pinned pieces composed in f32 -- shared expert x sigmoid(gate .
    # x) (scale_in_place), then + routed x weight per route in route order
    # (add_scaled_in_place, weights.rs:267-281)
    host, router, gate, x, mats = q4k_small_layer
    H = F = 256
    y, ids, w = host.forward_batch(x)
    for t in range(4):
        lid, lw = orc.router_from_logits(orc.f32_matvec(router, x[t]))
        assert np.array_equal(ids[t], lid) and np.array_equal(w[t], lw)
        logit = orc.f32_matvec(gate.reshape(1, -1), x[t])[0]
        out = orc.q4_k_expert_forward(*mats[256], H, F, x[t]) * np.float32(orc.sigmoid(logit))
        for k in range(8):
            out = out + orc.q4_k_expert_forward(*mats[int(ids[t, k])], H, F, x[t]) * w[t, k]
        assert out.dtype == np.float32 and np.array_equal(out.view(np.uint32), y[t].view(np.uint32))


def q8_k_rounded(v: np.ndarray) -> np.ndarray:
    """The values quantize_q8_k stands for (q x scale per 256-chunk), float64."""
    v = np.asarray(v, np.float32)
    out = np.empty(v.size)
    for c in range(v.size // 256):
        q, _, scale = orc.quantize_q8_k(v[c * 256:(c + 1) * 256])
        out[c * 256:(c + 1) * 256] = q.astype(np.float64) * float(scale)
    return out


def test_q4_k_moe_layer_against_float64_of_the_exact_decode(q4k_small_layer):
    # the same layer in float64 over the exactly decoded matrices (q4_k_exact)
    # and the Q8_K-rounded activations (x, and h = SwiGLU of the float64 gate
    # and up): only f32 rounding separates it from the oracle (~2e-7 here),
    # while dropping one route moves the output by 7e-2 or more
    host, router, gate, x, mats = q4k_small_layer
    H = F = 256
    y, ids, w = host.forward_batch(x)
    dense = {}

    def expert(e, xv):
        if e not in dense:
            dense[e] = (q4_k_dense(mats[e][0], F, H), q4_k_dense(mats[e][1], F, H),
                        q4_k_dense(mats[e][2], H, F))
        g, u, d = dense[e]
        xq = q8_k_rounded(xv)
        gv, uv = g @ xq, u @ xq
        return d @ q8_k_rounded((gv / (1 + np.exp(-gv)) * uv).astype(np.float32))

    for t in range(4):
        want = expert(256, x[t]) / (1 + math.exp(-float(gate.astype(np.float64) @ x[t].astype(np.float64))))
        for k in range(8):
            want = want + float(w[t, k]) * expert(int(ids[t, k]), x[t])
        err = np.max(np.abs(y[t] - want)) / max(np.max(np.abs(want)), 1.0)
        assert err < 1e-5, err


# ---- f3: Q6_K (the canonical LM head) -------------------------------------------
def q6_k_values_np(block: np.ndarray) -> np.ndarray:
    """q - 32 of the 256 elements by array slicing (ggml's block_q6_K: two
    128-element halves of four interleaved 32-element groups)."""
    b = np.asarray(block, np.uint8).astype(np.int64)
    q = np.empty(256, np.int64)
    for h in range(2):
        lo, hb = b[64 * h:64 * h + 64], b[128 + 32 * h:128 + 32 * h + 32]
        base = 128 * h
        q[base:base + 32] = (lo[:32] & 15) | ((hb & 3) << 4)
        q[base + 32:base + 64] = (lo[32:] & 15) | (((hb >> 2) & 3) << 4)
        q[base + 64:base + 96] = (lo[:32] >> 4) | (((hb >> 4) & 3) << 4)
        q[base + 96:base + 128] = (lo[32:] >> 4) | (((hb >> 6) & 3) << 4)
    return q - 32


def q6_k_exact(block: np.ndarray) -> np.ndarray:
    b = np.asarray(block, np.uint8)
    d = float(b[208:210].view(np.float16)[0])
    sc = b[192:208].view(np.int8).astype(np.float64)
    return d * np.repeat(sc, 16) * q6_k_values_np(b)


def random_q6_k(n: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    blk = rng.integers(0, 256, size=(n, 210), dtype=np.uint8)
    blk[:, 208:210] = rng.uniform(0.001, 0.05, n).astype(np.float16).view(np.uint8).reshape(n, 2)
    return blk


def test_q6_k_kats():
    # dequant.rs:308-315 and weights.rs:2532-2543: zero ql / qh (q = -32
    # everywhere), group scales 1, d = 1; x = ones gives 256 x -32
    b = np.zeros(210, np.uint8)
    b[192:208] = 1
    b[208:210] = (0x00, 0x3C)
    assert np.all(orc.dequantize_q6_k(b) == -32.0)
    assert orc.q6_k_matvec(b, 1, 256, np.ones(256, np.float32))[0] == -8192.0
    with pytest.raises(ValueError):
        orc.q6_k_matvec(b, 1, 200, np.ones(200, np.float32))


def test_q6_k_dequant_is_the_once_rounded_exact_value():
    # d * scale needs 19 bits (exact); times q - 32 it is rounded once
    for blk in random_q6_k(300, 51):
        assert np.array_equal(orc.dequantize_q6_k(blk), q6_k_exact(blk).astype(np.float32))


def test_q6_k_single_field_probes():
    # one low nibble, one high-bit pair, one scale: the element each field
    # feeds moves alone
    b = np.zeros(210, np.uint8)
    b[192:208] = 1
    b[208:210] = (0x00, 0x3C)
    base = orc.dequantize_q6_k(b)
    for byte, val, elem in ((0, 0x01, 0), (0, 0x10, 64), (32, 0x01, 32), (63, 0x10, 127),
                            (64, 0x01, 128), (127, 0x10, 255), (128, 0x01, 0), (128, 0x04, 32),
                            (128, 0x10, 64), (128, 0x40, 96), (191, 0x40, 255)):
        p = b.copy()
        p[byte] = val
        diff = np.flatnonzero(orc.dequantize_q6_k(p) != base)
        assert list(diff) == [elem], (byte, val, diff)
    p = b.copy()
    p[192 + 5] = 3  # group 5 = elements 80..95
    assert list(np.flatnonzero(orc.dequantize_q6_k(p) != base)) == list(range(80, 96))


def test_q6_k_dot_pre_against_float64_and_lane_sums():
    rng = np.random.default_rng(52)
    nb = 3
    row = random_q6_k(nb, 53).reshape(-1)
    x = rng.standard_normal(nb * 256).astype(np.float32)
    qs, _, scs = zip(*(orc.quantize_q8_k(x[b * 256:(b + 1) * 256]) for b in range(nb)))
    q8, scales = np.concatenate(qs), np.array(scs, np.float32)
    got = orc.q6_k_dot_pre(row, q8, scales)
    want = 0.0
    for b in range(nb):
        blk = row[b * 210:(b + 1) * 210]
        want += float(scales[b]) * float(np.dot(q6_k_exact(blk), q8[b * 256:(b + 1) * 256].astype(np.float64)))
    assert abs(got - want) <= 1e-5 * max(abs(want), 1.0)


def test_q6_k_matvec_within_the_q8_k_rounding_bound():
    rng = np.random.default_rng(54)
    rows, cols = 8, 512
    w = random_q6_k(rows * 2, 55).reshape(-1)
    x = rng.standard_normal(cols).astype(np.float32)
    y = orc.q6_k_matvec(w, rows, cols, x)
    steps = [abs(orc.quantize_q8_k(x[c * 256:(c + 1) * 256])[2]) for c in range(2)]
    for r in range(rows):
        dq = np.concatenate([q6_k_exact(w[(r * 2 + c) * 210:(r * 2 + c + 1) * 210]) for c in range(2)])
        exact = float(np.dot(dq, x.astype(np.float64)))
        bound = sum(steps[c] / 2 * np.abs(dq[c * 256:(c + 1) * 256]).sum() for c in range(2))
        assert abs(float(y[r]) - exact) <= bound * 1.001 + 1e-3
