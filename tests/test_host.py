"""CPU tests of the host-side logic: MTP accounting (runtime/mtp.rs), the
union golden from the reference's committed real router trace, and the
synthetic-weight generator shared by the device kernel and the host."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import cpu_oracle as orc
from turboqwenfare_amd import mtp, synth

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_verify_pair_kat():
    # mtp.rs:212-221
    assert mtp.verify_pair(42, 42) == mtp.VerifyOutcome(True, 2)
    assert mtp.verify_pair(42, 7) == mtp.VerifyOutcome(False, 1)


def test_statistics_kat():
    # mtp.rs:224-235
    s = mtp.MtpStatistics()
    s.record(True, 2, 1)
    s.record(False, 1, 1)
    s.record(True, 2, 1)
    assert (s.drafted_tokens, s.accepted_tokens, s.emitted_tokens, s.target_backbone_passes) == (3, 2, 5, 3)
    assert abs(s.acceptance_rate() - 2 / 3) < 1e-9
    assert abs(s.emitted_tokens_per_target_pass() - 5 / 3) < 1e-9
    assert mtp.MtpStatistics().acceptance_rate() == 0.0


def test_statistics_k_draft_verify():
    s = mtp.MtpStatistics()
    s.record_verify(3, 2)  # two of three drafts accepted, 3 tokens emitted
    s.record_verify(3, 3)
    assert (s.drafted_tokens, s.accepted_tokens, s.emitted_tokens, s.target_backbone_passes) == (6, 5, 7, 2)


def test_controller_hysteresis_kats():
    # mtp.rs:238-266
    c = mtp.MtpController(4)
    assert not c.enabled
    c.record_and_decide(2)
    assert not c.enabled
    for _ in range(4):
        c.record_and_decide(2)
    assert c.enabled
    for _ in range(4):
        c.record_and_decide(0)
    assert not c.enabled


def test_union_bandwidth_kat():
    # mtp.rs:269-298
    r = mtp.union_bandwidth([1, 2, 3, 4, 5, 6, 7, 8], [1, 2, 3, 4, 9, 10, 11, 12])
    assert r.union_experts == 12 and r.separate_experts_sum == 16
    assert r.saved_bytes > 0 and r.union_bytes + r.saved_bytes == r.separate_bytes_sum


def test_expert_bytes():
    # mtp.rs:38-42 with spec section 117 geometry: 1,769,472 B per expert,
    # equal for Q4_K (144 B / 256) and Q4_0 (18 B / 32)
    assert mtp.expert_bytes() == 1_769_472 == mtp.expert_bytes_q4_0()


def test_real_trace_union_savings_golden():
    # mtp.rs:310-343 over docs/research/qualification/raw-a-128-route-trace.json
    # (ids extracted by tests/golden/make_golden.py); the figures are the ones
    # the reference records in docs/research/phase-33-mtp.md:57
    ids = np.load(GOLDEN / "route_trace_ids.npy")
    union = separate = pairs = 0
    for s in range(ids.shape[0] - 1):
        for layer in range(ids.shape[1]):
            r = mtp.union_bandwidth(ids[s, layer], ids[s + 1, layer])
            union += r.union_bytes
            separate += r.separate_bytes_sum
            pairs += 1
    assert pairs == 5_080
    assert separate == 143_822_684_160
    assert union == 113_892_065_280
    assert round((separate - union) / separate * 100, 2) == 20.81


def test_routes_union_is_first_demand_order():
    routes = [[5, 3, 9, 1, 2, 4, 6, 7], [3, 8, 5, 10, 11, 12, 13, 14]]
    assert mtp.routes_union(routes) == [5, 3, 9, 1, 2, 4, 6, 7, 8, 10, 11, 12, 13, 14]
    assert mtp.routes_union(routes) == orc.batch_union(np.array(routes, np.uint16))
    bw = mtp.routes_union_bandwidth(routes)
    assert bw.union_experts == 14 and bw.separate_experts_sum == 16


def test_expected_tokens_per_step():
    # E[tokens / step] = (1 - a^(k+1)) / (1 - a) for k = 3
    assert abs(mtp.expected_tokens_per_step(0.6, 3) - 2.176) < 1e-12
    assert abs(mtp.expected_tokens_per_step(0.8, 3) - 2.952) < 1e-12


def test_synthetic_q4_0_definition():
    # the generator's definition: nibbles are Philox words, scales
    # 0.005 + 0.015 u rounded to binary16
    q = synth.q4_0_synthetic(3, 64, 17, 4).reshape(-1, 18)
    for b in range(q.shape[0]):
        words = orc.philox4x32_10([b, 0, 0, 0], [17, 4])
        assert q[b, 2:].tobytes() == words.astype("<u4").tobytes()
        w0 = orc.philox4x32_10([b, 0, 1, 0], [17, 4])[0]
        d = np.float32(0.005) + np.float32(0.015) * (np.float32(w0 >> 8) * np.float32(2 ** -24))
        assert q[b, 0:2].tobytes() == np.float16(d).tobytes()
    scales = q[:, 0:2].copy().view(np.float16).astype(np.float32)
    assert np.all((scales >= 0.00499) & (scales <= 0.02001))


def test_philox_uniforms_definition():
    u = synth.philox_uniforms(9, 1, 5)
    for i in range(5):
        w = orc.philox4x32_10([i, 1, 0, 0], [9, 0x243F6A88])[0]
        assert u[i] == np.float32(w >> 8) * np.float32(2 ** -24)
    assert np.all((u >= 0) & (u < 1))


@pytest.mark.parametrize("bad", [31, 48])
def test_synthetic_rejects_bad_cols(bad):
    if bad % 32:
        with pytest.raises(ValueError):
            synth.q4_0_synthetic(2, bad, 0, 0)
    else:
        assert synth.q4_0_synthetic(2, bad, 0, 0).size == 2 * (bad // 32) * 18


def test_zipf_routes_definition_and_config5_statistics():
    # config 5: 512 tokens, Zipf(s=1.1) popularity, Gumbel-top-k without
    # replacement, seed 0 (head expert M = 448, ~251 distinct, median ~5)
    ids, w = synth.zipf_routes(512, 256, 8, 1.1, 0)
    assert ids.shape == (512, 8) and ids.dtype == np.uint16 and w.dtype == np.float32
    assert all(len(set(r.tolist())) == 8 for r in ids)
    assert np.all(np.abs(w.sum(axis=1) - 1.0) < 1e-6) and np.all(np.diff(w, axis=1) <= 0)
    counts = np.bincount(ids.reshape(-1).astype(np.int64), minlength=256)
    assert counts.max() == 448 and 240 <= int((counts > 0).sum()) <= 256
    assert 4 <= float(np.median(counts[counts > 0])) <= 8
    # popularity follows the rank: the head expert is the rank-0 one
    rank = np.random.default_rng(0).permutation(256)
    assert int(np.argmax(counts)) == int(np.argmin(rank))
    a, b = synth.zipf_routes(64, seed=3), synth.zipf_routes(64, seed=3)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_bf16_round_nearest_even_kats():
    v = np.array([1.0, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -2.5, 3.0e38, 1.0e-40], np.float32)
    assert synth.bf16_round(v).tolist() == [0x3F80, 0x3F80, 0x3F82, 0xC020, 0x7F62, 0x0001]
    x = np.random.default_rng(0).standard_normal(1000).astype(np.float32)
    r = synth.bf16_to_f32(synth.bf16_round(x))
    assert np.all(np.abs(r - x) <= np.abs(x) * 2.0 ** -8)  # half an ulp of 8 significant bits
    assert np.array_equal(synth.bf16_to_f32(synth.bf16_round(r)), r)


def test_zero_mean_recipe_maps_only_nibble_zero():
    """Every nibble value at every position of a word: 0 -> 8, 1..15 kept,
    the other nibbles of the word untouched."""
    from turboqwenfare_amd import synth

    words = []
    for pos in range(8):
        for v in range(16):
            for fill in (0x0, 0xF, 0x5):
                w = 0
                for j in range(8):
                    w |= (v if j == pos else fill) << (4 * j)
                words.append(w)
    words = np.array(words, dtype=np.uint32)
    out = synth.zero_mean_nibbles(words)
    for w, o in zip(words.tolist(), out.tolist()):
        for j in range(8):
            n, m = (w >> (4 * j)) & 15, (o >> (4 * j)) & 15
            assert m == (8 if n == 0 else n)


def test_zero_mean_recipe_is_symmetric_and_keeps_scales():
    from turboqwenfare_amd import synth

    a = synth.q4_0_synthetic(64, 2048, 5, 1).reshape(-1, 18)
    b = synth.q4_0_synthetic(64, 2048, 5, 1, "zero_mean").reshape(-1, 18)
    assert np.array_equal(a[:, :2], b[:, :2])  # the same binary16 scales
    q = np.concatenate([b[:, 2:] & 15, b[:, 2:] >> 4]).astype(np.int64) - 8
    assert q.min() == -7 and q.max() == 7
    assert abs(q.mean()) < 0.01
    q0 = np.concatenate([a[:, 2:] & 15, a[:, 2:] >> 4]).astype(np.int64) - 8
    assert abs(q0.mean() + 0.5) < 0.01
    with pytest.raises(ValueError):
        synth.q4_0_synthetic(1, 32, 1, 1, 7)


def test_device_record_model_rounds_like_the_records():
    """make_stack40_spread.records (the 40-layer bound's model of the device's
    activation records): each 32-value block keeps rint(v / 2^(E-21)) with E
    the exponent of its largest |v|, so every value moves by at most 2^-22 of
    the block maximum, values on the grid do not move, a block at or below
    2^-100 is zero, and the largest value keeps 22-23 significant bits."""
    import sys
    from pathlib import Path

    sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
    import make_stack40_spread as ms

    rng = np.random.default_rng(5)
    for scale in (1e-30, 1e-3, 1.0, 3e4):
        v = (rng.standard_normal(256) * scale).astype(np.float32)
        r = ms.records(v)
        for b in range(8):
            blk, rb = v[32 * b:32 * b + 32].astype(np.float64), r[32 * b:32 * b + 32]
            amax = np.abs(blk).max()
            assert np.abs(rb - blk).max() <= amax * 2.0 ** -22
            step = 2.0 ** (np.floor(np.log2(amax)) - 21)
            assert np.array_equal(rb / step, np.rint(rb / step))
        assert np.array_equal(ms.records(r), r)
    assert not ms.records(np.full(32, 2.0 ** -101, np.float32)).any()
    grid = np.arange(-16, 16, dtype=np.float32) * 2.0 ** -10
    assert np.array_equal(ms.records(grid), grid)


def test_q4k_stack_routes_change_under_rounding_noise():
    """The Q4_K 40-layer stack (workloads.SyntheticQ4KStack, host copy) is
    chaotic at rounding level, which is why its GPU test checks the device
    layer by layer: with the input rows perturbed by 2^-24 relative noise
    (trial 2 of make_stack40_spread.py --q4k, M = 1) the oracle takes other
    routes from layer 5 on and ends O(1) away at layer 40, as recorded."""
    import json
    import sys
    from pathlib import Path

    golden = Path(__file__).resolve().parent / "golden"
    sys.path.insert(0, str(golden))
    import make_stack40_spread as ms
    from stack_oracle import oracle_replay

    spread = json.loads((golden / "stack40_spread.json").read_text())
    st = ms.HostQ4KStack(ms.LAYERS)
    h0 = synth.normal((4, 2048), seed=1)[:1]
    h, ids, _ = oracle_replay(st, h0)
    first, dist = ms.first_flip(st, h0, ids, h, 2, False)
    assert first == spread["q4k_m1_first_flip"][2] == 5
    assert dist == pytest.approx(spread["q4k_m1"][2], rel=1e-6)
    assert dist > 1.0
