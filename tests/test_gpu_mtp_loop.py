"""The MTP decode loop (turboqwenfare_amd/mtp_loop.py) on the GPU against the
CPU oracle, stage by stage and step by step.

For every step each device stage is replayed on the host from the device's
own inputs to that stage:
- embedding rows: exact against dequantize_q4_0 of the row;
- draft-head input: exact, h_prev plus the previous token's embedding (the
  embedding alone when self-drafting);
- stack and draft MoE layer: within 1e-3 (backend/metal/expert.rs:309);
- final norms: within 1e-5;
- LM-head logits: bit-exact (the Q8_K matvec);
- draft token: bit-exact (top-1, or the k = 0 acceptance draw);
- accepted length and emitted tokens: bit-exact.

The statistics and the controller must equal a replay from the accepted
lengths (runtime/mtp.rs:48-83, 112-168)."""
import numpy as np
import pytest

import cpu_oracle as orc
from conftest import rel_err
from stack_oracle import oracle_replay
from turboqwenfare_amd import mtp
from turboqwenfare_amd.mtp_loop import DeviceEngine, MtpLoop, MtpModel
from turboqwenfare_amd.workloads import H

pytestmark = pytest.mark.gpu

LAYERS, VOCAB, K, T = 2, 32768, 3, 0.7


@pytest.fixture(scope="module")
def mtp_model(backend):
    model = MtpModel(backend, LAYERS, VOCAB, seed=3)
    model.emb_host = model.embed_q4_0().reshape(VOCAB, (H // 32) * 18)
    yield model
    model.free()


def emb_rows(model, tokens):
    out = []
    for t in tokens:
        blocks = model.emb_host[t].reshape(H // 32, 18)
        out.append(np.concatenate([orc.dequantize_q4_0(b) for b in blocks]))
    return np.stack(out).astype(np.float32)


def lm_head(model, x):
    return orc.q6_k_matvec(model.lm_head_host, VOCAB, H, x)


def select(row, greedy, u, sampler="fast"):
    if greedy:
        return int(orc.top_logit_candidates(row)[0][0])
    if sampler == "reference":
        return orc.softmax_draw(row, T, float(np.float32(u)))
    _, toks = orc.accept(row[None, :], np.zeros((0, VOCAB), np.float32), [], T, False,
                         np.zeros(0, np.float32), np.array([u], np.float32))
    return toks[0]


def check_target_pass(model, tr):
    toks = tr["tokens"]
    assert np.array_equal(tr["hin"], emb_rows(model, toks)), "embedding rows"
    h, _, _ = oracle_replay(model.target, tr["hin"])
    assert rel_err(tr["h"], h) < 1e-3
    hn = np.stack([orc.qwen_rmsnorm(r, model.norm_host) for r in tr["h"]])
    assert rel_err(tr["hn"], hn) < 1e-5
    for i in range(len(toks)):
        assert np.array_equal(tr["target"][i], lm_head(model, tr["hn"][i])), f"target logits row {i}"


@pytest.mark.parametrize("self_draft,greedy,sampler", [
    (False, False, "fast"), (True, False, "fast"), (False, True, "fast"), (True, True, "fast"),
    (False, False, "reference"), (True, False, "reference")],
    ids=["mtp_head-stochastic", "self_draft-stochastic", "mtp_head-greedy", "self_draft-greedy",
         "mtp_head-reference_sampler", "self_draft-reference_sampler"])
def test_mtp_loop_matches_the_oracle_step_by_step(backend, mtp_model, greedy, self_draft, sampler):
    """The draft head's drafts are almost always rejected (its weights are
    unrelated to the target's); self-drafting makes q = p, so drafts are
    accepted and the bonus draw, h_prev at a > 0 and the controller's
    enabling are exercised too.  With the reference sampler every draft and
    plain pick is Sampler::select's token (orc_softmax_draw), the plain picks'
    uniforms from the reference generator seeded with the loop's seed."""
    md = mtp_model
    eng = DeviceEngine(backend, md, k=K, temperature=T, greedy=greedy, seed=5, trace=True,
                       self_draft=self_draft, sampler=sampler)
    loop = MtpLoop(eng, k=K, window=3)
    try:
        recs = loop.run(1234, 6)
    finally:
        eng.free()
    r0 = recs[0]
    check_target_pass(md, r0.trace)
    assert r0.emitted == [select(r0.trace["target"][0], greedy, r0.trace["u_select"], sampler)]
    if sampler == "reference":
        assert np.float32(r0.trace["u_select"]) == np.float32(orc.Xoshiro(5).next_f32())
    prev_h, boundary = r0.trace["h"][0], r0.emitted[0]
    stats, ctl = mtp.MtpStatistics(), mtp.MtpController(3)
    for s, r in enumerate(recs[1:]):
        tr = r.trace
        if r.speculative:
            # the draft head, token by token
            prev = boundary
            stack, norm = (md.target, md.norm_host) if self_draft else (md.draft, md.draft_norm_host)
            for i in range(K):
                x_want = emb_rows(md, [prev])[0]
                if not self_draft:
                    x_want = (prev_h if i == 0 else tr["draft_y"][i - 1]) + x_want
                assert np.array_equal(tr["draft_x"][i], x_want.astype(np.float32)), (s, i)
                y, _, _ = oracle_replay(stack, tr["draft_x"][i][None, :])
                assert rel_err(tr["draft_y"][i], y[0]) < 1e-3
                yn = orc.qwen_rmsnorm(tr["draft_y"][i], norm)
                assert rel_err(tr["draft_yn"][i], yn) < 1e-5
                assert np.array_equal(tr["draft"][i], lm_head(md, tr["draft_yn"][i])), (s, i)
                d = select(tr["draft"][i], greedy, float(tr["ud"][i]), sampler)
                assert d == tr["drafts"][i], (s, i)
                prev = d
            # the verify pass and the acceptance
            assert tr["tokens"] == [boundary] + tr["drafts"]
            check_target_pass(md, tr)
            want = orc.accept(tr["target"], None if greedy else tr["draft"], tr["drafts"], T,
                              greedy, None if greedy else tr["u"], None if greedy else tr["ur"])
            assert (r.accepted, r.emitted) == want, f"step {s}"
            prev_h = tr["h"][r.accepted]
            stats.record_verify(K, r.accepted)
            assert ctl.record_and_decide(r.accepted + 1) == r.enabled
        else:
            check_target_pass(md, tr)
            assert r.emitted == [select(tr["target"][0], greedy, tr["u_select"], sampler)]
            prev_h = tr["h"][0]
        boundary = r.emitted[-1]
    assert stats == loop.stats
    assert ctl.enabled == loop.controller.enabled
    accepted = [r.accepted for r in recs[1:] if r.speculative]
    print(f"{'greedy' if greedy else 'stochastic'} {'self' if self_draft else 'head'}: accepted "
          f"{accepted}, speculative {[r.speculative for r in recs[1:]]}, "
          f"enabled {loop.controller.enabled}")
    if self_draft:
        assert max(accepted) > 0 and loop.controller.enabled
