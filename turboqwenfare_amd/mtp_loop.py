"""The MTP decode loop on the HIP backend: draft k tokens with the draft head,
verify them with the target stack, accept, account, and let the controller
switch speculation on and off.

The reference has the accounting and the controller, but no loop that
drives them: ``MtpStatistics`` (runtime/mtp.rs:48-83) and ``MtpController``
(runtime/mtp.rs:112-168) are never fed from a verify pass. Its MTP sidecar
(source/pinned.rs:24-38, a Q4_0 module) is never executed. One token of
the target is ``Qwen36Runtime::decode_step`` (model/qwen36/runtime.rs:
386-450): the embedding row, the layers, the final norm, the Q6_K LM head and
the selection.

Every stage here is a HIP entry point, and the state stays on the device
between stages:

- target pass: ``h = stack(embed(token))`` for each verify row, then the
  final rmsnorm and the LM head (``tqf_hip_embed_rows_device``,
  ``tqf_hip_stack_forward_device``, ``tqf_hip_rmsnorm_rows_device``,
  ``tqf_hip_lm_head_logits_device``);
- draft head: ``x = h_prev + embed(d_prev)``, then ``x += MoE_mtp(rmsnorm(x))``
  (one Q4_0 MoE layer, the sidecar's FFN), then its final norm and the shared
  LM head. This build has no attention at all, so each verify row is computed
  from its own token, and the draft head's attention and its
  embedding/hidden projection are out of scope. The sum stands in for that
  projection;
- selection: greedy takes the LM head's fused top-1
  (``top_logit_candidates``). Stochastic, with ``sampler="fast"`` (the
  default), makes one draw from E_x / S of the row: the acceptance kernel at
  k = 0 with one uniform (exact fixed-point sums, microseconds). With
  ``sampler="reference"`` it is ``Sampler::select`` bit for bit
  (``tqf_hip_sampler_select_device``: f32::exp, the token-order f32 total,
  the stable sort, the inverse-CDF walk; about a millisecond per pick), and
  the plain-decode picks take their uniforms from a ``Sampler`` seeded with
  the loop's seed (Xoshiro256PlusPlus::from_seed, one next_f32 per pick), as
  the reference's generation loop does: a loop that never speculates then
  emits the reference's token stream for the same logits;
- verification: ``tqf_hip_accept_device`` over the k + 1 target rows and the
  k draft rows.

Policy for the controller (the reference leaves it open). Speculation runs
while the controller is enabled, and also during its warm-up, before the
window has filled for the first time: the controller starts disabled and can
only enable on evidence. Once the window has filled and the controller is
disabled, steps decode one token without drafts and feed nothing to it, so
it stays off. Each speculative step records ``k`` drafts and ``accepted + 1``
emitted tokens for one target pass (``MtpStatistics.record_verify``), and
feeds ``accepted + 1`` to ``record_and_decide``. Under the reference's net
benefit (emitted - 1), a verify pass never counts below 0. The -0.05 disable
threshold is therefore reached only by outcomes that emit nothing, which no
pass of this loop produces.

The uniforms are Philox draws keyed by (seed + step, stream):
- stream 0: acceptance;
- stream 1: resample;
- stream 2: draft draws;
- stream 3: plain-decode draws;
- stream 4: the first token's draw (keyed by the seed alone).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import mtp, synth
from .backend import DeviceBuffer
from .sampling import Sampler
from .workloads import H, SyntheticStack

EMBED_TENSOR = 2_000_000_000
DRAFT_FIRST_LAYER = 999  # the draft head's MoE layer ids: base 1,000,000,000


def q6k_synthetic(rows: int, cols: int, seed: int) -> np.ndarray:
    """Seeded GGML Q6_K bytes [rows x cols/256 x 210]: random quants and
    scales, and a small positive f16 d per super-block (as the LM head bench
    draws them)."""
    rng = np.random.default_rng(seed)
    n = rows * (cols // 256)
    blk = rng.integers(0, 256, size=(n, 210), dtype=np.uint8)
    blk[:, 208:210] = rng.uniform(0.001, 0.05, n).astype(np.float16).view(np.uint8).reshape(n, 2)
    return blk.reshape(-1)


class MtpModel:
    """The resident pieces of the loop:
    - the target stack (``n_layers`` seeded Q4_0 MoE layers);
    - the draft head's MoE layer;
    - a Q4_0 embedding [vocab x H];
    - the target and draft final-norm weights;
    - one Q6_K LM head [vocab x H] shared by both passes.

    The host copies the oracle needs are kept as well."""

    def __init__(self, be, n_layers: int, vocab: int, seed: int = 0, recipe: str = "zero_mean",
                 log=None):
        self.be, self.vocab, self.seed = be, vocab, seed
        self.target = SyntheticStack(be, n_layers, seed=seed, recipe=recipe, log=log)
        self.draft = SyntheticStack(be, 1, seed=seed, recipe=recipe, first_layer=DRAFT_FIRST_LAYER)
        self.embed = be.synth_q4_0(vocab, H, EMBED_TENSOR, seed, recipe)
        self.norm_host = (1.0 + 0.05 * synth.normal((H,), seed=seed + 11)).astype(np.float32)
        self.draft_norm_host = (1.0 + 0.05 * synth.normal((H,), seed=seed + 12)).astype(np.float32)
        self.norm = be.upload_f32(self.norm_host)
        self.draft_norm = be.upload_f32(self.draft_norm_host)
        self.lm_head_host = q6k_synthetic(vocab, H, seed + 13)
        self.lm_head = be.upload_q6_k(self.lm_head_host, vocab, H)

    def embed_q4_0(self) -> np.ndarray:
        """GGML Q4_0 bytes of the embedding (device download)."""
        return self.be.download_q4_0(self.embed)

    def free(self) -> None:
        be = self.be
        self.target.free()
        self.draft.free()
        be.free_weights(self.embed)
        be.free_tensor(self.norm)
        be.free_tensor(self.draft_norm)
        be.free_weights(self.lm_head)


@dataclass
class StepRecord:
    """One loop step: the tokens it emitted, how many drafts were accepted
    (-1 on a step without drafts), and the controller state after it."""

    emitted: list
    accepted: int
    speculative: bool
    enabled: bool
    trace: dict = field(default_factory=dict)


class MtpLoop:
    """The loop's policy and accounting over an engine that runs the passes
    (``DeviceEngine`` on the HIP backend):
    - ``engine.start(token)`` -> (first token, trace);
    - ``engine.plain(step, boundary)`` -> (token, trace);
    - ``engine.speculative(step, boundary)`` -> (emitted tokens, accepted, trace).
    See the module docstring for the policy."""

    def __init__(self, engine, k: int = 3, window: int = 8):
        if not 1 <= k <= 7:
            raise ValueError("k must be in 1..7")
        self.engine, self.k = engine, k
        self.stats = mtp.MtpStatistics()
        self.controller = mtp.MtpController(window)
        self.step_index = 0
        self.boundary = None  # the last emitted token

    def speculating(self) -> bool:
        """Speculate while enabled, and while the window has not yet filled."""
        c = self.controller
        return c.enabled or len(c.window) < c.window_capacity

    def start(self, token: int) -> StepRecord:
        t, trace = self.engine.start(token)
        self.boundary = t
        return StepRecord([t], -1, False, self.controller.enabled, trace)

    def step(self) -> StepRecord:
        if self.boundary is None:
            raise RuntimeError("call start(token) first")
        s = self.step_index
        self.step_index += 1
        if not self.speculating():
            t, trace = self.engine.plain(s, self.boundary)
            self.boundary = t
            return StepRecord([t], -1, False, self.controller.enabled, trace)
        emitted, a, trace = self.engine.speculative(s, self.boundary)
        self.boundary = emitted[-1]
        self.stats.record_verify(self.k, a)
        enabled = self.controller.record_and_decide(a + 1)
        return StepRecord(emitted, a, True, enabled, trace)

    def run(self, token: int, steps: int) -> list:
        """start(token), then `steps` steps; the records of all of them."""
        out = [self.start(token)]
        for _ in range(steps):
            out.append(self.step())
        return out


class DeviceEngine:
    """The passes of the loop as HIP entry points, state resident on the
    device between them. ``trace=True`` keeps host copies of every stage's
    inputs and outputs; the tests check them stage by stage.
    ``self_draft=True`` drafts with the target itself: ``x = embed(d_prev)``
    through the target stack and norm. The draft distribution is then the
    target's, and drafts are accepted, which exercises the accepting half of
    the loop."""

    def __init__(self, be, model: MtpModel, k: int = 3, temperature: float = 0.7,
                 greedy: bool = False, seed: int = 0, trace: bool = False,
                 self_draft: bool = False, sampler: str = "fast"):
        if sampler not in ("fast", "reference"):
            raise ValueError("sampler must be 'fast' or 'reference'")
        self.be, self.model, self.k, self.T, self.greedy = be, model, k, temperature, greedy
        self.seed, self.trace_on, self.self_draft = seed, trace, self_draft
        self.sampler = sampler
        # the plain-decode picks' Sampler (reference mode): Sampler::new's
        # generator, seeded once per generation
        self.ref_sampler = Sampler(be, temperature, seed) if sampler == "reference" and not greedy else None
        V, m, L = model.vocab, k + 1, max(model.target.n_layers, 1)
        self.d_tok = be.alloc(4 * m)
        self.d_hin, self.d_h, self.d_hn = (be.alloc(4 * m * H) for _ in range(3))
        self.d_target = be.alloc(4 * m * V)
        self.d_draft = be.alloc(4 * k * V)
        self.d_x, self.d_xn, self.d_hprev = be.alloc(4 * H), be.alloc(4 * H), be.alloc(4 * H)
        self.d_t4, self.d_l4 = be.alloc(16 * m), be.alloc(16 * m)
        self.d_ids, self.d_w = be.alloc(2 * 8 * m * L), be.alloc(4 * 8 * m * L)
        self.d_status = be.alloc(4)
        self.d_sel_u, self.d_sel_acc, self.d_sel_tok = be.alloc(4), be.alloc(4), be.alloc(4 * m)
        # a speculative step's host traffic, one write and one read: the verify
        # rows' tokens (boundary, then the drafts as the device picks them),
        # the uniforms u [k], ur [k + 1], ud [k], then the acceptance's outputs
        # (accepted length, emitted tokens [k + 1])
        self.io_words = (k + 1) + k + (k + 1) + k + 1 + (k + 1)
        self.d_io = be.alloc(4 * self.io_words)
        be.write(self.d_status, np.zeros(1, np.int32))

    # ---- stages ------------------------------------------------------------------------
    def _check_status(self) -> None:
        st = int(self.be.read(self.d_status, np.int32, (1,))[0])
        if st != 0:
            raise RuntimeError(f"device status {st} in the MTP loop")

    def _target_pass(self, tokens: list) -> None:
        """d_h <- stack(embed(tokens)); d_hn <- rmsnorm; d_target <- LM head."""
        be, md, n = self.be, self.model, len(tokens)
        be.write(self.d_tok, np.asarray(tokens, np.int32))
        be.embed_rows_device(md.embed, self.d_tok, n, self.d_hin, d_status=self.d_status)
        be.copy_device(self.d_h, self.d_hin, 4 * n * H)
        be.stack_forward_device(md.target.stack, self.d_h, n, self.d_ids, self.d_w, self.d_status)
        be.rmsnorm_rows_device(self.d_h, n, H, md.norm, self.d_hn)
        be.lm_head_logits_device(md.lm_head, self.d_hn, n, self.d_target, self.d_t4, self.d_l4)

    def _pick(self, d_logits: DeviceBuffer, row: int, uniform: float) -> int:
        """One token from logits row `row` of the last LM head call: its
        fused top-1 (greedy), or a draw with one uniform (the acceptance at
        k = 0, whose draft pointer is unused; or Sampler::select)."""
        be, V = self.be, self.model.vocab
        if self.greedy:
            return int(be.read(self.d_t4, np.uint32, (row + 1, 4))[row, 0])
        d_row = be.view(d_logits, 4 * row * V, 4 * V)
        be.write(self.d_sel_u, np.array([uniform], np.float32))
        if self.sampler == "reference":
            be.sampler_select_device(d_row, 1, V, self.T, self.d_sel_u, self.d_sel_tok)
        else:
            be.accept_device(d_row, d_row, self.d_tok, 0, V, self.T, False, self.d_sel_u,
                             self.d_sel_u, self.d_sel_acc, self.d_sel_tok)
        return int(be.read(self.d_sel_tok, np.int32, (1,))[0])

    def _plain_uniform(self, stream: int, step) -> float:
        """The plain pick's uniform: the reference Sampler's next_f32, or a
        Philox draw keyed by (seed + step, stream)."""
        if self.ref_sampler is not None:
            return float(self.ref_sampler.rng.next_f32())
        key = self.seed if step is None else self.seed + step
        return float(synth.philox_uniforms(key, stream, 1)[0])

    def _snap(self, buf, shape) -> np.ndarray:
        return self.be.read(buf, np.float32, shape).copy()

    def _plain_trace(self, tokens, u) -> dict:
        if not self.trace_on:
            return {}
        n, V = len(tokens), self.model.vocab
        return dict(tokens=list(tokens), hin=self._snap(self.d_hin, (n, H)),
                    h=self._snap(self.d_h, (n, H)), hn=self._snap(self.d_hn, (n, H)),
                    target=self._snap(self.d_target, (n, V)), u_select=u)

    # ---- the passes ----------------------------------------------------------------------
    def start(self, token: int):
        """A plain decode of the prompt's last token."""
        if not 0 <= token < self.model.vocab:
            raise ValueError("token out of vocabulary")
        u = self._plain_uniform(4, None)
        return self.plain(None, token, u)

    def plain(self, step, boundary: int, u: float | None = None):
        """One token without drafts; its hidden row becomes h_prev."""
        if u is None:
            u = self._plain_uniform(3, step)
        self._target_pass([boundary])
        t = self._pick(self.d_target, 0, u)
        self._check_status()
        self.be.copy_device(self.d_hprev, self.d_h, 4 * H)
        return t, self._plain_trace([boundary], u)

    def _io(self, word: int, n: int = 1) -> DeviceBuffer:
        return self.be.view(self.d_io, 4 * word, 4 * n)

    def speculative(self, step: int, boundary: int):
        """Draft k tokens, verify [boundary, drafts], accept.  The drafts are
        picked on the device and feed the next draft's embedding from device
        memory, so the step's only host traffic is one write (tokens and
        uniforms) before it and one read (drafts, acceptance) after it, unless
        tracing."""
        be, md, k, V = self.be, self.model, self.k, self.model.vocab
        u = synth.philox_uniforms(self.seed + step, 0, k)
        ur = synth.philox_uniforms(self.seed + step, 1, k + 1)
        ud = synth.philox_uniforms(self.seed + step, 2, k)
        w_tok, w_u, w_ur, w_ud = 0, k + 1, 2 * k + 1, 3 * k + 2
        w_acc, w_toks = 4 * k + 2, 4 * k + 3
        io = np.zeros(w_acc, np.uint32)
        io[w_tok] = boundary
        io[w_u:w_u + k] = u.view(np.uint32)
        io[w_ur:w_ur + k + 1] = ur.view(np.uint32)
        io[w_ud:w_ud + k] = ud.view(np.uint32)
        be.write(self.d_io, io)
        trace = dict(draft_x=[], draft_y=[], draft_yn=[]) if self.trace_on else {}
        # draft: x = h_prev + embed(d_prev); x += MoE_mtp(rmsnorm(x)); logits
        stack, norm = (md.target, md.norm) if self.self_draft else (md.draft, md.draft_norm)
        be.copy_device(self.d_x, self.d_hprev, 4 * H)
        for i in range(k):
            be.embed_rows_device(md.embed, self._io(w_tok + i), 1, self.d_x,
                                 d_add=None if self.self_draft else self.d_x, d_status=self.d_status)
            if self.trace_on:
                trace["draft_x"].append(self._snap(self.d_x, (H,)))
            be.stack_forward_device(stack.stack, self.d_x, 1, self.d_ids, self.d_w, self.d_status)
            be.rmsnorm_rows_device(self.d_x, 1, H, norm, self.d_xn)
            d_row = be.view(self.d_draft, 4 * i * V, 4 * V)
            be.lm_head_logits_device(md.lm_head, self.d_xn, 1, d_row, self.d_t4, self.d_l4)
            if self.trace_on:
                trace["draft_y"].append(self._snap(self.d_x, (H,)))
                trace["draft_yn"].append(self._snap(self.d_xn, (H,)))
            # the draft token, into the verify rows: the fused top-1, or one
            # draw (the acceptance at k = 0 with its uniform ud[i])
            if self.greedy:
                be.copy_device(self._io(w_tok + 1 + i), be.view(self.d_t4, 0, 4), 4)
            elif self.sampler == "reference":
                be.sampler_select_device(d_row, 1, V, self.T, self._io(w_ud + i), self._io(w_tok + 1 + i))
            else:
                d_ud = self._io(w_ud + i)
                be.accept_device(d_row, d_row, self._io(w_tok), 0, V, self.T, False, d_ud, d_ud,
                                 self.d_sel_acc, self.d_sel_tok)
                be.copy_device(self._io(w_tok + 1 + i), be.view(self.d_sel_tok, 0, 4), 4)
        # verify and accept
        self._target_pass_device(self._io(w_tok, k + 1), k + 1)
        be.accept_device(self.d_target, None if self.greedy else self.d_draft, self._io(w_tok + 1, k),
                         k, V, self.T, self.greedy, None if self.greedy else self._io(w_u, k),
                         None if self.greedy else self._io(w_ur, k + 1), self._io(w_acc),
                         self._io(w_toks, k + 1))
        out = be.read(self.d_io, np.int32, (self.io_words,))
        self._check_status()
        drafts = [int(v) for v in out[w_tok + 1:w_tok + 1 + k]]
        a = int(out[w_acc])
        if a < 0:
            raise RuntimeError("the acceptance kernel reported a timed-out exchange")
        emitted = [int(v) for v in out[w_toks:w_toks + a + 1]]
        if self.trace_on:
            trace.update(self._plain_trace([boundary] + drafts, None))
            trace.update(drafts=drafts, u=u, ur=ur, ud=ud, draft=self._snap(self.d_draft, (k, V)))
        # the hidden row whose prediction produced the last emitted token
        be.copy_device(self.d_hprev, be.view(self.d_h, 4 * a * H, 4 * H), 4 * H)
        return emitted, a, trace

    def _target_pass_device(self, d_tokens: DeviceBuffer, n: int) -> None:
        """_target_pass over tokens already on the device."""
        be, md = self.be, self.model
        be.embed_rows_device(md.embed, d_tokens, n, self.d_hin, d_status=self.d_status)
        be.copy_device(self.d_h, self.d_hin, 4 * n * H)
        be.stack_forward_device(md.target.stack, self.d_h, n, self.d_ids, self.d_w, self.d_status)
        be.rmsnorm_rows_device(self.d_h, n, H, md.norm, self.d_hn)
        be.lm_head_logits_device(md.lm_head, self.d_hn, n, self.d_target, self.d_t4, self.d_l4)

    def free(self) -> None:
        for name, b in list(vars(self).items()):
            if name.startswith("d_"):
                self.be.free(b)
        if self.ref_sampler is not None:
            self.ref_sampler.free()
