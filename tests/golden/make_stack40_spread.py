"""Writes stack40_spread.json: how far the CPU oracle's own 40-layer result
moves when its input moves by rounding-level noise.

The 40-layer verify stack (turboqwenfare_amd/workloads.SyntheticStack) is
replayed by the oracle (tests/stack_oracle.oracle_replay, the reference's
h <- h + MoE_l(rmsnorm_l(h)), model/qwen36/runtime.rs:777-802) from the
benchmark's rows h0 and from h0 * (1 + 2^-24 n), n ~ N(0, 1) (three seeds);
and with the same noise injected before every layer (an implementation
that rounds differently from the oracle at every layer); the expert
matrices come from the host Philox generator
(synth.q4_0_synthetic), the same bytes the device generator writes.  The
spread rel_err(h(h0 perturbed), h(h0)) is the floor below which no
implementation that rounds differently from the oracle can be checked at
this depth: tests/test_gpu_stack40.py bounds the GPU's error by a multiple of
it.  CPU only, a few minutes:

    python tests/golden/make_stack40_spread.py
"""
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path[:0] = [str(HERE.parent.parent), str(HERE.parent), str(HERE.parent.parent / "oracle")]

from conftest import rel_err  # noqa: E402
from stack_oracle import oracle_replay  # noqa: E402
from turboqwenfare_amd import synth  # noqa: E402
from turboqwenfare_amd.workloads import F, H, expert_tensor_ids, layer_host_f32  # noqa: E402

LAYERS, TRIALS = 40, 3


class HostStack:
    """The SyntheticStack's tensors generated on the host (oracle_replay's interface)."""

    def __init__(self, n_layers, recipe):
        self.n_layers, self.recipe = n_layers, recipe
        self.host_f32 = [layer_host_f32(l) for l in range(n_layers)]
        self.cache = {}

    def expert_q4_0(self, l, e):
        if (l, e) not in self.cache:
            tg, tu, td = expert_tensor_ids(l, e)
            self.cache[(l, e)] = (synth.q4_0_synthetic(F, H, tg, 0, self.recipe),
                                  synth.q4_0_synthetic(F, H, tu, 0, self.recipe),
                                  synth.q4_0_synthetic(H, F, td, 0, self.recipe))
        return self.cache[(l, e)]


def replay_noisy(st, h0, seed):
    """oracle_replay with rounding-level noise injected into h before every
    layer (the model of an implementation that rounds differently from the
    oracle at every layer), returning (h, routes)."""
    rng = np.random.default_rng(seed)
    h = np.array(h0, np.float32)
    routes = []
    for l in range(st.n_layers):
        h = (h * (1 + 2.0 ** -24 * rng.standard_normal(h.shape))).astype(np.float32)
        one = _OneLayer(st, l)
        h, ids, _ = oracle_replay(one, h)
        routes.append(ids[0])
    return h, np.stack(routes)


class _OneLayer:
    """Layer l of a HostStack as a one-layer stack."""

    def __init__(self, st, l):
        self.st, self.l, self.n_layers = st, l, 1
        self.host_f32 = [st.host_f32[l]]

    def expert_q4_0(self, _, e):
        return self.st.expert_q4_0(self.l, e)


def main():
    out = {"layers": LAYERS,
           "noise": "h * (1 + 2^-24 n), n ~ N(0,1), numpy default_rng(seed): "
                    "<recipe>_m<M> on the input only (seeds 0..2), "
                    "<recipe>_m<M>_every_layer before every layer (seeds 100..102)"}
    for recipe in ("zero_mean", "uniform"):
        st = HostStack(LAYERS, recipe)
        for m in (4, 1):
            h0 = synth.normal((4, H), seed=1)[:m]
            h, ids, _ = oracle_replay(st, h0)
            spreads = []
            for seed in range(TRIALS):
                n = np.random.default_rng(seed).standard_normal(h0.shape)
                hp = (h0 * (1 + 2.0 ** -24 * n)).astype(np.float32)
                h2, ids2, _ = oracle_replay(st, hp)
                assert np.array_equal(ids, ids2), "a perturbation changed the routes"
                spreads.append(float(rel_err(h2, h)))
            out[f"{recipe}_m{m}"] = spreads
            every = []
            for seed in range(TRIALS):
                h3, ids3 = replay_noisy(st, h0, 100 + seed)
                assert np.array_equal(ids, ids3), "a perturbation changed the routes"
                every.append(float(rel_err(h3, h)))
            out[f"{recipe}_m{m}_every_layer"] = every
            print(recipe, m, spreads, every, flush=True)
        st.cache.clear()
    (HERE / "stack40_spread.json").write_text(json.dumps(out, indent=1) + "\n")


if __name__ == "__main__":
    main()
