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
this depth.  It also replays the stack with only the device's activation
rounding (replay_device_model: every matvec input as its 22-bit block
records) and records that replay's distance from the oracle
(``*_device_records``): tests/test_gpu_stack40.py bounds the GPU's error by
it plus twice the every-layer spread.

The Q4_K stack (workloads.SyntheticQ4KStack, whose expert bytes are host
generated) is chaotic at this depth: the Q8_K quantization of every matvec
input (weights.rs:898-931) turns a rounding-level change of its input into
whole quantization steps, and the oracle's own routes change within 5-16
layers under the same noise.  For it the script records, per trial, the
first layer whose routes differ from the unperturbed replay
(``q4k_m<M>_first_flip``, ``q4k_m<M>_every_layer_first_flip``) and the
distance at layer 40; no implementation that rounds differently from the
oracle can be compared with it end to end, so tests/test_gpu_stack40_q4k.py
checks the device layer by layer instead.  CPU only, a few minutes:

    python tests/golden/make_stack40_spread.py          # everything
    python tests/golden/make_stack40_spread.py --q4k    # the Q4_K entries only (merged)
"""
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path[:0] = [str(HERE.parent.parent), str(HERE.parent), str(HERE.parent.parent / "oracle")]

from conftest import rel_err  # noqa: E402
from stack_oracle import OneLayer, oracle_replay  # noqa: E402
from turboqwenfare_amd import synth  # noqa: E402
from turboqwenfare_amd.workloads import (E, F, H, expert_tensor_ids, layer_host_f32,  # noqa: E402
                                         q4k_layer_host_f32, q4k_matrices, q4k_matrix_index)

E_SHARED = E  # the shared expert's index in a layer's expert table

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


class HostQ4KStack:
    """The SyntheticQ4KStack's tensors on the host (oracle_replay's interface)."""

    fmt = "q4_k"

    def __init__(self, n_layers):
        self.n_layers = n_layers
        self.host_f32 = [q4k_layer_host_f32(l) for l in range(n_layers)]
        self.host_q4k = q4k_matrices(0)

    def expert_q4_k(self, l, e):
        return tuple(self.host_q4k[i][q4k_matrix_index(l, e, i)] for i in range(3))


def replay_noisy(st, h0, seed):
    """oracle_replay with rounding-level noise injected into h before every
    layer (the model of an implementation that rounds differently from the
    oracle at every layer), returning (h, routes)."""
    rng = np.random.default_rng(seed)
    h = np.array(h0, np.float32)
    routes = []
    for l in range(st.n_layers):
        h = (h * (1 + 2.0 ** -24 * rng.standard_normal(h.shape))).astype(np.float32)
        one = OneLayer(st, l)
        h, ids, _ = oracle_replay(one, h)
        routes.append(ids[0])
    return h, np.stack(routes)


def records(v: np.ndarray) -> np.ndarray:
    """The device's activation records of each 32-element block of v
    (turboqwenfare_amd/csrc/tqf_device.h, block_scale and split_digits16):
    with E the binary exponent of the block's largest |v| (blocks below
    2^-100 are zero), every value becomes rint(v / 2^(E-21)) * 2^(E-21) --
    a 22-bit integer of the block's scale."""
    b = np.asarray(v, np.float64).reshape(-1, 32)
    amax = np.abs(b).max(axis=1)
    e = np.where(amax >= 2.0 ** -100, np.floor(np.log2(np.maximum(amax, 2.0 ** -100))) - 21, 0.0)
    step = np.where(amax >= 2.0 ** -100, 2.0 ** e, 0.0)
    q = np.where(step[:, None] > 0, np.rint(b / np.where(step > 0, step, 1.0)[:, None]) * step[:, None], 0.0)
    return q.reshape(np.shape(v))


def q4_0_dense(q: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """GGML Q4_0 bytes -> the exact float64 matrix [rows x cols]."""
    blk = np.asarray(q, np.uint8).reshape(rows, cols // 32, 18)
    d = blk[:, :, 0:2].copy().view(np.float16)[:, :, 0].astype(np.float64)
    qs = blk[:, :, 2:18]
    lo = (qs & 15).astype(np.float64) - 8.0
    hi = (qs >> 4).astype(np.float64) - 8.0
    return (np.concatenate([lo, hi], axis=2) * d[:, :, None]).reshape(rows, cols)


def replay_device_model(st, h0, routes):
    """The persistent kernel's arithmetic with only its activation rounding
    kept: per layer, y = h * w_norm (f32), 1/rms from the row's sum of
    squares, gate/up = (1/rms) * (W . records(y)), h_ffn = silu(gate) * up,
    down = W_d . records(h_ffn), the shared pair scaled by sigmoid(gate . x)
    and each route by its weight, h <- f32(h + sum).  Everything else in
    float64, the routes taken from the oracle (the device's are bit-equal at
    every layer), so the distance from the oracle's h is the activation
    records' share of the device's."""
    h = np.array(h0, np.float32)
    m = h.shape[0]
    for l in range(st.n_layers):
        router, gate_vec, norm = st.host_f32[l]
        y = (h * norm).astype(np.float32).astype(np.float64)
        inv = 1.0 / np.sqrt((h.astype(np.float64) ** 2).sum(axis=1) / H + 1e-6)
        ids = routes[l]
        experts = sorted(set(int(v) for v in ids.reshape(-1)))
        dense = {e: [q4_0_dense(mat, r, c) for mat, (r, c) in zip(st.expert_q4_0(l, e), ((F, H), (F, H), (H, F)))]
                 for e in experts + [E_SHARED]}
        xs = np.stack([records(y[t]) for t in range(m)])
        out = np.zeros((m, H))
        logits = (router.astype(np.float64) @ (y * inv[:, None]).T).T  # [m, E]
        for t in range(m):
            def expert(e):
                g, u, dn = dense[e]
                gt, ut = inv[t] * (g @ xs[t]), inv[t] * (u @ xs[t])
                hf = gt / (1.0 + np.exp(-gt)) * ut
                return dn @ records(hf)
            gl = float(gate_vec.astype(np.float64) @ (y[t] * inv[t]))
            acc = expert(E_SHARED) / (1.0 + np.exp(-gl))
            lg = logits[t]
            p = np.exp(lg - lg.max())
            p /= p.sum()
            top = ids[t].astype(int)
            w = p[top] / p[top].sum()
            for k in range(8):
                acc = acc + w[k] * expert(int(top[k]))
            out[t] = acc
        h = (h.astype(np.float64) + out).astype(np.float32)
    return h


def spreads_of(st, h0, ids, h):
    """(input-only spreads, every-layer spreads) of the oracle's 40-layer h."""
    spreads, every = [], []
    for seed in range(TRIALS):
        n = np.random.default_rng(seed).standard_normal(h0.shape)
        hp = (h0 * (1 + 2.0 ** -24 * n)).astype(np.float32)
        h2, ids2, _ = oracle_replay(st, hp)
        assert np.array_equal(ids, ids2), "a perturbation changed the routes"
        spreads.append(float(rel_err(h2, h)))
    for seed in range(TRIALS):
        h3, ids3 = replay_noisy(st, h0, 100 + seed)
        assert np.array_equal(ids, ids3), "a perturbation changed the routes"
        every.append(float(rel_err(h3, h)))
    return spreads, every


def first_flip(st, h0, ids, h, seed, every):
    """(first layer whose routes differ from ids, distance from h at the last
    layer) of a replay with the input perturbed (every=False) or with noise
    before every layer (every=True)."""
    rng = np.random.default_rng(seed)
    x = np.array(h0, np.float32)
    if not every:
        x = (x * (1 + 2.0 ** -24 * rng.standard_normal(x.shape))).astype(np.float32)
    first = None
    for l in range(st.n_layers):
        if every:
            x = (x * (1 + 2.0 ** -24 * rng.standard_normal(x.shape))).astype(np.float32)
        x, r, _ = oracle_replay(OneLayer(st, l), x)
        if first is None and not np.array_equal(r[0], ids[l]):
            first = l
    return first, float(rel_err(x, h))


def q4k_entries(out):
    st = HostQ4KStack(LAYERS)
    for m in (4, 1):
        h0 = synth.normal((4, H), seed=1)[:m]
        h, ids, _ = oracle_replay(st, h0)
        for key, every, seeds in (("", False, range(TRIALS)), ("_every_layer", True, range(100, 100 + TRIALS))):
            res = [first_flip(st, h0, ids, h, sd, every) for sd in seeds]
            out[f"q4k_m{m}{key}_first_flip"] = [r[0] for r in res]
            out[f"q4k_m{m}{key}"] = [r[1] for r in res]
            print("q4k", m, key, res, flush=True)


NOISE = ("h * (1 + 2^-24 n), n ~ N(0,1), numpy default_rng(seed): "
         "<recipe>_m<M> on the input only (seeds 0..2), "
         "<recipe>_m<M>_every_layer before every layer (seeds 100..102); "
         "<recipe>_m<M>_device_records: the replay with only the device's 22-bit "
         "block activation records (no noise); q4k_m<M>, q4k_m<M>_every_layer: the same "
         "distances at layer 40 for the Q4_K stack (workloads.SyntheticQ4KStack), whose "
         "routes change under this noise: *_first_flip is the first layer with other routes")


def main():
    path = HERE / "stack40_spread.json"
    if "--q4k" in sys.argv[1:]:
        out = json.loads(path.read_text())
        out["noise"] = NOISE
        q4k_entries(out)
        path.write_text(json.dumps(out, indent=1) + "\n")
        return
    out = {"layers": LAYERS, "noise": NOISE}
    for recipe in ("zero_mean", "uniform"):
        st = HostStack(LAYERS, recipe)
        for m in (4, 1):
            h0 = synth.normal((4, H), seed=1)[:m]
            h, ids, _ = oracle_replay(st, h0)
            spreads, every = spreads_of(st, h0, ids, h)
            out[f"{recipe}_m{m}"] = spreads
            out[f"{recipe}_m{m}_every_layer"] = every
            hd = replay_device_model(st, h0, ids)
            out[f"{recipe}_m{m}_device_records"] = float(rel_err(hd, h))
            print(recipe, m, spreads, every, out[f"{recipe}_m{m}_device_records"], flush=True)
        st.cache.clear()
    q4k_entries(out)
    path.write_text(json.dumps(out, indent=1) + "\n")


if __name__ == "__main__":
    main()
