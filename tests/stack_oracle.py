"""Host oracle of a resident SyntheticStack: h <- h + MoE_l(rmsnorm_l(h)) per
layer (model/qwen36/runtime.rs:777-802, experts/mod.rs:1540-1577), each
layer's host copy holding only the experts the oracle's own routes use (plus
the shared one): for Q4_0 downloaded from the device, for Q4_K the host
bytes the device repacked."""
import os

import numpy as np

import cpu_oracle as orc
from turboqwenfare_amd.workloads import E, F, H

THREADS = max(1, min(16, len(os.sched_getaffinity(0))))


def oracle_moe(model, l: int, xn: np.ndarray):
    """(y [m, H], route ids [m, 8], route weights [m, 8]) of layer l's MoE
    block on the normalised rows xn (experts/mod.rs:1540-1577), the layer's
    host copy holding the experts the oracle's own routes use."""
    # the expert matrices' format: Q4_0 (SyntheticStack) or Q4_K (SyntheticQ4KStack)
    fmt = getattr(model, "fmt", "q4_0")
    expert = model.expert_q4_k if fmt == "q4_k" else model.expert_q4_0
    # an unused expert: zero bytes (every value 0); gate/up and down have the
    # same byte size, 589,824 B in both formats at these shapes
    blank = np.zeros(F * (H // 32) * 18, np.uint8)
    assert blank.size == F * (H // 256) * 144
    router, gate, _ = model.host_f32[l]
    ids = np.stack([orc.router_from_logits(orc.f32_matvec(router, x))[0] for x in xn])
    g, u, d = [blank] * E, [blank] * E, [blank] * E
    for e in sorted(set(int(v) for v in ids.reshape(-1))):
        g[e], u[e], d[e] = expert(l, e)
    host = orc.MoeLayerHost(router, gate, *expert(l, E), g, u, d, fmt=fmt)
    y, ids2, w = host.forward_batch(xn, nthreads=THREADS)
    assert np.array_equal(ids, ids2)
    return y, ids2, w


def oracle_norm(model, l: int, h: np.ndarray) -> np.ndarray:
    """Layer l's RMSNorm of the rows of h (weights.rs:216-239)."""
    norm = model.host_f32[l][2]
    return np.stack([orc.qwen_rmsnorm(row, norm) for row in h])


def oracle_replay(model, h0: np.ndarray, inputs: list | None = None):
    """(h [m, H], route ids [L, m, 8], route weights [L, m, 8]) of the stack over h0 [m, H];
    `inputs`, when given, receives each layer's input h."""
    h = np.array(h0, dtype=np.float32, copy=True)
    routes, weights = [], []
    for l in range(model.n_layers):
        if inputs is not None:
            inputs.append(h.copy())
        y, ids, w = oracle_moe(model, l, oracle_norm(model, l, h))
        h = (h + y).astype(np.float32)
        routes.append(ids)
        weights.append(w)
    return h, np.stack(routes), np.stack(weights)


class OneLayer:
    """Layer l of a stack model (SyntheticStack, SyntheticQ4KStack or a host
    copy of either) as a one-layer model for oracle_replay."""

    def __init__(self, model, l):
        self.model, self.l, self.n_layers = model, l, 1
        self.host_f32 = [model.host_f32[l]]
        self.fmt = getattr(model, "fmt", "q4_0")

    def expert_q4_0(self, _, e):
        return self.model.expert_q4_0(self.l, e)

    def expert_q4_k(self, _, e):
        return self.model.expert_q4_k(self.l, e)
