"""Host oracle of a resident SyntheticStack: h <- h + MoE_l(rmsnorm_l(h)) per
layer (model/qwen36/runtime.rs:777-802, experts/mod.rs:1540-1577), each
layer's host copy holding only the experts the oracle's own routes use (plus
the shared one), downloaded from the device."""
import os

import numpy as np

import cpu_oracle as orc
from turboqwenfare_amd.workloads import E, F, H

THREADS = max(1, min(16, len(os.sched_getaffinity(0))))


def oracle_replay(model, h0: np.ndarray, inputs: list | None = None):
    """(h [m, H], route ids [L, m, 8], route weights [L, m, 8]) of the stack over h0 [m, H];
    `inputs`, when given, receives each layer's input h."""
    h = np.array(h0, dtype=np.float32, copy=True)
    m = h.shape[0]
    blank = np.zeros(F * (H // 32) * 18, np.uint8)  # gate/up and down have the same byte size
    routes, weights = [], []
    for l in range(model.n_layers):
        if inputs is not None:
            inputs.append(h.copy())
        router, gate, norm = model.host_f32[l]
        xn = np.stack([orc.qwen_rmsnorm(h[t], norm) for t in range(m)])
        ids = np.stack([orc.router_from_logits(orc.f32_matvec(router, xn[t]))[0] for t in range(m)])
        g, u, d = [blank] * E, [blank] * E, [blank] * E
        for e in sorted(set(int(v) for v in ids.reshape(-1))):
            g[e], u[e], d[e] = model.expert_q4_0(l, e)
        host = orc.MoeLayerHost(router, gate, *model.expert_q4_0(l, E), g, u, d)
        y, ids2, w = host.forward_batch(xn, nthreads=THREADS)
        assert np.array_equal(ids, ids2)
        h = (h + y).astype(np.float32)
        routes.append(ids2)
        weights.append(w)
    return h, np.stack(routes), np.stack(weights)
