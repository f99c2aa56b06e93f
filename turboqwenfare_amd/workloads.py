"""The benchmark configurations' synthetic models resident in HBM.

No reference counterpart: the reference runs real checkpoints, while the
MI355X configurations are defined on seeded synthetic weights.  A stack of
MoE layers here is what ``Qwen36Runtime`` walks per token
(model/qwen36/runtime.rs:777-802): per layer an fp32 router [E x H], the
shared-expert input gate [H], the RMSNorm weight [H], and E + 1 experts of
Q4_0 gate/up [F x H] and down [H x F] matrices.

Seeding (kept from the first benchmark definition, so its numbers stay
reproducible): layer l has base = 1,000,000 (l + 1); expert e's gate / up /
down are tensor ids base + 3e, base + 3e + 1, base + 3e + 2 (e = E is the
shared expert); the router is N(0, 1/H) from numpy seed base + 7, the shared
input gate N(0, 1/H) from base + 8, the norm weight 1 + 0.05 N(0, 1) from
base + 9.
"""
from __future__ import annotations

import numpy as np

from . import synth

E, H, F = 256, 2048, 512


def layer_host_f32(layer: int, hidden: int = H, experts: int = E):
    """(router [E x H], shared input gate [H], norm weight [H]) of a layer."""
    base = 1_000_000 * (layer + 1)
    router = synth.normal((experts, hidden), seed=base + 7, std=hidden ** -0.5)
    gate = synth.normal((hidden,), seed=base + 8, std=hidden ** -0.5)
    norm = (1.0 + 0.05 * synth.normal((hidden,), seed=base + 9)).astype(np.float32)
    return router, gate, norm


def expert_tensor_ids(layer: int, expert: int) -> tuple[int, int, int]:
    base = 1_000_000 * (layer + 1)
    return base + 3 * expert, base + 3 * expert + 1, base + 3 * expert + 2


class SyntheticStack:
    """n_layers seeded Q4_0 MoE layers generated in HBM (device synth), with
    the f32 host tensors kept for checks; ``recipe`` is the nibble recipe of
    every expert matrix ("uniform" or "zero_mean", ``synth.q4_0_synthetic``)."""

    def __init__(self, be, n_layers: int, seed: int = 0, recipe: str = "zero_mean",
                 log=None, first_layer: int = 0):
        self.be, self.n_layers, self.seed, self.recipe = be, n_layers, seed, recipe
        self.layers, self.norms, self.mats, self.host_f32 = [], [], [], []
        for l in range(first_layer, first_layer + n_layers):
            mats = []
            for e in range(E + 1):
                tg, tu, td = expert_tensor_ids(l, e)
                mats.append((be.synth_q4_0(F, H, tg, seed, recipe),
                             be.synth_q4_0(F, H, tu, seed, recipe),
                             be.synth_q4_0(H, F, td, seed, recipe)))
            router, gate, norm = layer_host_f32(l)
            self.layers.append(be.prepare_moe_layer(
                be.upload_f32(router), be.upload_f32(gate), mats[E], [m[0] for m in mats[:E]],
                [m[1] for m in mats[:E]], [m[2] for m in mats[:E]]))
            self.norms.append(be.upload_f32(norm))
            self.mats.append(mats)
            self.host_f32.append((router, gate, norm))
            if log and (l - first_layer + 1) % 10 == 0:
                log(f"{l - first_layer + 1}/{n_layers} layers resident")
        self.stack = be.prepare_stack(self.layers, self.norms)

    # layer indices below are positions in this stack (0 .. n_layers - 1)
    def expert_q4_0(self, layer: int, expert: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        """GGML Q4_0 bytes of one expert's gate, up and down (device download)."""
        return tuple(self.be.download_q4_0(w) for w in self.mats[layer][expert])

    def free(self) -> None:
        be = self.be
        be.free_stack(self.stack)
        for L in self.layers:
            be.free_moe_layer(L)
            be.free_tensor(L.owned[0])  # router
            be.free_tensor(L.owned[1])  # shared input gate
        for t in self.norms:
            be.free_tensor(t)
        for mats in self.mats:
            for m in mats:
                for w in m:
                    be.free_weights(w)
        self.layers, self.norms, self.mats = [], [], []


# ---- Q4_K experts (the canonical checkpoint's expert format) ---------------------
# Layer l has base = 3,000,000 (l + 1): router N(0, 1/H) from seed base + 7,
# shared input gate from base + 8, norm weight 1 + 0.05 N(0, 1) from base + 9.
# The experts share 8 seeded centred GGML Q4_K matrices per shape
# (synth.centered_q4_k, seed 1000 seed + 10 i + j for shape i = gate, up,
# down): expert e of layer l takes matrix (5 l + 3 e + i) mod 8 of shape i,
# each at its own HBM address (a device repack of the GGML bytes).
Q4K_SHAPES = ((F, H), (F, H), (H, F))


def q4k_layer_host_f32(layer: int, hidden: int = H, experts: int = E):
    """(router [E x H], shared input gate [H], norm weight [H]) of a Q4_K layer."""
    base = 3_000_000 * (layer + 1)
    router = synth.normal((experts, hidden), seed=base + 7, std=hidden ** -0.5)
    gate = synth.normal((hidden,), seed=base + 8, std=hidden ** -0.5)
    norm = (1.0 + 0.05 * synth.normal((hidden,), seed=base + 9)).astype(np.float32)
    return router, gate, norm


def q4k_matrices(seed: int = 0) -> list[list[np.ndarray]]:
    """The 8 GGML Q4_K matrices of each shape (gate, up, down)."""
    return [[synth.centered_q4_k(r, c, seed * 1000 + 10 * i + j) for j in range(8)]
            for i, (r, c) in enumerate(Q4K_SHAPES)]


def q4k_matrix_index(layer: int, expert: int, shape: int) -> int:
    return (layer * 5 + expert * 3 + shape) % 8


class SyntheticQ4KStack:
    """n_layers MoE layers with Q4_K experts resident in HBM (every expert
    matvec on the Q8_K integer path), with the host tensors kept for checks;
    the same seeds as the Q4_K verify-step benchmark."""

    fmt = "q4_k"

    def __init__(self, be, n_layers: int, seed: int = 0, log=None):
        self.be, self.n_layers, self.seed = be, n_layers, seed
        self.host_q4k = q4k_matrices(seed)
        staging = [[be.to_device(q) for q in row] for row in self.host_q4k]
        self.layers, self.norms, self.weights, self.host_f32 = [], [], [], []
        try:
            for l in range(n_layers):
                mats = [tuple(be.upload_q4_k_device(staging[i][q4k_matrix_index(l, e, i)], r, c)
                              for i, (r, c) in enumerate(Q4K_SHAPES)) for e in range(E + 1)]
                self.weights += [w for m in mats for w in m]
                router, gate, norm = q4k_layer_host_f32(l)
                self.layers.append(be.prepare_moe_layer(
                    be.upload_f32(router), be.upload_f32(gate), mats[E], [m[0] for m in mats[:E]],
                    [m[1] for m in mats[:E]], [m[2] for m in mats[:E]]))
                self.norms.append(be.upload_f32(norm))
                self.host_f32.append((router, gate, norm))
                if log and (l + 1) % 10 == 0:
                    log(f"{l + 1}/{n_layers} Q4_K layers resident")
        finally:
            for b in (b for row in staging for b in row):
                be.free(b)
        self.stack = be.prepare_stack(self.layers, self.norms)

    def expert_q4_k(self, layer: int, expert: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        """GGML Q4_K bytes of one expert's gate, up and down (host copies)."""
        return tuple(self.host_q4k[i][q4k_matrix_index(layer, expert, i)] for i in range(3))

    def free(self) -> None:
        be = self.be
        be.free_stack(self.stack)
        for L in self.layers:
            be.free_moe_layer(L)
            be.free_tensor(L.owned[0])  # router
            be.free_tensor(L.owned[1])  # shared input gate
        for t in self.norms:
            be.free_tensor(t)
        for w in self.weights:
            be.free_weights(w)
