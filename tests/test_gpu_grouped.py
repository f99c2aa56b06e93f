"""GPU parity of the prefill grouped expert GEMM (tqf_hip_grouped_gemm, the
routed loop of Qwen36StreamingMoe::forward_batch, experts/mod.rs:1562-1566)
against the CPU oracle's routed accumulate on the same seeded inputs.
Tolerance: |g - c| / max(|c|, 1) < 1e-3 (backend/metal/expert.rs:309-310).
Routes are Zipf(1.1) Gumbel-top-k (config 5) or hand-made edge cases."""
import os

import numpy as np
import pytest

import cpu_oracle as orc
from conftest import rel_err
from turboqwenfare_amd import synth
from turboqwenfare_amd._lib import ERR_INVALID, GROUPED_MAX_TOKENS, HipError

pytestmark = pytest.mark.gpu

FFN_TOL = 1e-3
E = 256
THREADS = min(16, os.cpu_count() or 1)


class _Layer:
    def __init__(self, backend, hidden, width, seed):
        self.be = backend
        self.H, self.F = hidden, width
        self.mats = [(backend.synth_q4_0(width, hidden, 3 * e, seed),
                      backend.synth_q4_0(width, hidden, 3 * e + 1, seed),
                      backend.synth_q4_0(hidden, width, 3 * e + 2, seed)) for e in range(E + 1)]
        router = synth.normal((E, hidden), seed=seed, std=hidden ** -0.5)
        gate = synth.normal((hidden,), seed=seed + 1, std=hidden ** -0.5)
        self.tensors = [backend.upload_f32(router), backend.upload_f32(gate)]
        self.layer = backend.prepare_moe_layer(self.tensors[0], self.tensors[1], self.mats[E],
                                               [m[0] for m in self.mats[:E]],
                                               [m[1] for m in self.mats[:E]],
                                               [m[2] for m in self.mats[:E]])
        host = [[backend.download_q4_0(m) for m in t] for t in self.mats]
        self.oracle = orc.MoeLayerHost(router, gate, *host[E], [h[0] for h in host[:E]],
                                       [h[1] for h in host[:E]], [h[2] for h in host[:E]],
                                       hidden=hidden, width=width)

    def close(self):
        self.be.free_moe_layer(self.layer)
        for t in self.mats:
            for w in t:
                self.be.free_weights(w)
        for t in self.tensors:
            self.be.free_tensor(t)

    def inputs(self, t, seed):
        x = synth.bf16_round(synth.normal((t, self.H), seed=100 + seed))
        ids, w = synth.zipf_routes(t, E, seed=seed)
        return x, ids, w

    def want(self, x_bf16, ids, w):
        return self.oracle.routed_combine(synth.bf16_to_f32(x_bf16), ids, w, nthreads=THREADS)


@pytest.fixture(scope="module")
def small(backend):
    L = _Layer(backend, 256, 256, 21)
    yield L
    L.close()


@pytest.fixture(scope="module")
def model(backend):
    L = _Layer(backend, 2048, 512, 22)
    yield L
    L.close()


@pytest.mark.parametrize("t", [1, 7, 64, 300])
def test_grouped_small_geometry_zipf(backend, small, t):
    x, ids, w = small.inputs(t, t)
    y = backend.grouped_gemm(small.layer, x, ids, w)
    err = rel_err(y, small.want(x, ids, w))
    print(f"t={t} rel err {err:.2e}")
    assert err < FFN_TOL


def test_grouped_config5_model_geometry(backend, model):
    """Config 5: 512 bf16 tokens, Zipf(1.1) top-8 over 256 experts (seed 0)."""
    x, ids, w = model.inputs(512, 0)
    y = backend.grouped_gemm(model.layer, x, ids, w)
    err = rel_err(y, model.want(x, ids, w))
    counts = np.bincount(ids.reshape(-1).astype(np.int64), minlength=E)
    print(f"config 5: {int((counts > 0).sum())} experts, head M {counts.max()}, rel err {err:.2e}")
    assert err < FFN_TOL


def test_grouped_hot_experts_span_many_tiles(backend, model):
    """Every token routed to the same 8 experts: 100 pairs per expert, i.e.
    three full 32-pair tiles and a 4-pair tail per expert."""
    t = 100
    x = synth.bf16_round(synth.normal((t, 2048), seed=7))
    ids = np.tile(np.array([5, 250, 0, 17, 99, 128, 3, 255], np.uint16), (t, 1))
    w = np.tile(np.array([0.3, 0.2, 0.15, 0.1, 0.1, 0.08, 0.05, 0.02], np.float32), (t, 1))
    y = backend.grouped_gemm(model.layer, x, ids, w)
    assert rel_err(y, model.want(x, ids, w)) < FFN_TOL


def test_grouped_max_tokens_small_geometry(backend, small):
    t = GROUPED_MAX_TOKENS
    x, ids, w = small.inputs(t, 3)
    y = backend.grouped_gemm(small.layer, x, ids, w)
    assert rel_err(y, small.want(x, ids, w)) < FFN_TOL


def test_grouped_duplicate_ids_and_zero_weights(backend, small):
    """A token may name one expert twice (each pair is computed) and a zero
    weight contributes exactly nothing."""
    t = 40
    x = synth.bf16_round(synth.normal((t, 256), seed=9))
    rng = np.random.default_rng(9)
    ids = rng.integers(0, 4, size=(t, 8)).astype(np.uint16)
    w = rng.random((t, 8)).astype(np.float32)
    w[:, 3] = 0.0
    y = backend.grouped_gemm(small.layer, x, ids, w)
    assert rel_err(y, small.want(x, ids, w)) < FFN_TOL
    w0 = np.zeros_like(w)
    assert np.array_equal(backend.grouped_gemm(small.layer, x, ids, w0), np.zeros((t, 256), np.float32))


def test_grouped_repeats_are_bit_identical_and_scale_exactly(backend, model):
    x, ids, w = model.inputs(256, 5)
    y1 = backend.grouped_gemm(model.layer, x, ids, w)
    y2 = backend.grouped_gemm(model.layer, x, ids, w)
    assert np.array_equal(y1, y2)
    # w -> 2 w scales every product and sum by a power of two: exact
    y3 = backend.grouped_gemm(model.layer, x, ids, (2 * w).astype(np.float32))
    assert np.array_equal(y3, 2 * y1)


def test_grouped_token_permutation_is_exact(backend, small):
    """Each output row depends only on its own token: permuting the tokens
    (and so the sorted positions inside every expert's tiles) permutes y."""
    x, ids, w = small.inputs(200, 11)
    y = backend.grouped_gemm(small.layer, x, ids, w)
    perm = np.random.default_rng(11).permutation(200)
    yp = backend.grouped_gemm(small.layer, x[perm], ids[perm], w[perm])
    assert np.array_equal(yp, y[perm])


def test_grouped_device_form_and_status(backend, small):
    t = 33
    x, ids, w = small.inputs(t, 4)
    dx, dids, dw = backend.to_device(x), backend.to_device(ids), backend.to_device(w)
    dy = backend.alloc(t * 256 * 4)
    dst = backend.to_device(np.zeros(1, np.int32))
    backend.grouped_gemm_device(small.layer, dx, t, dids, dw, dy, dst)
    y = backend.read(dy, np.float32, (t, 256))
    assert backend.read(dst, np.int32, (1,))[0] == 0
    assert np.array_equal(y, backend.grouped_gemm(small.layer, x, ids, w))
    bad = ids.copy()
    bad[5, 2] = 300
    backend.write(dids, bad)
    backend.grouped_gemm_device(small.layer, dx, t, dids, dw, dy, dst)
    assert backend.read(dst, np.int32, (1,))[0] == ERR_INVALID
    for b in (dx, dids, dw, dy, dst):
        backend.free(b)


def test_grouped_rejects_bad_arguments(backend, small):
    x, ids, w = small.inputs(4, 1)
    bad = ids.copy()
    bad[0, 0] = 256
    with pytest.raises(HipError) as e:
        backend.grouped_gemm(small.layer, x, bad, w)
    assert e.value.status == ERR_INVALID
    z = np.zeros((0, 256), np.uint16)
    with pytest.raises(HipError) as e:
        backend.grouped_gemm(small.layer, z, np.zeros((0, 8), np.uint16), np.zeros((0, 8), np.float32))
    assert e.value.status == ERR_INVALID
    # the context stays usable after an argument error
    assert rel_err(backend.grouped_gemm(small.layer, x, ids, w), small.want(x, ids, w)) < FFN_TOL


@pytest.mark.parametrize("t, where", [(700, (699, 7)), (700, (3, 0)), (1100, (600, 4))])
def test_grouped_bad_id_in_any_plan_batch(backend, small, t, where):
    """The plan counts pairs in batches of 4096: an out-of-range id in the
    first or a later batch sets the status and leaves y unwritten, and the
    next call on good ids is bit-identical to the host form."""
    x, ids, w = small.inputs(t, 6)
    dx, dids, dw = backend.to_device(x), backend.to_device(ids), backend.to_device(w)
    sentinel = np.full((t, 256), 7.25, np.float32)
    dy = backend.to_device(sentinel)
    dst = backend.to_device(np.zeros(1, np.int32))
    bad = ids.copy()
    bad[where] = 300
    backend.write(dids, bad)
    backend.grouped_gemm_device(small.layer, dx, t, dids, dw, dy, dst)
    assert backend.read(dst, np.int32, (1,))[0] == ERR_INVALID
    assert np.array_equal(backend.read(dy, np.float32, (t, 256)), sentinel)
    backend.write(dids, ids)
    backend.write(dst, np.zeros(1, np.int32))
    backend.grouped_gemm_device(small.layer, dx, t, dids, dw, dy, dst)
    assert backend.read(dst, np.int32, (1,))[0] == 0
    assert np.array_equal(backend.read(dy, np.float32, (t, 256)), backend.grouped_gemm(small.layer, x, ids, w))
    for b in (dx, dids, dw, dy, dst):
        backend.free(b)
