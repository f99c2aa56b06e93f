"""GPU parity of the MoE layer with Q4_K experts -- the canonical checkpoint's
expert format run through the same layer, stack and verify-step entry points
as the Q4_0 configs (experts/mod.rs:1540-1634 with matvec_payload's Q4_K arm,
weights.rs:680-735) -- against the CPU oracle (orc_moe_forward_batch_q4k) on
the same inputs:

  * routes equal, route weights within 1e-5;
  * y within 1e-3 of |g - c| / max(|c|, 1) (the reference's metric,
    expert.rs:309-310): every expert matvec is bit-identical to
    q4_k_dot_pre, while the router's f32 sums and the SwiGLU / sigmoid
    exponentials are the device's;
  * stacked layers (RMSNorm, MoE, residual) and the graph-replayed verify
    step with Q4_K layers; formats never mix within a layer or a stack."""
import numpy as np
import pytest

import cpu_oracle as orc
from conftest import rel_err
from turboqwenfare_amd import _lib, synth
from turboqwenfare_amd.synth import centered_q4_k
from turboqwenfare_amd._lib import ERR_INVALID, ERR_ROUTER, HipError

pytestmark = pytest.mark.gpu

FFN_TOL = 1e-3
E, H, F = 256, 2048, 512


class Q4KLayer:
    """One layer of random centred Q4_K experts (centered_q4_k: values
    d sc (q - 7.5), d sc ~ 0.008 on average, a spread of ~0.04 like trained
    expert weights), router and shared input gate ~N(0, 1/2048), resident on the
    device, with the GGML bytes kept for the oracle."""

    def __init__(self, be, layer_id: int, hidden: int = H, width: int = F):
        base = 70_000 + 1_000 * layer_id
        self.router = synth.normal((E, hidden), seed=base + 1, std=hidden ** -0.5)
        self.gate_vec = synth.normal((hidden,), seed=base + 2, std=hidden ** -0.5)
        shapes = ((width, hidden), (width, hidden), (hidden, width))
        host = [tuple(centered_q4_k(r, c, base + 10 + 3 * e + i)
                      for i, (r, c) in enumerate(shapes)) for e in range(E + 1)]
        mats = [tuple(be.upload_q4_k(q, r, c) for q, (r, c) in zip(h, shapes)) for h in host]
        self.dev = be.prepare_moe_layer(be.upload_f32(self.router), be.upload_f32(self.gate_vec),
                                        mats[E], [m[0] for m in mats[:E]],
                                        [m[1] for m in mats[:E]], [m[2] for m in mats[:E]])
        self.host = orc.MoeLayerHost(self.router, self.gate_vec, *host[E],
                                     [h[0] for h in host[:E]], [h[1] for h in host[:E]],
                                     [h[2] for h in host[:E]], hidden=hidden, width=width,
                                     fmt="q4_k")
        self.mats = mats


@pytest.fixture(scope="module")
def q4k_layers(backend):
    return [Q4KLayer(backend, 0), Q4KLayer(backend, 1)]


@pytest.mark.parametrize("m", [1, 4, 8])
def test_q4k_moe_layer_parity(backend, q4k_layers, m):
    L = q4k_layers[0]
    x = synth.normal((m, H), seed=200 + m)
    y, ids, w = backend.moe_forward_batch(L.dev, x)
    yc, idc, wc = L.host.forward_batch(x, nthreads=8)
    assert np.array_equal(ids, idc)
    assert rel_err(w, wc) < 1e-5
    assert rel_err(y, yc) < FFN_TOL
    print(f"m={m} rel err {rel_err(y, yc):.3e}")


@pytest.mark.parametrize("seed", range(4))
def test_q4k_moe_layer_parity_over_seeds(backend, q4k_layers, seed):
    L = q4k_layers[1]
    x = synth.normal((4, H), seed=2_000 + seed)
    y, ids, _ = backend.moe_forward_batch(L.dev, x)
    yc, idc, _ = L.host.forward_batch(x, nthreads=8)
    assert np.array_equal(ids, idc)
    assert rel_err(y, yc) < FFN_TOL


@pytest.mark.parametrize("hidden,width", [(256, 256), (512, 768)])
def test_q4k_moe_layer_small_geometries(backend, hidden, width):
    # one super-block per row (the layout pads to 16 sub-blocks) and an odd
    # super-block count: padding sub-blocks never enter the combine
    L = Q4KLayer(backend, 7, hidden, width)
    for m in (1, 3, 8):
        x = synth.normal((m, hidden), seed=700 + m)
        y, ids, _ = backend.moe_forward_batch(L.dev, x)
        yc, idc, _ = L.host.forward_batch(x, nthreads=8)
        assert np.array_equal(ids, idc)
        assert rel_err(y, yc) < FFN_TOL
    backend.free_moe_layer(L.dev)
    for m3 in L.mats:
        for w in m3:
            backend.free_weights(w)


def test_q4k_moe_layer_bf16_input(backend, q4k_layers):
    L = q4k_layers[0]
    x = synth.normal((4, H), seed=9)
    xb = (x.view(np.uint32) >> 16).astype(np.uint16)
    xf = (xb.astype(np.uint32) << 16).view(np.float32)
    y, ids, _ = backend.moe_forward_batch_bf16(L.dev, xb)
    yc, idc, _ = L.host.forward_batch(xf, nthreads=8)
    assert np.array_equal(ids, idc)
    assert rel_err(y, yc) < FFN_TOL


def test_q4k_moe_duplicate_rows_give_identical_outputs(backend, q4k_layers):
    x = np.repeat(synth.normal((1, H), seed=56), 4, axis=0)
    y, ids, _ = backend.moe_forward_batch(q4k_layers[0].dev, x)
    assert all(np.array_equal(ids[0], ids[t]) for t in range(4))
    assert all(np.array_equal(y[0].view(np.uint32), y[t].view(np.uint32)) for t in range(4))


def test_q4k_moe_device_entry_matches_host_entry(backend, q4k_layers):
    L = q4k_layers[0]
    x = synth.normal((3, H), seed=31)
    y, ids, w = backend.moe_forward_batch(L.dev, x)
    dx, dy = backend.to_device(x), backend.alloc(3 * H * 4)
    dids, dw = backend.alloc(3 * 8 * 2), backend.alloc(3 * 8 * 4)
    dst = backend.to_device(np.zeros(1, np.int32))
    backend.moe_layer_device(L.dev, dx, 3, dy, dids, dw, dst)
    assert np.array_equal(backend.read(dy, np.float32, (3, H)).view(np.uint32), y.view(np.uint32))
    assert np.array_equal(backend.read(dids, np.uint16, (3, 8)), ids)
    assert np.array_equal(backend.read(dw, np.float32, (3, 8)), w)
    assert int(backend.read(dst, np.int32, (1,))[0]) == 0
    for b in (dx, dy, dids, dw, dst):
        backend.free(b)


def test_q4k_moe_rejects_non_finite_router_input(backend, q4k_layers):
    L = q4k_layers[0]
    x = synth.normal((2, H), seed=4)
    x[1, 5] = np.nan
    with pytest.raises(HipError) as e:
        backend.moe_forward_batch(L.dev, x)
    assert e.value.status == ERR_ROUTER
    y, _, _ = backend.moe_forward_batch(L.dev, x[:1])
    assert np.all(np.isfinite(y))


def test_layer_formats_do_not_mix(backend, q4k_layers):
    L = q4k_layers[0]
    q0 = backend.synth_q4_0(F, H, 123, 0)
    gates = [m[0] for m in L.mats[:E]]
    gates[17] = q0
    router, gv = backend.upload_f32(L.router), backend.upload_f32(L.gate_vec)
    with pytest.raises(HipError) as e:
        backend.prepare_moe_layer(router, gv, L.mats[E], gates, [m[1] for m in L.mats[:E]],
                                  [m[2] for m in L.mats[:E]])
    assert e.value.status == ERR_INVALID
    backend.free_weights(q0)


def test_grouped_gemm_rejects_q4k_layers(backend, q4k_layers):
    x = np.zeros((4, H), np.uint16)
    ids = np.tile(np.arange(8, dtype=np.uint16), (4, 1))
    w = np.full((4, 8), 0.125, np.float32)
    with pytest.raises(HipError) as e:
        backend.grouped_gemm(q4k_layers[0].dev, x, ids, w)
    assert e.value.status == ERR_INVALID


# ---- stacked Q4_K layers (runtime.rs:777-802) and the verify step --------------
@pytest.fixture(scope="module")
def q4k_stack(backend, q4k_layers):
    norms = [1.0 + 0.1 * synth.normal((H,), seed=950 + i) for i in range(2)]
    st = backend.prepare_stack([l.dev for l in q4k_layers], [backend.upload_f32(n) for n in norms])
    return q4k_layers, norms, st


def oracle_q4k_stack(layers, norms, h):
    h = h.copy()
    routes = []
    for L, nw in zip(layers, norms):
        xn = np.stack([orc.qwen_rmsnorm(h[t], nw) for t in range(h.shape[0])])
        y, ids, _ = L.host.forward_batch(xn, nthreads=8)
        h = (h + y).astype(np.float32)
        routes.append(ids)
    return h, routes


@pytest.mark.parametrize("m", [1, 4, 8])
def test_q4k_stack_forward_parity(backend, q4k_stack, m):
    layers, norms, st = q4k_stack
    h0 = synth.normal((m, H), seed=500 + m)
    dh = backend.to_device(h0)
    dids = backend.alloc(2 * m * 8 * 2)
    dst = backend.to_device(np.zeros(1, np.int32))
    backend.stack_forward_device(st, dh, m, dids, None, dst)
    h = backend.read(dh, np.float32, (m, H))
    ids = backend.read(dids, np.uint16, (2, m, 8))
    assert int(backend.read(dst, np.int32, (1,))[0]) == 0
    hc, routes = oracle_q4k_stack(layers, norms, h0)
    for l in range(2):
        assert np.array_equal(ids[l], routes[l])
    assert rel_err(h, hc) < FFN_TOL
    for b in (dh, dids, dst):
        backend.free(b)


def test_stack_formats_do_not_mix(backend, q4k_stack):
    from test_gpu_parity import Layer

    layers, norms, _ = q4k_stack
    q0 = Layer(backend, 5)
    with pytest.raises(HipError) as e:
        backend.prepare_stack([layers[0].dev, q0.dev],
                              [backend.upload_f32(n) for n in norms])
    assert e.value.status == ERR_INVALID


def test_q4k_verify_step_graph_replays_match_eager(backend, q4k_stack):
    layers, norms, st = q4k_stack
    vocab, k = 151936, 3
    rng = np.random.default_rng(6)
    target = (rng.standard_normal((k + 1, vocab)) * 3).astype(np.float32)
    draft = (rng.standard_normal((k, vocab)) * 3).astype(np.float32)
    dtok = np.array([int(np.argmax(target[i])) for i in range(k)], np.int32)
    u = synth.philox_uniforms(1, 0, k)
    ur = synth.philox_uniforms(1, 1, k + 1)
    h0 = synth.normal((4, H), seed=89)
    bufs = {n: backend.to_device(a) for n, a in
            dict(t=target, d=draft, dt=dtok, u=u, ur=ur).items()}
    acc = backend.alloc(4)
    toks = backend.alloc(4 * (k + 1))
    dh_e = backend.to_device(h0)
    backend.profile_enable(True)  # eager launches
    backend.stack_forward_device(st, dh_e, 4)
    h_e = backend.read(dh_e, np.float32, (4, H))
    backend.profile_enable(False)
    hc, _ = oracle_q4k_stack(layers, norms, h0)
    assert rel_err(h_e, hc) < FFN_TOL
    want = orc.accept(target, draft, dtok, 0.7, False, u, ur)
    dh = backend.to_device(h0)
    for rep in range(3):
        backend.write(dh, h0)
        backend.synchronize()
        backend.verify_step_device(st, None, dh, 4, bufs["t"], bufs["d"], bufs["dt"], vocab,
                                   0.7, False, bufs["u"], bufs["ur"], acc, toks)
        h = backend.read(dh, np.float32, (4, H))
        a = int(backend.read(acc, np.int32, (1,))[0])
        tk = backend.read(toks, np.int32, (k + 1,))
        assert np.array_equal(h.view(np.uint32), h_e.view(np.uint32)), f"replay {rep} differs"
        assert (a, [int(v) for v in tk[: a + 1]]) == want
    for b in list(bufs.values()) + [acc, toks, dh, dh_e]:
        backend.free(b)



def test_q4k_folded_combine_equals_the_combine_launch(backend, q4k_stack):
    """The down launch's folded combine and q4k_moe_combine_kernel run the same
    arithmetic in the same order: a layer and a 2-layer stack give the same
    bits with the fold switched off (variant TQF_HIP_VARIANT_Q4K_FOLD = 0),
    graph-replayed (a variant change drops the captured graphs)."""
    layers, norms, st = q4k_stack
    x = synth.normal((4, H), seed=808)
    outs = []
    for fold in (True, False, True):
        with backend.variant(_lib.VARIANT_Q4K_FOLD, fold):
            y, _, _ = backend.moe_forward_batch(layers[0].dev, x)
            dh = backend.to_device(x)
            for _ in range(2):  # capture, then replay
                backend.write(dh, x)
                backend.stack_forward_device(st, dh, 4)
            outs.append((y, backend.read(dh, np.float32, (4, H))))
            backend.free(dh)
    for other in outs[1:]:
        for a, b in zip(outs[0], other):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
