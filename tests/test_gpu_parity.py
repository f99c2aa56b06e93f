"""GPU parity: the HIP path (through the C ABI) against the CPU oracle on the
same seeded inputs.  Tolerances: expert-FFN outputs within 1e-3 of the
reference metric |g - c| / max(|c|, 1) (backend/metal/expert.rs:309-310);
routes, union plans, acceptance decisions and tokens bit-exact."""
import numpy as np
import pytest

import cpu_oracle as orc
from conftest import rel_err
from turboqwenfare_amd import _lib, mtp, synth
from turboqwenfare_amd._lib import ERR_DEVICE, ERR_INVALID, ERR_ROUTER, HipError

pytestmark = pytest.mark.gpu

FFN_TOL = 1e-3


def q4_block(scale_bits: int, qs: bytes) -> bytes:
    return scale_bits.to_bytes(2, "little") + qs


# ---- device / layout --------------------------------------------------------
def test_device_is_gfx950(backend):
    name, cus = backend.device_info()
    print(name, cus)
    assert "gfx950" in name
    assert cus > 0


@pytest.mark.parametrize("rows,cols", [(1, 32), (7, 96), (64, 256), (65, 288), (130, 2080),
                                       (512, 2048), (2048, 512)])
def test_repack_is_lossless(backend, rows, cols):
    rng = np.random.default_rng(rows * 1000 + cols)
    q = rng.integers(0, 256, size=rows * (cols // 32) * 18, dtype=np.uint8)
    w = backend.upload_q4_0(q, rows, cols)
    assert np.array_equal(backend.download_q4_0(w), q)
    assert backend.weights_bytes(w) >= q.nbytes
    backend.free_weights(w)


def test_device_synth_matches_host_generator(backend):
    w = backend.synth_q4_0(512, 2048, 7, 3)
    assert np.array_equal(backend.download_q4_0(w), synth.q4_0_synthetic(512, 2048, 7, 3))
    w2 = backend.synth_q4_0(2048, 512, 123456, 0)
    assert np.array_equal(backend.download_q4_0(w2), synth.q4_0_synthetic(2048, 512, 123456, 0))
    w3 = backend.synth_q4_0(512, 2048, 7, 3, "zero_mean")
    assert np.array_equal(backend.download_q4_0(w3), synth.q4_0_synthetic(512, 2048, 7, 3, "zero_mean"))
    for w_ in (w, w2, w3):
        backend.free_weights(w_)
    with pytest.raises(HipError) as e:
        backend.synth_q4_0(64, 64, 1, 1, 2)
    assert e.value.status == ERR_INVALID


def test_upload_rejects_bad_shapes(backend):
    with pytest.raises(HipError) as e:
        backend.upload_q4_0(np.zeros(18, np.uint8), 1, 48)
    assert e.value.status == ERR_INVALID
    with pytest.raises(HipError) as e:
        backend.upload_q4_0(np.zeros(17, np.uint8), 1, 32)
    assert e.value.status == ERR_INVALID


# ---- a3: GEMV ---------------------------------------------------------------
def test_gemv_canonical_q4_zero_block_kat(backend):
    # weights.rs:2500-2508: scale 1.0, every nibble 15 -> 7 x 32 ones = 224.
    w = backend.upload_q4_0(np.frombuffer(q4_block(0x3C00, b"\xff" * 16), np.uint8), 1, 32)
    assert backend.q4_gemv(w, np.ones(32, np.float32))[0] == 224.0
    # weights.rs:2511-2530: the second plane (all-zero bytes) gives 0.0.
    two = np.frombuffer(q4_block(0x3C00, b"\xff" * 16) + bytes(18), np.uint8)
    w2 = backend.upload_q4_0(two, 2, 32)
    assert list(backend.q4_gemv(w2, np.ones(32, np.float32))) == [224.0, 0.0]


def test_gemv_one_hot_probe_recovers_every_element(backend):
    # kernels.rs:1168-1196 technique: x = e_j returns column j exactly.
    rows, cols = 64, 256
    q = synth.q4_0_synthetic(rows, cols, 11, 0)
    w = backend.upload_q4_0(q, rows, cols)
    dense = np.stack([np.concatenate([orc.dequantize_q4_0(q[(r * (cols // 32) + b) * 18:
                                                              (r * (cols // 32) + b + 1) * 18])
                                      for b in range(cols // 32)]) for r in range(rows)])
    eye = np.eye(cols, dtype=np.float32)
    for j0 in range(0, cols, 8):
        y = backend.q4_gemv(w, eye[j0:j0 + 8])
        assert np.array_equal(y, dense[:, j0:j0 + 8].T)


def test_gemv_config1_parity(backend):
    rows, cols = 512, 2048
    q = synth.q4_0_synthetic(rows, cols, 1, 0)
    x = synth.normal((cols,), seed=0)
    w = backend.upload_q4_0(q, rows, cols)
    assert rel_err(backend.q4_gemv(w, x), orc.q4_0_matvec(q, rows, cols, x)) < 1e-5


@pytest.mark.parametrize("rows,cols", [(1, 32), (7, 96), (65, 288), (130, 2080), (2048, 512)])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 8])
def test_gemv_shape_sweep(backend, rows, cols, m):
    q = synth.q4_0_synthetic(rows, cols, rows + cols, m)
    x = synth.normal((m, cols), seed=m, std=2.0)
    w = backend.upload_q4_0(q, rows, cols)
    y = backend.q4_gemv(w, x)
    for t in range(m):
        assert rel_err(y[t], orc.q4_0_matvec(q, rows, cols, x[t])) < 1e-5
    backend.free_weights(w)


def test_gemv_propagates_non_finite_input(backend):
    q = synth.q4_0_synthetic(64, 256, 5, 5)
    w = backend.upload_q4_0(q, 64, 256)
    x = np.ones(256, np.float32)
    x[40] = np.nan
    assert np.all(np.isnan(backend.q4_gemv(w, x)))


def test_gemv_wide_dynamic_range(backend):
    rows, cols = 64, 512
    q = synth.q4_0_synthetic(rows, cols, 9, 9)
    rng = np.random.default_rng(9)
    x = (rng.standard_normal(cols) * np.exp2(rng.integers(-40, 40, cols))).astype(np.float32)
    w = backend.upload_q4_0(q, rows, cols)
    got = backend.q4_gemv(w, x)
    want = orc.q4_0_matvec(q, rows, cols, x)
    scale = np.max(np.abs(x)) * 0.02 * 8
    assert np.max(np.abs(got - want)) <= 1e-5 * scale * np.sqrt(cols)


def test_gemv_batched_matches_single(backend):
    ws = [backend.synth_q4_0(512, 2048, 100 + i, 0) for i in range(5)]
    x = synth.normal((2048,), seed=4)
    dx = backend.to_device(x)
    dy = backend.alloc(5 * 512 * 4)
    backend.q4_gemv_batched_device(ws, dx, dy)
    y = backend.read(dy, np.float32, (5, 512))
    for i, w in enumerate(ws):
        assert np.array_equal(y[i], backend.q4_gemv(w, x))
    backend.free(dx)
    backend.free(dy)
    for w in ws:
        backend.free_weights(w)


def test_gemv_config1_matches_committed_golden(backend):
    import sys
    from pathlib import Path

    golden = Path(__file__).resolve().parent / "golden"
    sys.path.insert(0, str(golden))
    from golden_inputs import gemv_inputs

    w, x = gemv_inputs()
    dev = backend.upload_q4_0(w, 512, 2048)
    want = np.load(golden / "oracle_vectors.npz")["gemv_y"]
    assert rel_err(backend.q4_gemv(dev, x), want) < 1e-5
    backend.free_weights(dev)


# ---- a10: one expert --------------------------------------------------------
@pytest.mark.parametrize("m", [1, 4])
def test_expert_forward_parity(backend, m):
    g = backend.synth_q4_0(512, 2048, 21, 0)
    u = backend.synth_q4_0(512, 2048, 22, 0)
    d = backend.synth_q4_0(2048, 512, 23, 0)
    x = synth.normal((m, 2048), seed=m)
    y = backend.expert_forward(g, u, d, x)
    gq, uq, dq = (backend.download_q4_0(t) for t in (g, u, d))
    for t in range(m):
        assert rel_err(y[t], orc.expert_forward(gq, uq, dq, 2048, 512, x[t])) < FFN_TOL
    for t in (g, u, d):
        backend.free_weights(t)


# ---- a11/a12: MoE layer -----------------------------------------------------
class Layer:
    """One synthetic layer resident on the device with host copies for the
    oracle (router ~N(0, 1/2048), shared input gate ~N(0, 1/2048))."""

    def __init__(self, be, layer_id: int, seed: int = 0, router_std=2048 ** -0.5, router=None, E=256,
                 F=512):
        H = 2048
        base = 10_000 * (layer_id + 1)
        self.router = (synth.normal((E, H), seed=base + 1, std=router_std) if router is None
                       else np.ascontiguousarray(router, np.float32))
        self.gate_vec = synth.normal((H,), seed=base + 2, std=2048 ** -0.5)
        mats = []
        for e in range(E + 1):
            mats.append((be.synth_q4_0(F, H, base + 3 * e + 10, seed),
                         be.synth_q4_0(F, H, base + 3 * e + 11, seed),
                         be.synth_q4_0(H, F, base + 3 * e + 12, seed)))
        self.dev = be.prepare_moe_layer(be.upload_f32(self.router), be.upload_f32(self.gate_vec),
                                        mats[E], [m[0] for m in mats[:E]],
                                        [m[1] for m in mats[:E]], [m[2] for m in mats[:E]])
        host = [[be.download_q4_0(t) for t in m] for m in mats]
        self.host = orc.MoeLayerHost(self.router, self.gate_vec, *host[E],
                                     [h[0] for h in host[:E]], [h[1] for h in host[:E]],
                                     [h[2] for h in host[:E]], width=F)
        self.mats = mats


@pytest.fixture(scope="module")
def layer(backend):
    return Layer(backend, 0)


@pytest.mark.parametrize("m", [1, 4])
def test_moe_layer_parity(backend, layer, m):
    x = synth.normal((m, 2048), seed=100 + m)
    y, ids, w = backend.moe_forward_batch(layer.dev, x)
    yc, idc, wc = layer.host.forward_batch(x)
    assert np.array_equal(ids, idc)
    assert rel_err(w, wc) < 1e-5
    assert rel_err(y, yc) < FFN_TOL
    print(f"m={m} rel err {rel_err(y, yc):.3e} union {len(mtp.routes_union(ids))}")


def test_moe_layer_bf16_input(backend, layer):
    x = synth.normal((4, 2048), seed=7)
    xb = (x.view(np.uint32) >> 16).astype(np.uint16)
    xf = (xb.astype(np.uint32) << 16).view(np.float32)
    y, ids, _ = backend.moe_forward_batch_bf16(layer.dev, xb)
    yc, idc, _ = layer.host.forward_batch(xf)
    assert np.array_equal(ids, idc)
    assert rel_err(y, yc) < FFN_TOL


@pytest.mark.parametrize("seed", range(8))
def test_moe_routes_and_union_over_seeds(backend, layer, seed):
    x = synth.normal((4, 2048), seed=1000 + seed)
    y, ids, _ = backend.moe_forward_batch(layer.dev, x)
    yc, idc, _ = layer.host.forward_batch(x)
    assert np.array_equal(ids, idc)
    assert mtp.routes_union(ids) == orc.batch_union(idc)
    assert rel_err(y, yc) < FFN_TOL


def test_moe_duplicate_rows_give_identical_outputs(backend, layer):
    x = np.repeat(synth.normal((1, 2048), seed=55), 4, axis=0)
    y, ids, _ = backend.moe_forward_batch(layer.dev, x)
    assert all(np.array_equal(ids[0], ids[t]) for t in range(4))
    assert all(np.array_equal(y[0], y[t]) for t in range(4))


def test_moe_rejects_non_finite_router_input(backend, layer):
    x = synth.normal((2, 2048), seed=3)
    x[1, 17] = np.inf
    with pytest.raises(HipError) as e:
        backend.moe_forward_batch(layer.dev, x)
    assert e.value.status == ERR_ROUTER
    # the context stays usable afterwards
    y, _, _ = backend.moe_forward_batch(layer.dev, x[:1])
    assert np.all(np.isfinite(y))


# ---- stacked layers (runtime.rs:777-802) and the graph-replayed verify step --
@pytest.fixture(scope="module")
def stack3(backend, layer):
    layers = [layer, Layer(backend, 1), Layer(backend, 2)]
    norms = [1.0 + 0.1 * synth.normal((2048,), seed=900 + i) for i in range(3)]
    st = backend.prepare_stack([l.dev for l in layers], [backend.upload_f32(n) for n in norms])
    return layers, norms, st


def oracle_stack(layers, norms, h):
    h = h.copy()
    routes = []
    for L, nw in zip(layers, norms):
        xn = np.stack([orc.qwen_rmsnorm(h[t], nw) for t in range(h.shape[0])])
        y, ids, _ = L.host.forward_batch(xn)
        h = (h + y).astype(np.float32)
        routes.append(ids)
    return h, routes


def test_stack_forward_parity(backend, stack3):
    layers, norms, st = stack3
    h0 = synth.normal((4, 2048), seed=77)
    dh = backend.to_device(h0)
    dids = backend.alloc(3 * 4 * 8 * 2)
    backend.stack_forward_device(st, dh, 4, dids)
    h = backend.read(dh, np.float32, (4, 2048))
    ids = backend.read(dids, np.uint16, (3, 4, 8))
    hc, routes = oracle_stack(layers, norms, h0)
    for l in range(3):
        assert np.array_equal(ids[l], routes[l])
    assert rel_err(h, hc) < FFN_TOL
    backend.free(dh)
    backend.free(dids)


def test_verify_step_graph_replays_match_eager(backend, stack3):
    layers, norms, st = stack3
    vocab, k = 151936, 3
    rng = np.random.default_rng(5)
    target = (rng.standard_normal((k + 1, vocab)) * 3).astype(np.float32)
    draft = (rng.standard_normal((k, vocab)) * 3).astype(np.float32)
    dtok = np.array([int(np.argmax(target[i])) for i in range(k)], np.int32)
    u = synth.philox_uniforms(0, 0, k)
    ur = synth.philox_uniforms(0, 1, k + 1)
    h0 = synth.normal((4, 2048), seed=88)
    bufs = {n: backend.to_device(a) for n, a in
            dict(t=target, d=draft, dt=dtok, u=u, ur=ur).items()}
    acc = backend.alloc(4)
    toks = backend.alloc(4 * (k + 1))
    # eager reference (profiling forces eager launches): stack forward
    dh_e = backend.to_device(h0)
    backend.profile_enable(True)
    backend.stack_forward_device(st, dh_e, 4)
    h_e = backend.read(dh_e, np.float32, (4, 2048))
    backend.profile_enable(False)
    want = orc.accept(target, draft, dtok, 0.7, False, u, ur)
    dh = backend.to_device(h0)
    for rep in range(3):
        backend.write(dh, h0)
        backend.synchronize()
        backend.verify_step_device(st, None, dh, 4, bufs["t"], bufs["d"], bufs["dt"], vocab,
                                   0.7, False, bufs["u"], bufs["ur"], acc, toks)
        h = backend.read(dh, np.float32, (4, 2048))
        a = int(backend.read(acc, np.int32, (1,))[0])
        tk = backend.read(toks, np.int32, (k + 1,))
        assert np.array_equal(h, h_e), f"replay {rep} differs from the eager stack"
        assert (a, [int(v) for v in tk[: a + 1]]) == want
    for b in list(bufs.values()) + [acc, toks, dh, dh_e]:
        backend.free(b)


# ---- a16: top_logit_candidates ----------------------------------------------
def test_top_logit_candidates_parity(backend):
    rng = np.random.default_rng(0)
    rows = []
    for s in range(6):
        v = (rng.standard_normal(151936) * 3).astype(np.float32)
        rows.append(v)
    ties = np.full(151936, -5.0, np.float32)
    ties[[10, 7, 99999, 3]] = 2.0
    ties[50] = np.nan
    rows.append(ties)
    rows.append(np.full(151936, -np.inf, np.float32))
    allnan = np.full(151936, np.nan, np.float32)
    allnan[151935] = 1.0
    rows.append(allnan)
    lg = np.stack(rows)
    toks, vals = backend.top_logit_candidates(lg)
    for r in range(lg.shape[0]):
        tc, vc = orc.top_logit_candidates(lg[r])
        assert list(toks[r]) == list(tc)
        assert np.array_equal(vals[r], vc)


def test_small_geometry_layer_matches_committed_golden(backend):
    """hidden 256, width 256 (padded block counts: the 16-lane row layout with
    zero-scale padding blocks) against the committed oracle outputs."""
    import sys
    from pathlib import Path

    golden = Path(__file__).resolve().parent / "golden"
    sys.path.insert(0, str(golden))
    from golden_inputs import SMALL, small_layer_inputs

    router, gate, x, mats = small_layer_inputs()
    E, H, F = SMALL["experts"], SMALL["hidden"], SMALL["width"]
    dev = [(backend.upload_q4_0(g, F, H), backend.upload_q4_0(u, F, H), backend.upload_q4_0(d, H, F))
           for g, u, d in mats]
    layer = backend.prepare_moe_layer(backend.upload_f32(router), backend.upload_f32(gate), dev[E],
                                      [m[0] for m in dev[:E]], [m[1] for m in dev[:E]],
                                      [m[2] for m in dev[:E]])
    g = np.load(golden / "oracle_vectors.npz")
    for m in (1, 4):
        y, ids, w = backend.moe_forward_batch(layer, x[:m])
        assert np.array_equal(ids, g[f"moe_ids{m}"])
        assert rel_err(w, g[f"moe_w{m}"]) < 1e-5
        assert rel_err(y, g[f"moe_y{m}"]) < FFN_TOL
    backend.free_moe_layer(layer)
    for t in dev:
        for wt in t:
            backend.free_weights(wt)


# ---- the persistent whole-stack kernel ----------------------------------------
def _stack_run(backend, st, h0, m, n_layers, persistent, with_w=False):
    with backend.variant(_lib.VARIANT_PERSISTENT, persistent):
        dh = backend.to_device(h0[:m])
        dids = backend.alloc(n_layers * m * 8 * 2)
        dw = backend.alloc(n_layers * m * 8 * 4)
        dst = backend.to_device(np.zeros(1, np.int32))
        backend.stack_forward_device(st, dh, m, dids, dw, dst)
        out = (backend.read(dh, np.float32, (m, 2048)), backend.read(dids, np.uint16, (n_layers, m, 8)),
               backend.read(dw, np.float32, (n_layers, m, 8)), int(backend.read(dst, np.int32, (1,))[0]))
        for b in (dh, dids, dw, dst):
            backend.free(b)
        return out


@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_persistent_stack_matches_oracle_and_layer_kernels(backend, stack3, m):
    layers, norms, st = stack3
    h0 = synth.normal((4, 2048), seed=300 + m)
    h_p, ids_p, w_p, s_p = _stack_run(backend, st, h0, m, 3, True)
    h_k, ids_k, w_k, s_k = _stack_run(backend, st, h0, m, 3, False)
    assert s_p == 0 and s_k == 0
    assert np.array_equal(ids_p, ids_k)
    assert rel_err(w_p, w_k) < 1e-5
    # the persistent kernel scales the dot products of y = h * w_norm by
    # 1/rms, the layer kernels normalise x first: the two round differently
    # (this stack's rows reach |h| ~ 1e3), each within the oracle's bound
    assert rel_err(h_p, h_k) < FFN_TOL
    hc, routes = oracle_stack(layers, norms, h0[:m])
    for l in range(3):
        assert np.array_equal(ids_p[l], routes[l])
    assert rel_err(h_p, hc) < FFN_TOL


def test_routes_with_tied_router_rows(backend):
    """Bit-equal router rows give bit-equal probabilities: the top-8 must
    take tied experts in ascending id order (from_logits' stable descending
    sort, experts/mod.rs:134-197).  Token 0: its top expert's row copied to
    experts 3, 70, 130 and 200 (a five-way tie at rank 1, across all four of
    a lane's slots); token 1: its 8th expert's row copied to two more, one
    id below and one above (a three-way tie across the rank-8 boundary).
    Both stack paths and the single-layer kernel, against the oracle."""
    E, H = 256, 2048
    h0 = synth.normal((4, H), seed=4242)
    norm = (1.0 + 0.05 * synth.normal((H,), seed=4243)).astype(np.float32)
    router = synth.normal((E, H), seed=4244, std=H ** -0.5)

    def logits(R, t):
        return orc.f32_matvec(R, orc.qwen_rmsnorm(h0[t], norm))

    def ranking(R, t):
        lg = logits(R, t)
        return sorted(range(E), key=lambda e: (-lg[e], e))

    top = ranking(router, 0)[0]
    copies = [e for e in (3, 70, 130, 200, 5, 75) if e != top][:4]
    for e in copies:
        router[e] = router[top]
    r1 = ranking(router, 1)
    e8 = r1[7]
    free = [e for e in range(E) if e not in r1[:8] and e not in copies + [top]]
    below, above = free[0], free[-1]
    router[below] = router[e8]
    router[above] = router[e8]
    # the construction holds: five equal logits at token 0's top, three
    # across token 1's rank-8 boundary
    lg0, lg1 = logits(router, 0), logits(router, 1)
    assert len({float(lg0[e]) for e in copies + [top]}) == 1
    assert lg1[below] == lg1[e8] == lg1[above]
    L = Layer(backend, 9, router=router)
    st = backend.prepare_stack([L.dev], [backend.upload_f32(norm)])
    try:
        hc, routes = oracle_stack([L], [norm], h0)
        for persistent in (True, False):
            h, ids, w, status = _stack_run(backend, st, h0, 4, 1, persistent)
            assert status == 0
            assert np.array_equal(ids[0], routes[0]), (persistent, ids[0], routes[0])
            assert rel_err(h, hc) < FFN_TOL
        xn = np.stack([orc.qwen_rmsnorm(h0[t], norm) for t in range(4)])
        _, ids1, _ = backend.moe_forward_batch(L.dev, xn)
        assert np.array_equal(ids1, routes[0])
    finally:
        backend.free_stack(st)


def test_persistent_stack_repeats_bit_identically(backend, stack3):
    """Barrier and team counters return to zero at the end of every launch."""
    _, _, st = stack3
    h0 = synth.normal((4, 2048), seed=411)
    first = _stack_run(backend, st, h0, 4, 3, True)
    for _ in range(4):
        again = _stack_run(backend, st, h0, 4, 3, True)
        assert np.array_equal(again[0], first[0]) and np.array_equal(again[1], first[1])


def test_persistent_stack_reports_router_error(backend, stack3):
    _, _, st = stack3
    h0 = synth.normal((4, 2048), seed=412)
    h0[2, 100] = np.inf
    _, _, _, status = _stack_run(backend, st, h0, 4, 3, True)
    assert status == ERR_ROUTER


@pytest.mark.parametrize("fail_at", [0, 2])
def test_persistent_stack_abort_leaves_clean_state(backend, stack3, monkeypatch, fail_at):
    """A grid-barrier wait that times out aborts the launch: every workgroup
    leaves at its next bounded wait, the launch reports TQF_HIP_ERR_DEVICE,
    and the last workgroup out resets the barrier state (both counter levels,
    release, abort) and the logit accumulators, so the following launches are
    bit-identical to one before the failure.  The timeout is forced from the
    host (workgroup 0 takes the barrier-B wait of layer `fail_at` as timed
    out), so every kernel exits normally."""
    _, _, st = stack3
    h0 = synth.normal((4, 2048), seed=413)
    with backend.variant(_lib.VARIANT_RECOVER, False):
        first = _stack_run(backend, st, h0, 4, 3, True)
        assert first[3] == 0
        monkeypatch.setenv("TQF_HIP_STACK_FAIL_AT_LAYER", str(fail_at))
        _, _, _, status = _stack_run(backend, st, h0, 4, 3, True)
        assert status == ERR_DEVICE
        monkeypatch.delenv("TQF_HIP_STACK_FAIL_AT_LAYER")
        for _ in range(2):
            again = _stack_run(backend, st, h0, 4, 3, True)
            assert again[3] == 0
            assert np.array_equal(again[0], first[0]) and np.array_equal(again[1], first[1])


@pytest.mark.parametrize("fail_at", [0, 2])
@pytest.mark.parametrize("m", [1, 4])
def test_persistent_stack_abort_is_recovered(backend, stack3, monkeypatch, fail_at, m):
    """With recovery on (the default), a persistent launch whose barrier wait
    times out is re-run by the library through the per-layer kernels from the
    copy of h_in the launch's prologue made -- also in place, where the launch
    itself updates h: the call reports status 0, returns exactly the per-layer
    path's h and routes, and counts one stack re-run.  The timeout is forced
    from the host (TQF_HIP_STACK_FAIL_AT_LAYER), so every wait still ends."""
    _, _, st = stack3
    h0 = synth.normal((4, 2048), seed=415 + m)
    want = _stack_run(backend, st, h0, m, 3, False)
    assert want[3] == 0
    before = backend.recovery_counts()
    monkeypatch.setenv("TQF_HIP_STACK_FAIL_AT_LAYER", str(fail_at))
    got = _stack_run(backend, st, h0, m, 3, True)
    monkeypatch.delenv("TQF_HIP_STACK_FAIL_AT_LAYER")
    after = backend.recovery_counts()
    assert got[3] == 0
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
    assert np.array_equal(got[2], want[2])
    assert after == (before[0] + 1, before[1])
    # the next launch is the persistent path again, unrecovered
    again = _stack_run(backend, st, h0, m, 3, True)
    assert again[3] == 0 and backend.recovery_counts() == after
    assert np.array_equal(again[1], want[1]) and rel_err(again[0], want[0]) < FFN_TOL


@pytest.mark.parametrize("F", [256, 1024, 2048])
def test_persistent_stack_other_widths(backend, F):
    """Expert widths other than the model's 512 select the other kernel
    instantiations (down rows of 16 / 32 / 64 blocks; 64- and 32-row gate/up
    units, several per workgroup where 8 M F / R exceeds the grid): a 2-layer
    stack at M = 1, 2, 4 matches the per-layer kernels and the oracle's
    routes."""
    layers = [Layer(backend, 20 + F // 256 + i, F=F) for i in range(2)]
    norms = [1.0 + 0.1 * synth.normal((2048,), seed=950 + i) for i in range(2)]
    st = backend.prepare_stack([l.dev for l in layers], [backend.upload_f32(n) for n in norms])
    try:
        for m in (1, 2, 4):
            h0 = synth.normal((4, 2048), seed=960 + m)
            h_p, ids_p, _, s_p = _stack_run(backend, st, h0, m, 2, True)
            h_k, ids_k, _, s_k = _stack_run(backend, st, h0, m, 2, False)
            assert s_p == 0 and s_k == 0
            assert np.array_equal(ids_p, ids_k), (F, m)
            assert rel_err(h_p, h_k) < FFN_TOL, (F, m)
            hc, routes = oracle_stack(layers, norms, h0[:m])
            for l in range(2):
                assert np.array_equal(ids_p[l], routes[l]), (F, m, l)
            assert rel_err(h_p, hc) < FFN_TOL, (F, m, rel_err(h_p, hc))
    finally:
        backend.free_stack(st)
        for L in layers:
            backend.free_moe_layer(L.dev)


def test_persistent_stack_recovers_from_logit_range(backend, stack3):
    """Rows of h around 1e7 keep ordinary (normalised) router logits, but a
    team's partial sum of router row times y exceeds the persistent kernel's
    fixed-point range (2^20): with recovery on the launch aborts and the
    library re-runs the stack through the per-layer kernels, so the call
    returns exactly their h and routes with status 0 and counts one re-run;
    with recovery off the call reports the router error."""
    _, _, st = stack3
    h0 = (synth.normal((4, 2048), seed=433) * 1e7).astype(np.float32)
    want = _stack_run(backend, st, h0, 4, 3, False)
    assert want[3] == 0
    before = backend.recovery_counts()
    got = _stack_run(backend, st, h0, 4, 3, True)
    assert got[3] == 0
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
    assert backend.recovery_counts() == (before[0] + 1, before[1])
    with backend.variant(_lib.VARIANT_RECOVER, False):
        off = _stack_run(backend, st, h0, 4, 3, True)
    assert off[3] == ERR_ROUTER
    # a clean launch afterwards runs the persistent path bit-identically
    h1 = synth.normal((4, 2048), seed=434)
    a1, b1 = _stack_run(backend, st, h1, 4, 3, True), _stack_run(backend, st, h1, 4, 3, True)
    assert a1[3] == 0 and np.array_equal(a1[0], b1[0]) and backend.recovery_counts()[0] == before[0] + 1


def test_verify_step_recovers_both_parts(backend, stack3, monkeypatch):
    """A verify step whose persistent stack and one-launch acceptance both
    time out (forced from the host) still returns the per-layer stack's h
    and the oracle's acceptance, with one re-run of each counted."""
    _, _, st = stack3
    vocab, k = 151936, 3
    rng = np.random.default_rng(33)
    target = (rng.standard_normal((k + 1, vocab)) * 3).astype(np.float32)
    draft = (rng.standard_normal((k, vocab)) * 3).astype(np.float32)
    dtok = rng.integers(0, vocab, k).astype(np.int32)
    u = rng.random(k).astype(np.float32)
    ur = rng.random(k + 1).astype(np.float32)
    want_acc = orc.accept(target, draft, dtok, 0.7, False, u, ur)
    h0 = synth.normal((4, 2048), seed=431)
    want_h = _stack_run(backend, st, h0, 4, 3, False)[0]
    bufs = {n: backend.to_device(v) for n, v in dict(t=target, d=draft, dt=dtok, u=u, ur=ur, h0=h0).items()}
    dh, acc, toks = backend.alloc(4 * 2048 * 4), backend.alloc(4), backend.alloc(4 * (k + 1))
    dst = backend.to_device(np.zeros(1, np.int32))
    before = backend.recovery_counts()
    monkeypatch.setenv("TQF_HIP_STACK_FAIL_AT_LAYER", "1")
    monkeypatch.setenv("TQF_HIP_ACCEPT_FAIL_POLL", "1")
    backend.verify_step_device(st, bufs["h0"], dh, 4, bufs["t"], bufs["d"], bufs["dt"], vocab, 0.7, False,
                               bufs["u"], bufs["ur"], acc, toks, dst)
    monkeypatch.delenv("TQF_HIP_STACK_FAIL_AT_LAYER")
    monkeypatch.delenv("TQF_HIP_ACCEPT_FAIL_POLL")
    assert backend.recovery_counts() == (before[0] + 1, before[1] + 1)
    assert int(backend.read(dst, np.int32, (1,))[0]) == 0
    assert np.array_equal(backend.read(dh, np.float32, (4, 2048)), want_h)
    a = int(backend.read(acc, np.int32, (1,))[0])
    assert (a, [int(v) for v in backend.read(toks, np.int32, (k + 1,))[: a + 1]]) == want_acc
    for b in list(bufs.values()) + [dh, acc, toks, dst]:
        backend.free(b)


@pytest.mark.parametrize("persistent", [True, False], ids=["persistent", "per_layer"])
def test_verify_step_reports_router_error(backend, stack3, persistent):
    """A non-finite router logit inside the verify step reaches its d_status
    (TQF_HIP_ERR_ROUTER); the acceptance, which reads only the logits, still
    returns the oracle's decision, and a clean step afterwards reports 0."""
    _, _, st = stack3
    vocab, k = 4096, 3
    rng = np.random.default_rng(21)
    target = (rng.standard_normal((k + 1, vocab)) * 3).astype(np.float32)
    dtok = np.argmax(target[:k], axis=1).astype(np.int32)
    want = orc.accept(target, None, dtok, 0.7, True)
    h_bad = synth.normal((4, 2048), seed=413)
    h_bad[1, 7] = np.nan
    with backend.variant(_lib.VARIANT_PERSISTENT, persistent):
        for h0, expect in ((h_bad, ERR_ROUTER), (synth.normal((4, 2048), seed=414), 0)):
            dh0, dh = backend.to_device(h0), backend.alloc(4 * 2048 * 4)
            dt, ddt = backend.to_device(target), backend.to_device(dtok)
            acc, toks = backend.alloc(4), backend.alloc(4 * (k + 1))
            dst = backend.to_device(np.zeros(1, np.int32))
            backend.verify_step_device(st, dh0, dh, 4, dt, None, ddt, vocab, 0.7, True, None, None,
                                       acc, toks, dst)
            assert int(backend.read(dst, np.int32, (1,))[0]) == expect
            a = int(backend.read(acc, np.int32, (1,))[0])
            tk = backend.read(toks, np.int32, (k + 1,))
            assert (a, [int(v) for v in tk[: a + 1]]) == want
            for b in (dh0, dh, dt, ddt, acc, toks, dst):
                backend.free(b)
