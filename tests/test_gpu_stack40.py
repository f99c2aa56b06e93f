"""Config 4 at full depth: the 40-layer verify stack against the CPU oracle.

The model is the benchmark's own (``workloads.SyntheticStack``: 40 seeded
Q4_0 layers, 18.2 GB resident), built with both nibble recipes:
"zero_mean" (the benchmark's headline input, expert union ~30 per layer at
M = 4) and "uniform" (the literal configuration text, whose common-mode
weight bias collapses the four rows into one direction within a few layers).

The oracle replays h <- h + MoE_l(rmsnorm_l(h)) (model/qwen36/runtime.rs:
777-802, experts/mod.rs:1540-1577) layer by layer; each layer's host copy
holds only that layer's routed experts and the shared one (the routes come
from the oracle's own f32 router and from_logits first), downloaded from the
device.  Tolerances as everywhere: routes bit-equal, route weights within
1e-5, h within 1e-3 of |g - c| / max(|c|, 1) (backend/metal/expert.rs:309);
acceptance decisions and tokens bit-exact."""
import numpy as np
import pytest

import cpu_oracle as orc
from conftest import rel_err
from stack_oracle import oracle_replay
from turboqwenfare_amd import _lib, mtp, synth
from turboqwenfare_amd.workloads import H, SyntheticStack

pytestmark = pytest.mark.gpu

LAYERS = 40


@pytest.fixture(scope="module", params=["zero_mean", "uniform"])
def model40(request, backend):
    model = SyntheticStack(backend, LAYERS, seed=0, recipe=request.param)
    model.oracle = {}
    yield model
    model.free()


def h0_rows(m: int) -> np.ndarray:
    return synth.normal((4, H), seed=1)[:m]  # the benchmark's verify rows


def oracle_for(model, m):
    if m not in model.oracle:
        model.oracle[m] = oracle_replay(model, h0_rows(m))
    return model.oracle[m]


def run_stack(be, model, m, persistent):
    with be.variant(_lib.VARIANT_PERSISTENT, persistent):
        dh = be.to_device(h0_rows(m))
        dids = be.alloc(LAYERS * m * 8 * 2)
        dw = be.alloc(LAYERS * m * 8 * 4)
        dst = be.to_device(np.zeros(1, np.int32))
        be.stack_forward_device(model.stack, dh, m, dids, dw, dst)
        out = (be.read(dh, np.float32, (m, H)), be.read(dids, np.uint16, (LAYERS, m, 8)),
               be.read(dw, np.float32, (LAYERS, m, 8)), int(be.read(dst, np.int32, (1,))[0]))
        for b in (dh, dids, dw, dst):
            be.free(b)
    return out


@pytest.mark.parametrize("m", [4, 1])
@pytest.mark.parametrize("persistent", [True, False], ids=["persistent", "per_layer"])
def test_stack40_matches_oracle(backend, model40, m, persistent):
    hc, idc, wc = oracle_for(model40, m)
    h, ids, w, status = run_stack(backend, model40, m, persistent)
    assert status == 0
    for l in range(LAYERS):
        assert np.array_equal(ids[l], idc[l]), f"layer {l} routes differ"
    assert rel_err(w, wc) < 1e-5
    err = rel_err(h, hc)
    unions = [len(mtp.routes_union(idc[l])) for l in range(LAYERS)]
    print(f"{model40.recipe} m={m} {'persistent' if persistent else 'per-layer'}: h rel err "
          f"{err:.3e}, |h| rms {np.sqrt(np.mean(hc.astype(np.float64) ** 2)):.2f}, union mean "
          f"{np.mean(unions):.2f} min {min(unions)} max {max(unions)}")
    assert err < 1e-3
    if model40.recipe == "zero_mean" and m == 4:
        # the headline input stays an M = 4 workload at every depth
        assert np.mean(unions) >= 28 and min(unions) >= 24


def test_stack40_unions_follow_the_recipe(backend, model40):
    """The zero-mean rows stay apart (per-layer union near the i.i.d. 30.5);
    the uniform recipe's rows collapse onto one direction."""
    _, idc, _ = oracle_for(model40, 4)
    late = [len(mtp.routes_union(idc[l])) for l in range(10, LAYERS)]
    if model40.recipe == "zero_mean":
        assert np.mean(late) > 28
    else:
        assert np.mean(late) < 12


@pytest.mark.parametrize("greedy", [False, True], ids=["stochastic", "greedy"])
def test_verify_step40_matches_stack_and_acceptance_oracle(backend, model40, greedy):
    """The full verify step at config 4: h bit-identical to the stack forward,
    acceptance equal to the oracle's on the config-3 logits, status zero; the
    graph/persistent step replayed several times with eager work between."""
    be, m, k, vocab, T = backend, 4, 3, 151936, 0.7
    h_ref, _, _, _ = run_stack(be, model40, m, True)
    rng = np.random.default_rng(11)
    target = (rng.standard_normal((k + 1, vocab)) * 3.0).astype(np.float32)
    draft = (rng.standard_normal((k, vocab)) * 3.0).astype(np.float32)
    dtok = np.argmax(draft, axis=1).astype(np.int32)
    dtok[0] = int(np.argmax(target[0]))  # greedy: the first draft is accepted
    u = synth.philox_uniforms(0, 0, k)
    ur = synth.philox_uniforms(0, 1, k + 1)
    want = orc.accept(target, None if greedy else draft, dtok, T, greedy,
                      None if greedy else u, None if greedy else ur)
    bufs = {n: be.to_device(a) for n, a in dict(t=target, d=draft, dt=dtok, u=u, ur=ur,
                                                 h0=h0_rows(m)).items()}
    dh, acc, toks = be.alloc(m * H * 4), be.alloc(4), be.alloc(4 * (k + 1))
    dst = be.to_device(np.zeros(1, np.int32))
    for rep in range(3):
        be.verify_step_device(model40.stack, bufs["h0"], dh, m, bufs["t"],
                              None if greedy else bufs["d"], bufs["dt"], vocab, T, greedy,
                              None if greedy else bufs["u"], None if greedy else bufs["ur"],
                              acc, toks, dst)
        h = be.read(dh, np.float32, (m, H))
        a = int(be.read(acc, np.int32, (1,))[0])
        tk = be.read(toks, np.int32, (k + 1,))
        assert int(be.read(dst, np.int32, (1,))[0]) == 0
        assert np.array_equal(h, h_ref), f"step {rep}: h differs from the stack forward"
        assert (a, [int(v) for v in tk[: a + 1]]) == want
    for b in list(bufs.values()) + [dh, acc, toks, dst]:
        be.free(b)
