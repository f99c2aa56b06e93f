"""The allocation-free acceptance entry point (tqf_hip_accept_device_noalloc)
against tqf_hip_accept_device through the C ABI: identical accepted length
and token buffers, bit for bit, on two calls in a row (the second with a
smaller k and vocabulary, so it reuses the fixed scratch left by the first),
in stochastic and greedy modes; sizes beyond the fixed scratch are rejected."""
import numpy as np
import pytest

from turboqwenfare_amd import synth
from turboqwenfare_amd._lib import ERR_INVALID, HipError

pytestmark = pytest.mark.gpu


def _inputs(k, vocab, seed):
    rng = np.random.default_rng(seed)
    target = (rng.standard_normal((k + 1, vocab)) * 3.0).astype(np.float32)
    draft = (rng.standard_normal((k, vocab)) * 3.0).astype(np.float32)
    dtok = np.argmax(draft, axis=1).astype(np.int32)
    if k:
        dtok[0] = int(np.argmax(target[0]))
    return target, draft, dtok, synth.philox_uniforms(seed, 0, max(k, 1)), \
        synth.philox_uniforms(seed, 1, k + 1)


def _run(be, noalloc, k, vocab, greedy, bufs):
    acc, toks = be.to_device(np.full(1, -7, np.int32)), be.to_device(np.full(k + 1, -7, np.int32))
    fn = be.accept_device_noalloc if noalloc else be.accept_device
    fn(bufs["t"], None if greedy else bufs["d"], bufs["dt"] if k else None, k, vocab, 0.7, greedy,
       None if greedy else bufs["u"], None if greedy else bufs["ur"], acc, toks)
    out = int(be.read(acc, np.int32, (1,))[0]), be.read(toks, np.int32, (k + 1,)).copy()
    be.free(acc)
    be.free(toks)
    return out


@pytest.mark.parametrize("greedy", [False, True], ids=["stochastic", "greedy"])
def test_noalloc_accept_equals_accept_device(backend, greedy):
    for k, vocab, seed in ((3, 151936, 5), (1, 40000, 6)):  # the second call is smaller
        target, draft, dtok, u, ur = _inputs(k, vocab, seed)
        bufs = {n: backend.to_device(a) for n, a in dict(t=target, d=draft, dt=dtok, u=u, ur=ur).items()}
        want = _run(backend, False, k, vocab, greedy, bufs)
        got = _run(backend, True, k, vocab, greedy, bufs)
        assert got[0] == want[0] and np.array_equal(got[1], want[1]), (k, vocab, got, want)
        for b in bufs.values():
            backend.free(b)


def test_noalloc_accept_rejects_sizes_beyond_its_scratch(backend):
    tiny = backend.to_device(np.zeros(16, np.float32))
    out = backend.to_device(np.zeros(8, np.int32))
    with pytest.raises(HipError) as e:
        backend.accept_device_noalloc(tiny, None, out, 7, 8_000_000, 0.7, True, None, None, out, out)
    assert e.value.status == ERR_INVALID
    backend.free(tiny)
    backend.free(out)
