"""Routed-expert superextents of a hand-assembled .tqf container to the
device (tqf_hip_expert_upload): load_expert's checks
(model/qwen36/weights.rs:1404-1428), payload_parts (:552-561) and three Q4_K
uploads (stage_expert_values, experts/mod.rs:512-545).  The downloaded
matrices equal the payload bytes, and the uploaded expert's forward equals
the oracle's Q4_K expert on the same bytes; every rejected expert leaves
nothing allocated and the context usable."""
import numpy as np
import pytest

import cpu_oracle as orc
import tqf_fixture as fx
from conftest import rel_err
from turboqwenfare_amd import _lib, container, synth

pytestmark = pytest.mark.gpu

H, F = 2048, 512


def expert_parts(seed):
    return (synth.centered_q4_k(F, H, seed).tobytes(), synth.centered_q4_k(F, H, seed + 1).tobytes(),
            synth.centered_q4_k(H, F, seed + 2).tobytes())


@pytest.mark.parametrize("width", [None, 128, 64, 256], ids=["canonical", "n128", "n64", "n256"])
def test_upload_round_trips_and_computes(backend, width):
    p = expert_parts(40 + (width or 0))
    data, blob, _ = fx.build([dict(layer=7, expert=33, parts=expert_parts(1)),
                              dict(layer=7, expert=34, parts=p, width=width)])
    with container.ExpertTable(blob, 2, len(data), 16) as t:
        stored, device = t.reserve_bytes(7, 34)
        assert stored == len(p[0]) + len(p[1]) + len(p[2])
        g, u, d = t.upload(backend, 7, 34, data)
    try:
        got = [backend.download_q4_k(w).tobytes() for w in (g, u, d)]
        assert got == list(p), "payload parts"
        assert device == sum(backend.q4k_weights_bytes_for(w.rows, w.cols) for w in (g, u, d))
        x = synth.normal((2, H), seed=5)
        y = backend.q4k_expert_forward(g, u, d, x)
        for r in range(2):
            want = orc.q4_k_expert_forward(np.frombuffer(p[0], np.uint8), np.frombuffer(p[1], np.uint8),
                                           np.frombuffer(p[2], np.uint8), H, F, x[r])
            assert rel_err(y[r], want) < 1e-3
    finally:
        for w in (g, u, d):
            backend.free_weights(w)


def test_upload_rejects_what_load_expert_rejects(backend):
    good = expert_parts(60)
    bad_layout = dict(layer=0, expert=1, parts=good, layout_id=1)
    bad_tile_layout = dict(layer=0, expert=2, parts=good, tile_layout_id=1)
    short = dict(layer=0, expert=3, parts=(good[0], good[1], good[2][:-144]))
    data, blob, meta = fx.build([bad_layout, bad_tile_layout, short, dict(layer=0, expert=4, parts=good)])
    # expert 4 with its GateUp tile ending inside the down region: a
    # contiguous partition (the reader accepts it) that is not matrix-true
    tiles4 = meta[3][0][6]
    b = bytearray(blob)
    t0, t1 = 4 * 32 + tiles4 * 24, 4 * 32 + (tiles4 + 1) * 24
    b[t0 + 12:t0 + 16] = fx.le(2 * fx.GATE_BYTES + 144, 4)       # GateUp grows by one block
    b[t1 + 8:t1 + 12] = fx.le(2 * fx.GATE_BYTES + 144, 4)        # Down starts later
    b[t1 + 12:t1 + 16] = fx.le(fx.DOWN_BYTES - 144, 4)
    with container.ExpertTable(bytes(b), 4, len(data), 16) as t:
        for e in (1, 2, 3, 4):
            with pytest.raises(_lib.HipError) as err:
                t.upload(backend, 0, e, data)
            assert err.value.status == _lib.ERR_INVALID
        with pytest.raises(_lib.HipError):  # the container region is too short
            t.upload(backend, 0, 4, data[:meta[3][0][4] + 100])
    # the context still works
    w = backend.upload_q4_k(np.frombuffer(good[0], np.uint8), F, H)
    assert backend.download_q4_k(w).tobytes() == good[0]
    backend.free_weights(w)
