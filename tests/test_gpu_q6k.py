"""GPU parity of the Q6_K path and the LM head through the C ABI.

  * repack: lossless (download returns the uploaded bytes);
  * q6k_matvec (quantize_q8_k + q6_k_dot_pre, weights.rs:680-735,
    1023-1101): bit-identical to the oracle;
  * lm_head_logits: the same logits, plus per row the four candidates of
    top_logit_candidates (runtime/decode.rs:48-64) on those logits --
    descending, ties to the lower token, NaN never taken -- bit-identical,
    at the configs' vocabulary (151,936 x 2048)."""
import numpy as np
import pytest

import cpu_oracle as orc
from test_gpu_q4k import same_bits
from test_oracle import random_q6_k
from turboqwenfare_amd._lib import ERR_INVALID, HipError

pytestmark = pytest.mark.gpu


def q6_k_matrix(rows: int, cols: int, seed: int) -> np.ndarray:
    return random_q6_k(rows * (cols // 256), seed).reshape(-1)


def oracle_top4(logits: np.ndarray):
    toks, vals = [], []
    for row in logits:
        t, v = orc.top_logit_candidates(row)
        toks.append(t)
        vals.append(v)
    return np.array(toks, np.uint32), np.array(vals, np.float32)


@pytest.mark.parametrize("rows,cols", [(1, 256), (7, 512), (64, 2048), (65, 2304), (2048, 512),
                                       (3, 4096)])
def test_q6k_repack_is_lossless(backend, rows, cols):
    rng = np.random.default_rng(rows * 13 + cols)
    q = rng.integers(0, 256, size=rows * (cols // 256) * 210, dtype=np.uint8)
    w = backend.upload_q6_k(q, rows, cols)
    assert np.array_equal(backend.download_q6_k(w), q)
    assert backend.weights_bytes(w) >= q.nbytes
    backend.free_weights(w)


def test_q6k_rejects_bad_shapes_and_other_formats(backend):
    for rows, cols, n in ((1, 288, 420), (1, 256, 209), (2, 256, 210)):
        with pytest.raises(HipError) as e:
            backend.upload_q6_k(np.zeros(n, np.uint8), rows, cols)
        assert e.value.status == ERR_INVALID
    w6 = backend.upload_q6_k(q6_k_matrix(1, 256, 1), 1, 256)
    wk = backend.upload_q4_k(np.zeros(144, np.uint8), 1, 256)
    with pytest.raises(HipError) as e:
        backend.q4k_matvec(wk.__class__(w6.handle, 1, 256), np.ones(256, np.float32))
    assert e.value.status == ERR_INVALID
    with pytest.raises(HipError) as e:
        backend.q6k_matvec(w6.__class__(wk.handle, 1, 256), np.ones(256, np.float32))
    assert e.value.status == ERR_INVALID
    backend.free_weights(w6)
    backend.free_weights(wk)


def test_q6k_matvec_reference_kat(backend):
    # weights.rs:2532-2543: zero ql / qh, group scales 1, d = 1, x = ones
    b = np.zeros(210, np.uint8)
    b[192:208] = 1
    b[208:210] = (0x00, 0x3C)
    w = backend.upload_q6_k(b, 1, 256)
    assert backend.q6k_matvec(w, np.ones(256, np.float32))[0] == -8192.0
    backend.free_weights(w)


@pytest.mark.parametrize("rows,cols,m", [(1, 256, 1), (17, 512, 1), (512, 2048, 4),
                                         (2048, 512, 4), (65, 2304, 3), (130, 4096, 8),
                                         (200, 768, 2),
                                         # the streamed kernel (64 blocks a row): padded
                                         # super-blocks, padded rows, two token passes,
                                         # two rounds of row octets per wavefront
                                         (100, 1536, 3), (70, 2048, 8), (3001, 1792, 2),
                                         (20000, 2048, 2)])
def test_q6k_matvec_bit_identical(backend, rows, cols, m):
    w_bytes = q6_k_matrix(rows, cols, 3 * rows + cols)
    x = np.random.default_rng(rows + 7 * m).standard_normal((m, cols)).astype(np.float32)
    w = backend.upload_q6_k(w_bytes, rows, cols)
    got = backend.q6k_matvec(w, x)
    for t in range(m):
        want = orc.q6_k_matvec(w_bytes, rows, cols, x[t])
        assert same_bits(got[t], want), (t, np.flatnonzero(got[t] != want)[:5])
    backend.free_weights(w)


def test_q6k_matvec_extreme_scales_and_inputs(backend):
    rows, cols = 16, 768
    w_bytes = q6_k_matrix(rows, cols, 8).reshape(-1, 210)
    w_bytes[0, 208:210] = 0                  # d = 0
    w_bytes[1, 208:210] = (0xFF, 0x7B)       # d = 65504
    w_bytes[2, 192:208] = 0x80               # every scale -128
    w_bytes[3, 0:192] = 0xFF                 # q = 63 everywhere
    w_bytes = w_bytes.reshape(-1)
    x = np.random.default_rng(9).standard_normal(cols).astype(np.float32)
    x[0:256] = 0.0                           # an all-zero Q8_K chunk
    x[300] = np.nan                          # quantizes to 127
    x[600] = -np.inf
    w = backend.upload_q6_k(w_bytes, rows, cols)
    assert same_bits(backend.q6k_matvec(w, x), orc.q6_k_matvec(w_bytes, rows, cols, x))
    backend.free_weights(w)


def test_lm_head_candidates_ties_and_nan(backend):
    # rows with d = 0 give exactly 0.0 (ties broken by the lower token); rows
    # with d = NaN give NaN (never a candidate); the rest are negative
    rows, cols = 1000, 512
    w_bytes = q6_k_matrix(rows, cols, 10).reshape(rows, 2, 210)
    w_bytes[:, :, 208:210] = np.array([0.01], np.float16).view(np.uint8)
    w_bytes[:, :, 0:192] = 0x00              # q = 0 -> -32 * scale
    w_bytes[:, :, 192:208] = 1               # so every logit is -32 d sum(x) ...
    x = np.ones((3, cols), np.float32)       # ... negative for positive x
    for r in (5, 700, 41, 999, 600):
        w_bytes[r, :, 208:210] = 0           # logit 0.0: five ties
    for r in (2, 3):
        w_bytes[r, :, 208:210] = np.array([np.nan], np.float16).view(np.uint8)
    w_bytes = w_bytes.reshape(-1)
    w = backend.upload_q6_k(w_bytes, rows, cols)
    y, t4, l4 = backend.lm_head_logits(w, x)
    want = np.stack([orc.q6_k_matvec(w_bytes, rows, cols, x[t]) for t in range(3)])
    assert same_bits(y, want)
    tw, lw = oracle_top4(want)
    assert np.array_equal(t4, tw) and same_bits(l4, lw)
    assert list(t4[0]) == [5, 41, 600, 700]
    backend.free_weights(w)


@pytest.mark.parametrize("m", [1, 5])
def test_lm_head_candidates_ties_and_nan_streamed(backend, m):
    # the streamed kernel's per-lane lists: tied logits (0.0) in rows that one
    # lane meets in both of its rounds (5 and 16389, 16384 rows a round),
    # NaN rows in both rounds, the rest negative; m = 5 runs two token passes
    rows, cols = 20000, 2048
    w_bytes = q6_k_matrix(rows, cols, 14).reshape(rows, 8, 210)
    w_bytes[:, :, 208:210] = np.array([0.01], np.float16).view(np.uint8)
    w_bytes[:, :, 0:192] = 0x00
    w_bytes[:, :, 192:208] = 1
    x = np.ones((m, cols), np.float32)
    for r in (16389, 5, 19999, 600, 41):
        w_bytes[r, :, 208:210] = 0
    for r in (2, 16384):
        w_bytes[r, :, 208:210] = np.array([np.nan], np.float16).view(np.uint8)
    w_bytes = w_bytes.reshape(-1)
    w = backend.upload_q6_k(w_bytes, rows, cols)
    y, t4, l4 = backend.lm_head_logits(w, x)
    want = np.stack([orc.q6_k_matvec(w_bytes, rows, cols, x[t]) for t in range(m)])
    assert same_bits(y, want)
    tw, lw = oracle_top4(want)
    assert np.array_equal(t4, tw) and same_bits(l4, lw)
    assert list(t4[0]) == [5, 41, 600, 16389]
    backend.free_weights(w)


@pytest.mark.parametrize("m", [1, 4])
def test_lm_head_full_vocab(backend, m):
    # the configs' vocabulary and hidden size (Q6_K 151,936 x 2048, 255 MB)
    V, H = 151_936, 2048
    w_bytes = q6_k_matrix(V, H, 11)
    x = np.random.default_rng(12 + m).standard_normal((m, H)).astype(np.float32)
    w = backend.upload_q6_k(w_bytes, V, H)
    y, t4, l4 = backend.lm_head_logits(w, x)
    for t in range(m):
        want = orc.q6_k_matvec(w_bytes, V, H, x[t])
        assert same_bits(y[t], want), (t, np.flatnonzero(y[t] != want)[:5])
        tw, lw = orc.top_logit_candidates(want)
        assert list(t4[t]) == list(tw) and same_bits(l4[t], lw)
    # the device form writes the same
    d_x = backend.to_device(x)
    d_y, d_t, d_l = backend.alloc(m * V * 4), backend.alloc(m * 16), backend.alloc(m * 16)
    backend.lm_head_logits_device(w, d_x, m, d_y, d_t, d_l)
    assert same_bits(backend.read(d_y, np.float32, (m, V)), y)
    assert np.array_equal(backend.read(d_t, np.uint32, (m, 4)), t4)
    for b in (d_x, d_y, d_t, d_l):
        backend.free(b)
    backend.free_weights(w)
