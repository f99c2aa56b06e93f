"""GPU parity of the canonical Q4_K path (GGML 144-byte super-blocks) through
the C ABI against the CPU oracle on the same inputs.

  * repack: lossless (download returns the uploaded bytes);
  * q4k_gemv (backend::reference::q4k_gemv semantics, fp32): within 1e-5 of
    the reference metric |g - c| / max(|c|, 1) on the reference's fixture,
    within 1e-3 on random shapes whose sums reach ~1e3, and within twice
    the oracle's own fp32 error of the float64 value of the exact decode (the reference's test bound for its GPU kernel is 1e-2 absolute,
    kernels.rs:1140-1165);
  * q4k_matvec (quantize_q8_k + q4_k_dot_pre): bit-identical;
  * q4k_expert_forward (LoadedQwen36Expert::forward): within 1e-3 (the SwiGLU
    exponential is the device's expf)."""
import numpy as np
import pytest

import cpu_oracle as orc
from conftest import rel_err
from test_oracle import lcg_q4_k_weights, lcg_vector, q4_k_exact
from turboqwenfare_amd._lib import ERR_INVALID, HipError

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-5
FFN_TOL = 1e-3


def sane_q4_k(rows: int, cols: int, seed: int, d_range=(0.002, 0.05)) -> np.ndarray:
    """Random Q4_K bytes whose f16 d and dmin are finite and modest."""
    rng = np.random.default_rng(seed)
    n = rows * (cols // 256)
    blk = rng.integers(0, 256, size=(n, 144), dtype=np.uint8)
    d = rng.uniform(*d_range, size=n).astype(np.float16)
    dmin = rng.uniform(*d_range, size=n).astype(np.float16)
    blk[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    blk[:, 2:4] = dmin.view(np.uint8).reshape(n, 2)
    return blk.reshape(-1)


def exact_gemv(w: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    nb = cols // 256
    dq = np.concatenate([q4_k_exact(w[i * 144:(i + 1) * 144]) for i in range(rows * nb)])
    return dq.reshape(rows, cols) @ np.asarray(x, np.float64).T


def same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(nan | (a.view(np.uint32) == b.view(np.uint32))))


# ---- repack -------------------------------------------------------------------
@pytest.mark.parametrize("rows,cols", [(1, 256), (7, 512), (64, 2048), (65, 2304), (512, 2048),
                                       (2048, 512), (3, 4096)])
def test_q4k_repack_is_lossless(backend, rows, cols):
    rng = np.random.default_rng(rows * 7 + cols)
    q = rng.integers(0, 256, size=rows * (cols // 256) * 144, dtype=np.uint8)
    w = backend.upload_q4_k(q, rows, cols)
    assert np.array_equal(backend.download_q4_k(w), q)
    assert backend.weights_bytes(w) >= q.nbytes
    backend.free_weights(w)


def test_q4k_upload_rejects_bad_shapes(backend):
    # cols not a multiple of 256; a byte length that does not match the shape
    for rows, cols, n in ((1, 288, 288), (1, 256, 143), (2, 256, 144)):
        with pytest.raises(HipError) as e:
            backend.upload_q4_k(np.zeros(n, np.uint8), rows, cols)
        assert e.value.status == ERR_INVALID


def test_formats_are_not_interchangeable(backend):
    wk = backend.upload_q4_k(lcg_q4_k_weights(1, 256), 1, 256)
    w0 = backend.upload_q4_0(np.zeros(8 * 18, np.uint8), 1, 256)
    with pytest.raises(HipError) as e:
        backend.q4_gemv(w0.__class__(wk.handle, 1, 256), np.ones(256, np.float32))
    assert e.value.status == ERR_INVALID
    with pytest.raises(HipError) as e:
        backend.q4k_matvec(wk.__class__(w0.handle, 1, 256), np.ones(256, np.float32))
    assert e.value.status == ERR_INVALID
    with pytest.raises(HipError):
        backend.download_q4_0(w0.__class__(wk.handle, 1, 256))
    backend.free_weights(wk)
    backend.free_weights(w0)


# ---- fp32-semantics GEMV (backend::reference::q4k_gemv) -------------------------
def test_q4k_gemv_dequant_kat(backend):
    # dequant.rs:287-306: d = 1, dmin = 0, every sub-block scale 1, qs[0] = 0x12
    b = np.zeros(144, np.uint8)
    b[0:2] = (0x00, 0x3C)
    b[4:12] = 1
    b[16] = 0x12
    w = backend.upload_q4_k(b, 1, 256)
    eye = np.eye(256, dtype=np.float32)
    assert backend.q4k_gemv(w, eye[0])[0] == 2.0
    assert backend.q4k_gemv(w, eye[32])[0] == 1.0
    assert backend.q4k_gemv(w, eye[1])[0] == 0.0
    backend.free_weights(w)


def test_q4k_gemv_reference_fixture(backend):
    # kernels.rs:1140-1165: the LCG fixture, 17 x 512, x = (i % 11) 0.3 - 1.5
    rows, cols = 17, 512
    w_bytes = lcg_q4_k_weights(rows, cols)
    x = lcg_vector(cols)
    w = backend.upload_q4_k(w_bytes, rows, cols)
    got = backend.q4k_gemv(w, x)
    assert rel_err(got, orc.q4k_gemv(w_bytes, rows, cols, x)) < GEMV_TOL
    assert rel_err(got, exact_gemv(w_bytes, rows, cols, x)) < GEMV_TOL
    assert np.max(np.abs(got - exact_gemv(w_bytes, rows, cols, x))) < 1e-2
    backend.free_weights(w)


def test_q4k_gemv_one_hot_probe(backend):
    # kernels.rs:1168-1196: x = e_k returns decoded element k (to 1 ulp here)
    w_bytes = lcg_q4_k_weights(8, 256)
    w = backend.upload_q4_k(w_bytes, 8, 256)
    dense = np.stack([orc.dequantize_q4_k(w_bytes[r * 144:(r + 1) * 144]) for r in range(8)])
    eye = np.eye(256, dtype=np.float32)
    for k0 in range(0, 256, 8):
        y = backend.q4k_gemv(w, eye[k0:k0 + 8])
        want = dense[:, k0:k0 + 8].T
        assert np.all(np.abs(y - want) <= 2.0 ** -22 * np.maximum(np.abs(want), 1.0)), k0
    backend.free_weights(w)


@pytest.mark.parametrize("rows,cols,m", [(1, 256, 1), (64, 2048, 1), (512, 2048, 4),
                                         (2048, 512, 3), (65, 2304, 2), (130, 4096, 8),
                                         (200, 768, 5)])
def test_q4k_gemv_shape_sweep(backend, rows, cols, m):
    w_bytes = sane_q4_k(rows, cols, rows + cols + m)
    x = np.random.default_rng(m).standard_normal((m, cols)).astype(np.float32)
    w = backend.upload_q4_k(w_bytes, rows, cols)
    got = backend.q4k_gemv(w, x)
    want = np.stack([orc.q4k_gemv(w_bytes, rows, cols, x[t]) for t in range(m)])
    exact = exact_gemv(w_bytes, rows, cols, x).T
    # sums reach ~1e3 here, so the oracle's own sequential fp32 sum is ~1e-3
    # off the exact value; the device's error (activations held to 2^-23 of
    # each 32-block's max, chunked fp32 sums) must stay within twice that
    assert rel_err(got, want) < FFN_TOL
    err_gpu = np.max(np.abs(got - exact))
    err_orc = np.max(np.abs(want - exact))
    print(rows, cols, m, "max |gpu - exact|", err_gpu, "max |oracle - exact|", err_orc)
    assert err_gpu <= max(2 * err_orc, 1e-4)
    backend.free_weights(w)


def test_q4k_gemv_propagates_non_finite_input(backend):
    w_bytes = sane_q4_k(64, 512, 3)
    w = backend.upload_q4_k(w_bytes, 64, 512)
    x = np.ones(512, np.float32)
    x[300] = np.nan
    assert np.all(np.isnan(backend.q4k_gemv(w, x)))
    backend.free_weights(w)


# ---- Q8_K integer matvec (quantize_q8_k + q4_k_dot_pre): bit-identical ---------
@pytest.mark.parametrize("rows,cols,m", [(1, 256, 1), (17, 512, 1), (512, 2048, 4),
                                         (2048, 512, 4), (65, 2304, 3), (130, 4096, 8),
                                         (200, 768, 2)])
def test_q4k_matvec_bit_identical(backend, rows, cols, m):
    w_bytes = sane_q4_k(rows, cols, 11 * rows + cols)
    x = np.random.default_rng(rows + m).standard_normal((m, cols)).astype(np.float32)
    w = backend.upload_q4_k(w_bytes, rows, cols)
    got = backend.q4k_matvec(w, x)
    for t in range(m):
        want = orc.q4_k_matvec(w_bytes, rows, cols, x[t])
        assert same_bits(got[t], want), (t, np.flatnonzero(got[t] != want)[:5])
    backend.free_weights(w)


def test_q4k_matvec_reference_fixture(backend):
    rows, cols = 17, 512
    w_bytes = lcg_q4_k_weights(rows, cols)
    w = backend.upload_q4_k(w_bytes, rows, cols)
    x = lcg_vector(cols)
    assert same_bits(backend.q4k_matvec(w, x), orc.q4_k_matvec(w_bytes, rows, cols, x))
    backend.free_weights(w)


def test_q4k_matvec_quantizer_edge_cases(backend):
    # chunks of: all zeros; ties after scaling (signed maximum -127 -> inverse 1);
    # a repeated maximum of both signs (the first one sets the sign); a NaN
    # (never the maximum, quantizes to 127); an infinity (inverse -0, NaN
    # products -> 127); subnormal values only
    cols = 256 * 6
    x = np.random.default_rng(5).standard_normal(cols).astype(np.float32)
    x[0:256] = 0.0
    x[256:512] = np.float32(0.5) + np.arange(256, dtype=np.float32) % 7 - 3
    x[256 + 17] = -127.0
    x[512:768] = np.random.default_rng(6).uniform(-2, 2, 256).astype(np.float32)
    x[512 + 40] = 3.0
    x[512 + 9] = -3.0
    x[768 + 5] = np.nan
    x[1024 + 100] = np.inf
    x[1280:1536] = np.float32(1e-40) * np.arange(256, dtype=np.float32) % 5
    rows = 64
    w_bytes = sane_q4_k(rows, cols, 77)
    w = backend.upload_q4_k(w_bytes, rows, cols)
    assert same_bits(backend.q4k_matvec(w, x), orc.q4_k_matvec(w_bytes, rows, cols, x))
    backend.free_weights(w)


def test_q4k_matvec_zero_and_extreme_scales(backend):
    rows, cols = 16, 512
    w_bytes = sane_q4_k(rows, cols, 9).reshape(-1, 144)
    w_bytes[0, 0:4] = 0                          # d = dmin = 0
    w_bytes[1, 0:2] = (0xFF, 0x7B)               # d = 65504 (largest f16)
    w_bytes[2, 2:4] = (0x01, 0x00)               # dmin = smallest subnormal
    w_bytes[3, 4:16] = 0xFF                      # every 6-bit scale and min 63
    w_bytes = w_bytes.reshape(-1)
    x = np.random.default_rng(10).standard_normal(cols).astype(np.float32)
    w = backend.upload_q4_k(w_bytes, rows, cols)
    assert same_bits(backend.q4k_matvec(w, x), orc.q4_k_matvec(w_bytes, rows, cols, x))
    backend.free_weights(w)


def test_q4k_batched_match_single(backend):
    rows, cols = 512, 2048
    ws_bytes = [sane_q4_k(rows, cols, 100 + i) for i in range(4)]
    ws = [backend.upload_q4_k(b, rows, cols) for b in ws_bytes]
    x = np.random.default_rng(1).standard_normal(cols).astype(np.float32)
    d_x = backend.to_device(x)
    d_y = backend.alloc(4 * rows * 4)
    backend.q4k_gemv_batched_device(ws, d_x, d_y)
    yg = backend.read(d_y, np.float32, (4, rows))
    backend.q4k_matvec_batched_device(ws, d_x, d_y)
    ym = backend.read(d_y, np.float32, (4, rows))
    for i, w in enumerate(ws):
        assert same_bits(yg[i], backend.q4k_gemv(w, x))
        assert same_bits(ym[i], orc.q4_k_matvec(ws_bytes[i], rows, cols, x))
        backend.free_weights(w)
    backend.free(d_x)
    backend.free(d_y)


# ---- Q4_K expert (LoadedQwen36Expert::forward) -----------------------------------
@pytest.mark.parametrize("m", [1, 4])
def test_q4k_expert_forward_parity(backend, m):
    H, F = 2048, 512
    gate_b, up_b = sane_q4_k(F, H, 1), sane_q4_k(F, H, 2)
    down_b = sane_q4_k(H, F, 3)
    gate, up, down = (backend.upload_q4_k(gate_b, F, H), backend.upload_q4_k(up_b, F, H),
                      backend.upload_q4_k(down_b, H, F))
    x = np.random.default_rng(m).standard_normal((m, H)).astype(np.float32)
    got = backend.q4k_expert_forward(gate, up, down, x)
    for t in range(m):
        want = orc.q4_k_expert_forward(gate_b, up_b, down_b, H, F, x[t])
        assert rel_err(got[t], want) < FFN_TOL
    for w in (gate, up, down):
        backend.free_weights(w)
