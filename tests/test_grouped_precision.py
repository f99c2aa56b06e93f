"""Why the grouped GEMM's down projection runs two bf16 MFMAs per k step.

The down GEMM's A operand is the SwiGLU output h, computed in fp32.  As one
bf16 value h keeps 8 significant bits; the down sums then cancel (|y| is far
below the sum of |w h| terms), so bf16 h alone moves y by ~5e-2 of the
reference metric |g - c| / max(|c|, 1) (backend/metal/expert.rs:309) at
config-5 shapes, far outside the 1e-3 the GPU tests hold the grouped GEMM to.
h = hi + lo as two bf16 values keeps 16 bits and lands near 1e-4: the
kernel (tqf_grouped.hip) therefore issues the second MFMA.  CPU only, on
Q4_0-shaped random weights."""
import numpy as np

H, F, T = 2048, 512, 16


def bf16(a):
    b = np.ascontiguousarray(a, np.float32).view(np.uint32)
    return ((b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)


def q4_like(rng, rows, cols):
    q = rng.integers(0, 16, (rows, cols)).astype(np.float32) - 8
    d = (0.005 + 0.015 * rng.random((rows, cols // 32))).astype(np.float32)
    return q * np.repeat(d, 32, axis=1)


def test_bf16_rounding_is_round_to_nearest_even():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -9, -3.0, 0.0], np.float32)
    assert bf16(x).tolist() == [1.0, 1.0, 1.0 + 2 ** -7, -3.0, 0.0]


def test_down_needs_h_as_bf16_hi_plus_lo():
    rng = np.random.default_rng(0)
    wg, wu, wd = q4_like(rng, F, H), q4_like(rng, F, H), q4_like(rng, H, F)
    x = rng.standard_normal((T, H)).astype(np.float32)
    g, u = x @ wg.T, x @ wu.T
    h = (g / (1 + np.exp(-g))) * u
    hi = bf16(h)
    lo = bf16(h - hi)
    y = h.astype(np.float64) @ wd.T.astype(np.float64)

    def err(hh):
        yy = hh.astype(np.float64) @ wd.T.astype(np.float64)
        return float(np.max(np.abs(yy - y) / np.maximum(np.abs(y), 1.0)))

    assert err(hi) > 1e-2
    assert err(hi + lo) < 2e-4
