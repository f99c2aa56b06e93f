"""TEST INFRASTRUCTURE ONLY: ctypes wrapper of the CPU oracle
(``oracle/libtqf_oracle.so``, built from ``oracle/tqf_oracle.c``).

Only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
load this module; the product never does.  See ``tqf_oracle.h`` for the
reference file:line each function restates and what pins it.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libtqf_oracle.so"

_vp = C.c_void_p
_u32 = C.c_uint32
_i32 = C.c_int32
_f32 = C.c_float
_u64 = C.c_uint64


class _MoeLayer(C.Structure):
    _fields_ = [
        ("router", _vp), ("shared_input_gate", _vp), ("shared_gate", _vp), ("shared_up", _vp),
        ("shared_down", _vp), ("routed_gate", _vp), ("routed_up", _vp), ("routed_down", _vp),
        ("n_experts", _u32), ("hidden", _u32), ("width", _u32),
    ]


class _Xoshiro(C.Structure):
    _fields_ = [("s", _u64 * 4)]


_SIGS = {
    "orc_f16_to_f32": (_f32, [C.c_uint16]),
    "orc_f16_to_f32_indep": (_f32, [C.c_uint16]),
    "orc_f32_to_f16": (C.c_uint16, [_f32]),
    "orc_dequantize_q4_0": (None, [_vp, _vp]),
    "orc_dequantize_q4_0_indep": (None, [_vp, _vp]),
    "orc_q4_0_matvec": (_i32, [_vp, C.c_size_t, _u32, _u32, _vp, _vp]),
    "orc_f32_matvec": (None, [_vp, _u32, _u32, _vp, _vp]),
    "orc_router_from_logits": (_i32, [_vp, _u32, _vp, _vp]),
    "orc_router_validate": (_i32, [_vp, _vp]),
    "orc_silu_mul": (None, [_vp, _vp, _vp, _u32]),
    "orc_qwen_rmsnorm": (None, [_vp, _vp, _u32, _vp]),
    "orc_sigmoid": (_f32, [_f32]),
    "orc_expert_forward": (_i32, [_vp, _vp, _vp, _u32, _u32, _vp, _vp]),
    "orc_moe_forward_batch": (_i32, [C.POINTER(_MoeLayer), _vp, _u32, _vp, _vp, _vp, C.c_int]),
    "orc_moe_forward_batch_q4k": (_i32, [C.POINTER(_MoeLayer), _vp, _u32, _vp, _vp, _vp, C.c_int]),
    "orc_batch_union": (_u32, [_vp, _u32, _vp]),
    "orc_top_logit_candidates": (None, [_vp, _u32, _vp, _vp]),
    "orc_softmax_draw": (_u32, [_vp, _u32, _f32, _f32]),
    "orc_softmax_draw_sums": (_u32, [_vp, _u32, _f32, _f32, _vp, _vp]),
    "orc_xoshiro_seed": (None, [C.POINTER(_Xoshiro), _u64]),
    "orc_xoshiro_next_u64": (_u64, [C.POINTER(_Xoshiro)]),
    "orc_xoshiro_next_f32": (_f32, [C.POINTER(_Xoshiro)]),
    "orc_philox4x32_10": (None, [_vp, _vp, _vp]),
    "orc_routed_combine": (_i32, [_vp, _vp, _u32, _vp, _vp, _vp, C.c_int]),
    "orc_accept": (_i32, [_vp, _vp, _vp, _u32, _u32, _f32, C.c_int, _vp, _vp, _vp, _vp]),
    "orc_accept_exp": (_f32, [_f32]),
    "orc_fix40": (_u64, [_f32]),
    "orc_fix62": (_u64, [_f32]),
    "orc_u64_to_f32": (_f32, [_u64]),
    "orc_scale_floor": (_u64, [_u64, _f32]),
    "orc_dequantize_q4_k": (None, [_vp, _vp]),
    "orc_dequantize_q4_k_indep": (None, [_vp, _vp]),
    "orc_q4k_gemv": (_i32, [_vp, _u32, _u32, _vp, _vp]),
    "orc_quantize_q8_k": (None, [_vp, _vp, _vp, _vp]),
    "orc_q4_k_dot_pre": (_f32, [_vp, _u32, _vp, _vp, _vp]),
    "orc_q4_k_matvec": (_i32, [_vp, _u32, _u32, _vp, _vp]),
    "orc_dequantize_q6_k": (None, [_vp, _vp]),
    "orc_q6_k_dot_pre": (_f32, [_vp, _u32, _vp, _vp]),
    "orc_q6_k_matvec": (_i32, [_vp, _u32, _u32, _vp, _vp]),
}

_LIB = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def _f32a(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- a1/a2 -------------------------------------------------------------------
def f16_to_f32(bits: int) -> float:
    return lib().orc_f16_to_f32(bits)


def f16_to_f32_indep(bits: int) -> float:
    return lib().orc_f16_to_f32_indep(bits)


def f32_to_f16(v: float) -> int:
    return lib().orc_f32_to_f16(v)


def dequantize_q4_0(block: bytes | np.ndarray, independent: bool = False) -> np.ndarray:
    b = np.frombuffer(bytes(block), dtype=np.uint8) if not isinstance(block, np.ndarray) \
        else np.ascontiguousarray(block, dtype=np.uint8)
    out = np.empty(32, dtype=np.float32)
    fn = lib().orc_dequantize_q4_0_indep if independent else lib().orc_dequantize_q4_0
    fn(_p(b), _p(out))
    return out


# ---- a3/a5 -------------------------------------------------------------------
def q4_0_matvec(w: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = _f32a(x)
    y = np.empty(rows, dtype=np.float32)
    if lib().orc_q4_0_matvec(_p(w), w.nbytes, rows, cols, _p(x), _p(y)) != 0:
        raise ValueError("shape error (ModelError::Shape)")
    return y


def f32_matvec(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    w = _f32a(w)
    x = _f32a(x)
    rows, cols = w.shape
    y = np.empty(rows, dtype=np.float32)
    lib().orc_f32_matvec(_p(w), rows, cols, _p(x), _p(y))
    return y


# ---- a6 ----------------------------------------------------------------------
def router_from_logits(logits: np.ndarray):
    lg = _f32a(logits)
    ids = np.empty(8, dtype=np.uint16)
    w = np.empty(8, dtype=np.float32)
    if lib().orc_router_from_logits(_p(lg), lg.size, _p(ids), _p(w)) != 0:
        raise ValueError("router error")
    return ids, w


def router_validate(ids, weights) -> bool:
    i = np.ascontiguousarray(ids, dtype=np.uint16)
    w = _f32a(weights)
    return lib().orc_router_validate(_p(i), _p(w)) == 0


# ---- a7/a21 ------------------------------------------------------------------
def silu_mul(g, u) -> np.ndarray:
    g = _f32a(g)
    u = _f32a(u)
    out = np.empty_like(g)
    lib().orc_silu_mul(_p(g), _p(u), _p(out), g.size)
    return out


def qwen_rmsnorm(x, w) -> np.ndarray:
    x = _f32a(x)
    w = _f32a(w)
    out = np.empty_like(x)
    lib().orc_qwen_rmsnorm(_p(x), _p(w), x.size, _p(out))
    return out


def sigmoid(v: float) -> float:
    return lib().orc_sigmoid(v)


# ---- a10 ---------------------------------------------------------------------
def expert_forward(gate, up, down, hidden: int, width: int, x) -> np.ndarray:
    g = np.ascontiguousarray(gate, dtype=np.uint8)
    u = np.ascontiguousarray(up, dtype=np.uint8)
    d = np.ascontiguousarray(down, dtype=np.uint8)
    x = _f32a(x)
    y = np.empty(hidden, dtype=np.float32)
    if lib().orc_expert_forward(_p(g), _p(u), _p(d), hidden, width, _p(x), _p(y)) != 0:
        raise ValueError("shape error")
    return y


# ---- a11/a12 -----------------------------------------------------------------
class MoeLayerHost:
    """Host copies of one layer's tensors (f32 router; expert matrices as
    GGML Q4_0 bytes, or Q4_K bytes with fmt="q4_k")."""

    def __init__(self, router, shared_input_gate, shared_gate, shared_up, shared_down,
                 routed_gate, routed_up, routed_down, hidden=2048, width=512, fmt="q4_0"):
        if fmt not in ("q4_0", "q4_k"):
            raise ValueError("fmt must be 'q4_0' or 'q4_k'")
        self.fmt = fmt
        self.router = _f32a(router)
        self.shared_input_gate = _f32a(shared_input_gate)
        self.shared = [np.ascontiguousarray(a, dtype=np.uint8)
                       for a in (shared_gate, shared_up, shared_down)]
        self.routed_gate = [np.ascontiguousarray(a, dtype=np.uint8) for a in routed_gate]
        self.routed_up = [np.ascontiguousarray(a, dtype=np.uint8) for a in routed_up]
        self.routed_down = [np.ascontiguousarray(a, dtype=np.uint8) for a in routed_down]
        self.hidden = hidden
        self.width = width
        E = len(self.routed_gate)
        self._g = (_vp * E)(*[_p(a) for a in self.routed_gate])
        self._u = (_vp * E)(*[_p(a) for a in self.routed_up])
        self._d = (_vp * E)(*[_p(a) for a in self.routed_down])
        self._s = _MoeLayer(_p(self.router), _p(self.shared_input_gate), _p(self.shared[0]),
                            _p(self.shared[1]), _p(self.shared[2]), C.cast(self._g, _vp),
                            C.cast(self._u, _vp), C.cast(self._d, _vp), E, hidden, width)

    def forward_batch(self, x: np.ndarray, nthreads: int = 1):
        x = _f32a(x)
        if x.ndim == 1:
            x = x.reshape(1, -1)
        m = x.shape[0]
        y = np.empty((m, self.hidden), dtype=np.float32)
        ids = np.empty((m, 8), dtype=np.uint16)
        w = np.empty((m, 8), dtype=np.float32)
        fn = lib().orc_moe_forward_batch_q4k if self.fmt == "q4_k" else lib().orc_moe_forward_batch
        if fn(C.byref(self._s), _p(x), m, _p(y), _p(ids), _p(w), nthreads) != 0:
            raise ValueError("router error")
        return y, ids, w


    def routed_combine(self, x: np.ndarray, ids: np.ndarray, w: np.ndarray,
                       nthreads: int = 1) -> np.ndarray:
        """y[t] = sum_k w[t,k] * expert_{ids[t,k]}(x[t]) in route order."""
        if self.fmt != "q4_0":
            raise ValueError("routed_combine reads Q4_0 experts")
        x = _f32a(x)
        ids = np.ascontiguousarray(ids, dtype=np.uint16)
        w = _f32a(w)
        t = x.shape[0]
        y = np.empty((t, self.hidden), dtype=np.float32)
        if lib().orc_routed_combine(C.byref(self._s), _p(x), t, _p(ids), _p(w), _p(y),
                                    nthreads) != 0:
            raise ValueError("expert id out of range")
        return y


def batch_union(ids: np.ndarray) -> list[int]:
    i = np.ascontiguousarray(ids, dtype=np.uint16)
    out = np.empty(i.size, dtype=np.uint16)
    n = lib().orc_batch_union(_p(i), i.shape[0], _p(out))
    return [int(v) for v in out[:n]]


# ---- a16/a17/a18 -------------------------------------------------------------
def top_logit_candidates(logits):
    lg = _f32a(logits)
    toks = np.empty(4, dtype=np.uint32)
    vals = np.empty(4, dtype=np.float32)
    lib().orc_top_logit_candidates(_p(lg), lg.size, _p(toks), _p(vals))
    return toks, vals


def softmax_draw(logits, temperature: float, u: float) -> int:
    lg = _f32a(logits)
    return int(lib().orc_softmax_draw(_p(lg), lg.size, temperature, u))


def softmax_draw_sums(logits, temperature: float, u: float):
    """(token, total, psum): the draw with its token-order sum of the
    exponentials and its sorted-order sum of the probabilities."""
    lg = _f32a(logits)
    t, ps = C.c_float(), C.c_float()
    tok = int(lib().orc_softmax_draw_sums(_p(lg), lg.size, temperature, u, C.byref(t), C.byref(ps)))
    return tok, np.float32(t.value), np.float32(ps.value)


class Xoshiro:
    def __init__(self, seed: int | None = None, state=None):
        self._st = _Xoshiro()
        if state is not None:
            for i in range(4):
                self._st.s[i] = state[i]
        else:
            lib().orc_xoshiro_seed(C.byref(self._st), seed or 0)

    def next_u64(self) -> int:
        return int(lib().orc_xoshiro_next_u64(C.byref(self._st)))

    def next_f32(self) -> float:
        return float(lib().orc_xoshiro_next_f32(C.byref(self._st)))


def philox4x32_10(ctr, key) -> np.ndarray:
    c = np.ascontiguousarray(ctr, dtype=np.uint32)
    k = np.ascontiguousarray(key, dtype=np.uint32)
    out = np.empty(4, dtype=np.uint32)
    lib().orc_philox4x32_10(_p(c), _p(k), _p(out))
    return out


# ---- a22 ---------------------------------------------------------------------
def accept(target, draft, draft_tokens, temperature: float, greedy: bool, u=None, u_resample=None):
    t = _f32a(target)
    kp1, vocab = t.shape
    k = kp1 - 1
    d = None if draft is None else _f32a(draft)
    dt = np.ascontiguousarray(np.asarray(draft_tokens, dtype=np.int32).reshape(-1))
    uu = None if u is None else _f32a(u)
    ur = None if u_resample is None else _f32a(u_resample)
    acc = C.c_int32()
    toks = np.empty(k + 1, dtype=np.int32)
    rc = lib().orc_accept(_p(t), None if d is None else _p(d), _p(dt) if k else None, k, vocab,
                          temperature, 1 if greedy else 0, None if uu is None else _p(uu),
                          None if ur is None else _p(ur), C.byref(acc), _p(toks))
    if rc != 0:
        raise ValueError("invalid acceptance arguments")
    a = acc.value
    return a, [int(v) for v in toks[: a + 1]]


def accept_exp(z: float) -> float:
    return lib().orc_accept_exp(z)


def fix40(v: float) -> int:
    return int(lib().orc_fix40(v))


def fix62(v: float) -> int:
    return int(lib().orc_fix62(v))


def u64_to_f32(v: int) -> float:
    return lib().orc_u64_to_f32(v)


def scale_floor(total: int, u: float) -> int:
    return int(lib().orc_scale_floor(total, u))


# ---- f1 / a4 / a20: Q4_K -------------------------------------------------------
Q4_K_BLOCK_BYTES = 144
Q4_K_BLOCK_ELEMS = 256


def dequantize_q4_k(block, independent: bool = False) -> np.ndarray:
    b = np.ascontiguousarray(np.frombuffer(bytes(block), dtype=np.uint8) if not isinstance(block, np.ndarray)
                             else block, dtype=np.uint8)
    out = np.empty(256, dtype=np.float32)
    fn = lib().orc_dequantize_q4_k_indep if independent else lib().orc_dequantize_q4_k
    fn(_p(b), _p(out))
    return out


def q4k_gemv(w: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    """backend/reference.rs:49-67: fp32 dequantize-and-accumulate per row."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = _f32a(x)
    y = np.empty(rows, dtype=np.float32)
    if lib().orc_q4k_gemv(_p(w), rows, cols, _p(x), _p(y)) != 0:
        raise ValueError("cols must be a multiple of 256")
    return y


def quantize_q8_k(values) -> tuple[np.ndarray, np.ndarray, float]:
    v = _f32a(values)
    assert v.size == 256
    q = np.empty(256, dtype=np.int8)
    sums = np.empty(16, dtype=np.int16)
    scale = np.zeros(1, dtype=np.float32)
    lib().orc_quantize_q8_k(_p(v), _p(q), _p(sums), _p(scale))
    return q, sums, float(scale[0])


def q4_k_dot_pre(row: np.ndarray, q8: np.ndarray, sums: np.ndarray, scales: np.ndarray) -> float:
    row = np.ascontiguousarray(row, dtype=np.uint8)
    q8 = np.ascontiguousarray(q8, dtype=np.int8)
    sums = np.ascontiguousarray(sums, dtype=np.int16)
    scales = _f32a(scales)
    return float(lib().orc_q4_k_dot_pre(_p(row), scales.size, _p(q8), _p(sums), _p(scales)))


def q4_k_matvec(w: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    """weights.rs:680-735 with the Q4_K branch: Q8_K activations, integer dot."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = _f32a(x)
    y = np.empty(rows, dtype=np.float32)
    if lib().orc_q4_k_matvec(_p(w), rows, cols, _p(x), _p(y)) != 0:
        raise ValueError("cols must be a multiple of 256")
    return y


def q4_k_expert_forward(gate: np.ndarray, up: np.ndarray, down: np.ndarray, hidden: int,
                        width: int, x: np.ndarray) -> np.ndarray:
    """LoadedQwen36Expert::forward (weights.rs:566-610) for one row: Q4_K
    gate and up matvecs, silu_mul (weights.rs:241-260), Q4_K down matvec,
    each matvec with the Q8_K path of matvec_payload."""
    g = q4_k_matvec(gate, width, hidden, x)
    u = q4_k_matvec(up, width, hidden, x)
    return q4_k_matvec(down, hidden, width, silu_mul(g, u))


Q6_K_BLOCK_BYTES = 210


def dequantize_q6_k(block: np.ndarray) -> np.ndarray:
    """dequant.rs:190-218 (the canonical LM head format)."""
    b = np.ascontiguousarray(block, dtype=np.uint8)
    out = np.empty(256, np.float32)
    lib().orc_dequantize_q6_k(_p(b), _p(out))
    return out


def q6_k_dot_pre(row: np.ndarray, q8: np.ndarray, scales: np.ndarray) -> float:
    """weights.rs:1023-1101 over len(row) / 210 blocks."""
    row = np.ascontiguousarray(row, dtype=np.uint8)
    q8 = np.ascontiguousarray(q8, dtype=np.int8)
    scales = _f32a(scales)
    return float(lib().orc_q6_k_dot_pre(_p(row), row.size // Q6_K_BLOCK_BYTES, _p(q8), _p(scales)))


def q6_k_matvec(w: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    """weights.rs:680-735 with the Q6_K branch: Q8_K activations, integer dot."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = _f32a(x)
    y = np.empty(rows, dtype=np.float32)
    if lib().orc_q6_k_matvec(_p(w), rows, cols, _p(x), _p(y)) != 0:
        raise ValueError("cols must be a multiple of 256")
    return y
