"""Host-side mirror of the reference's compute-backend seams, over the HIP
C ABI (``include/tqf_hip.h``).

Reference seams mirrored (paths in the reference checkout):
  * ``backend::reference::q4k_gemv(weights, x, rows, cols)`` and
    ``q4k_gemm`` (backend/reference.rs:61-92)  -> ``HipBackend.q4_gemv``
  * ``GpuResidentExpert::{upload, forward}`` (backend/metal/expert.rs:110-172)
                                                -> ``upload_q4_0``, ``expert_forward``
  * ``Qwen36StreamingMoe::forward_batch`` (experts/mod.rs:1540-1577) with the
    arithmetic of ``Qwen36ResidentMoe::forward`` (:1600-1634)
                                                -> ``moe_forward_batch``
  * ``top_logit_candidates`` (runtime/decode.rs:48-64) -> ``top_logit_candidates``
  * ``Sampler::select`` + ``mtp::verify_pair`` generalised to k drafts
                                                -> ``accept``
Errors surface as ``HipError`` (the analogue of BackendError::Gpu, error.rs:
285-288); shape violations are errors, not panics.  Every call runs on the
GPU through the library; there is no CPU path here.
"""
from __future__ import annotations

import contextlib
import ctypes as C
from dataclasses import dataclass
from typing import Sequence

import numpy as np

from . import _lib
from ._lib import HipError


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


@dataclass
class Q4Weights:
    handle: int
    rows: int
    cols: int


@dataclass
class Q4KWeights:
    """A Q4_K matrix on the device (GGML 144-byte super-blocks of 256)."""
    handle: int
    rows: int
    cols: int


@dataclass
class Q6KWeights:
    """A Q6_K matrix on the device (GGML 210-byte super-blocks of 256)."""
    handle: int
    rows: int
    cols: int


@dataclass
class F32Tensor:
    handle: int
    count: int


@dataclass
class DeviceBuffer:
    ptr: int
    nbytes: int


class MoeLayer:
    """A prepared layer (device expert table) plus the handles it uses."""

    def __init__(self, handle: int, hidden: int, width: int, n_experts: int, owned: list):
        self.handle = handle
        self.hidden = hidden
        self.width = width
        self.n_experts = n_experts
        self.owned = owned


class Stack:
    def __init__(self, handle: int, layers: list, norms: list):
        self.handle = handle
        self.layers = layers
        self.norms = norms


class HipBackend:
    """The GpuExecutionState analogue (backend/metal/expert.rs:77-95): one
    device, one stream, the loaded kernels and a reusable scratch arena."""

    def __init__(self, device: int = 0):
        self.lib = _lib.load()
        h = C.c_void_p()
        st = self.lib.tqf_hip_create(device, C.byref(h))
        if st != _lib.OK:
            raise HipError(st, f"tqf_hip_create(device={device}) failed")
        self.ctx = h.value

    # ---- lifecycle -------------------------------------------------------
    def close(self) -> None:
        if self.ctx:
            self.lib.tqf_hip_destroy(self.ctx)
            self.ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _check(self, status: int) -> None:
        if status != _lib.OK:
            msg = self.lib.tqf_hip_last_error(self.ctx)
            raise HipError(status, msg.decode() if msg else "")

    def synchronize(self) -> None:
        self._check(self.lib.tqf_hip_synchronize(self.ctx))

    def device_info(self) -> tuple[str, int]:
        buf = C.create_string_buffer(256)
        cu = C.c_int32()
        self._check(self.lib.tqf_hip_device_info(self.ctx, buf, 256, C.byref(cu)))
        return buf.value.decode(), cu.value

    # ---- plain device buffers -------------------------------------------
    def alloc(self, nbytes: int) -> DeviceBuffer:
        p = C.c_void_p()
        self._check(self.lib.tqf_hip_buffer_alloc(self.ctx, nbytes, C.byref(p)))
        return DeviceBuffer(p.value, nbytes)

    def free(self, buf: DeviceBuffer) -> None:
        self._check(self.lib.tqf_hip_buffer_free(self.ctx, buf.ptr))

    def to_device(self, a: np.ndarray) -> DeviceBuffer:
        a = np.ascontiguousarray(a)
        buf = self.alloc(max(a.nbytes, 1))
        self._check(self.lib.tqf_hip_memcpy_h2d(self.ctx, buf.ptr, _ptr(a), a.nbytes))
        return buf

    def write(self, buf: DeviceBuffer, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        if a.nbytes > buf.nbytes:
            raise ValueError("array larger than the device buffer")
        self._check(self.lib.tqf_hip_memcpy_h2d(self.ctx, buf.ptr, _ptr(a), a.nbytes))

    def copy_device(self, dst: DeviceBuffer, src: DeviceBuffer, nbytes: int) -> None:
        """Stream-ordered device-to-device copy of nbytes."""
        if nbytes > dst.nbytes or nbytes > src.nbytes:
            raise ValueError("copy larger than a buffer")
        self._check(self.lib.tqf_hip_memcpy_d2d(self.ctx, dst.ptr, src.ptr, nbytes))

    @staticmethod
    def view(buf: DeviceBuffer, offset: int, nbytes: int) -> DeviceBuffer:
        """A sub-range of a buffer (not to be freed on its own)."""
        if offset < 0 or offset + nbytes > buf.nbytes:
            raise ValueError("view outside the buffer")
        return DeviceBuffer(buf.ptr + offset, nbytes)

    def read(self, buf: DeviceBuffer, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        self._check(self.lib.tqf_hip_memcpy_d2h(self.ctx, _ptr(out), buf.ptr, out.nbytes))
        return out

    # ---- weights -----------------------------------------------------------
    @staticmethod
    def weights_bytes_for(rows: int, cols: int) -> int:
        return int(_lib.load().tqf_hip_weights_bytes_for(rows, cols))

    def upload_q4_0(self, q4_0: np.ndarray | bytes, rows: int, cols: int) -> Q4Weights:
        a = np.frombuffer(bytes(q4_0), dtype=np.uint8) if isinstance(q4_0, (bytes, bytearray)) \
            else np.ascontiguousarray(q4_0, dtype=np.uint8)
        h = C.c_void_p()
        self._check(self.lib.tqf_hip_weights_upload(self.ctx, _ptr(a), a.nbytes, rows, cols,
                                                    C.byref(h)))
        return Q4Weights(h.value, rows, cols)

    def synth_q4_0(self, rows: int, cols: int, tensor_id: int, seed: int,
                   recipe: int | str = 0) -> Q4Weights:
        """Seeded synthetic Q4_0 matrix generated in HBM; ``recipe`` "uniform"
        (0) or "zero_mean" (1), as ``synth.q4_0_synthetic``."""
        from . import synth

        r = synth.RECIPES.get(recipe, recipe) if isinstance(recipe, str) else int(recipe)
        h = C.c_void_p()
        self._check(self.lib.tqf_hip_weights_synth_recipe(self.ctx, rows, cols, tensor_id, seed,
                                                          r, C.byref(h)))
        return Q4Weights(h.value, rows, cols)

    def download_q4_0(self, w: Q4Weights) -> np.ndarray:
        out = np.empty(w.rows * (w.cols // 32) * 18, dtype=np.uint8)
        self._check(self.lib.tqf_hip_weights_download(self.ctx, w.handle, _ptr(out), out.nbytes))
        return out

    def weights_bytes(self, w: Q4Weights) -> int:
        return int(self.lib.tqf_hip_weights_bytes(w.handle))

    def free_weights(self, w: Q4Weights) -> None:
        self._check(self.lib.tqf_hip_weights_free(self.ctx, w.handle))

    def upload_f32(self, a: np.ndarray) -> F32Tensor:
        a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
        h = C.c_void_p()
        self._check(self.lib.tqf_hip_tensor_upload(self.ctx, _ptr(a), a.size, C.byref(h)))
        return F32Tensor(h.value, a.size)

    def free_tensor(self, t: F32Tensor) -> None:
        self._check(self.lib.tqf_hip_tensor_free(self.ctx, t.handle))

    # ---- GEMV / expert ---------------------------------------------------------
    def q4_gemv(self, w: Q4Weights, x: np.ndarray) -> np.ndarray:
        """y = W x for x [cols] or [m, cols] (m <= 8); y [rows] or [m, rows]."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        squeeze = x.ndim == 1
        x2 = x.reshape(1, -1) if squeeze else x
        if x2.shape[1] != w.cols:
            raise ValueError(f"x has {x2.shape[1]} columns, matrix has {w.cols}")
        m = x2.shape[0]
        y = np.empty((m, w.rows), dtype=np.float32)
        self._check(self.lib.tqf_hip_q4_gemv(self.ctx, w.handle, _ptr(x2), m, _ptr(y)))
        return y[0] if squeeze else y

    def q4_gemv_device(self, w: Q4Weights, d_x: DeviceBuffer, m: int, d_y: DeviceBuffer) -> None:
        self._check(self.lib.tqf_hip_q4_gemv_device(self.ctx, w.handle, d_x.ptr, m, d_y.ptr))

    def q4_gemv_batched_device(self, ws: Sequence[Q4Weights], d_x: DeviceBuffer,
                               d_y: DeviceBuffer) -> None:
        arr = (C.c_void_p * len(ws))(*[w.handle for w in ws])
        self._check(self.lib.tqf_hip_q4_gemv_batched_device(self.ctx, arr, len(ws), d_x.ptr,
                                                            d_y.ptr))

    def expert_forward(self, gate: Q4Weights, up: Q4Weights, down: Q4Weights,
                       x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        squeeze = x.ndim == 1
        x2 = x.reshape(1, -1) if squeeze else x
        m = x2.shape[0]
        y = np.empty((m, down.rows), dtype=np.float32)
        self._check(self.lib.tqf_hip_expert_forward(self.ctx, gate.handle, up.handle, down.handle,
                                                    _ptr(x2), m, _ptr(y)))
        return y[0] if squeeze else y

    # ---- Q4_K ------------------------------------------------------------------
    @staticmethod
    def q4k_weights_bytes_for(rows: int, cols: int) -> int:
        return int(_lib.load().tqf_hip_q4k_weights_bytes_for(rows, cols))

    def upload_q4_k(self, q4_k: np.ndarray | bytes, rows: int, cols: int) -> Q4KWeights:
        a = np.frombuffer(bytes(q4_k), dtype=np.uint8) if isinstance(q4_k, (bytes, bytearray)) \
            else np.ascontiguousarray(q4_k, dtype=np.uint8)
        h = C.c_void_p()
        self._check(self.lib.tqf_hip_q4k_weights_upload(self.ctx, _ptr(a), a.nbytes, rows, cols,
                                                        C.byref(h)))
        return Q4KWeights(h.value, rows, cols)

    def upload_q4_k_device(self, d_q4_k: DeviceBuffer, rows: int, cols: int) -> Q4KWeights:
        h = C.c_void_p()
        self._check(self.lib.tqf_hip_q4k_weights_upload_device(
            self.ctx, d_q4_k.ptr, rows * (cols // 256) * 144, rows, cols, C.byref(h)))
        return Q4KWeights(h.value, rows, cols)

    def download_q4_k(self, w: Q4KWeights) -> np.ndarray:
        out = np.empty(w.rows * (w.cols // 256) * 144, dtype=np.uint8)
        self._check(self.lib.tqf_hip_q4k_weights_download(self.ctx, w.handle, _ptr(out),
                                                          out.nbytes))
        return out

    def _q4k_call(self, fn, w: Q4KWeights, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        squeeze = x.ndim == 1
        x2 = x.reshape(1, -1) if squeeze else x
        if x2.shape[1] != w.cols:
            raise ValueError(f"x has {x2.shape[1]} columns, matrix has {w.cols}")
        m = x2.shape[0]
        y = np.empty((m, w.rows), dtype=np.float32)
        self._check(fn(self.ctx, w.handle, _ptr(x2), m, _ptr(y)))
        return y[0] if squeeze else y

    def q4k_gemv(self, w: Q4KWeights, x: np.ndarray) -> np.ndarray:
        """backend::reference::q4k_gemv semantics (fp32 dequant-and-accumulate)."""
        return self._q4k_call(self.lib.tqf_hip_q4k_gemv, w, x)

    def q4k_matvec(self, w: Q4KWeights, x: np.ndarray) -> np.ndarray:
        """matvec_payload Q4_K semantics (Q8_K activations, q4_k_dot_pre)."""
        return self._q4k_call(self.lib.tqf_hip_q4k_matvec, w, x)

    def q4k_gemv_device(self, w: Q4KWeights, d_x: DeviceBuffer, m: int, d_y: DeviceBuffer) -> None:
        self._check(self.lib.tqf_hip_q4k_gemv_device(self.ctx, w.handle, d_x.ptr, m, d_y.ptr))

    def q4k_matvec_device(self, w: Q4KWeights, d_x: DeviceBuffer, m: int,
                          d_y: DeviceBuffer) -> None:
        self._check(self.lib.tqf_hip_q4k_matvec_device(self.ctx, w.handle, d_x.ptr, m, d_y.ptr))

    def q4k_gemv_batched_device(self, ws: Sequence[Q4KWeights], d_x: DeviceBuffer,
                                d_y: DeviceBuffer) -> None:
        arr = (C.c_void_p * len(ws))(*[w.handle for w in ws])
        self._check(self.lib.tqf_hip_q4k_gemv_batched_device(self.ctx, arr, len(ws), d_x.ptr,
                                                             d_y.ptr))

    def q4k_matvec_batched_device(self, ws: Sequence[Q4KWeights], d_x: DeviceBuffer,
                                  d_y: DeviceBuffer) -> None:
        arr = (C.c_void_p * len(ws))(*[w.handle for w in ws])
        self._check(self.lib.tqf_hip_q4k_matvec_batched_device(self.ctx, arr, len(ws), d_x.ptr,
                                                               d_y.ptr))

    def q4k_expert_forward(self, gate: Q4KWeights, up: Q4KWeights, down: Q4KWeights,
                           x: np.ndarray) -> np.ndarray:
        """LoadedQwen36Expert::forward with Q4_K payloads."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        squeeze = x.ndim == 1
        x2 = x.reshape(1, -1) if squeeze else x
        m = x2.shape[0]
        y = np.empty((m, down.rows), dtype=np.float32)
        self._check(self.lib.tqf_hip_q4k_expert_forward(self.ctx, gate.handle, up.handle,
                                                        down.handle, _ptr(x2), m, _ptr(y)))
        return y[0] if squeeze else y

    def q4k_expert_forward_device(self, gate: Q4KWeights, up: Q4KWeights, down: Q4KWeights,
                                  d_x: DeviceBuffer, m: int, d_y: DeviceBuffer) -> None:
        self._check(self.lib.tqf_hip_q4k_expert_forward_device(
            self.ctx, gate.handle, up.handle, down.handle, d_x.ptr, m, d_y.ptr))

    # ---- Q6_K / LM head ---------------------------------------------------------
    @staticmethod
    def q6k_weights_bytes_for(rows: int, cols: int) -> int:
        return int(_lib.load().tqf_hip_q6k_weights_bytes_for(rows, cols))

    def upload_q6_k(self, q6_k: np.ndarray | bytes, rows: int, cols: int) -> Q6KWeights:
        a = np.frombuffer(bytes(q6_k), dtype=np.uint8) if isinstance(q6_k, (bytes, bytearray)) \
            else np.ascontiguousarray(q6_k, dtype=np.uint8)
        h = C.c_void_p()
        self._check(self.lib.tqf_hip_q6k_weights_upload(self.ctx, _ptr(a), a.nbytes, rows, cols,
                                                        C.byref(h)))
        return Q6KWeights(h.value, rows, cols)

    def upload_q6_k_device(self, d_q6_k: DeviceBuffer, rows: int, cols: int) -> Q6KWeights:
        h = C.c_void_p()
        self._check(self.lib.tqf_hip_q6k_weights_upload_device(
            self.ctx, d_q6_k.ptr, rows * (cols // 256) * 210, rows, cols, C.byref(h)))
        return Q6KWeights(h.value, rows, cols)

    def download_q6_k(self, w: Q6KWeights) -> np.ndarray:
        out = np.empty(w.rows * (w.cols // 256) * 210, dtype=np.uint8)
        self._check(self.lib.tqf_hip_q6k_weights_download(self.ctx, w.handle, _ptr(out),
                                                          out.nbytes))
        return out

    def q6k_matvec(self, w: Q6KWeights, x: np.ndarray) -> np.ndarray:
        """matvec_payload Q6_K semantics (Q8_K activations, q6_k_dot_pre)."""
        return self._q4k_call(self.lib.tqf_hip_q6k_matvec, w, x)

    def q6k_matvec_device(self, w: Q6KWeights, d_x: DeviceBuffer, m: int,
                          d_y: DeviceBuffer) -> None:
        self._check(self.lib.tqf_hip_q6k_matvec_device(self.ctx, w.handle, d_x.ptr, m, d_y.ptr))

    def lm_head_logits(self, w: Q6KWeights, x: np.ndarray):
        """logits [m, V] and the top_logit_candidates (tokens [m, 4], logits [m, 4])."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        x2 = x.reshape(1, -1) if x.ndim == 1 else x
        if x2.shape[1] != w.cols:
            raise ValueError(f"x has {x2.shape[1]} columns, matrix has {w.cols}")
        m = x2.shape[0]
        y = np.empty((m, w.rows), dtype=np.float32)
        t4 = np.empty((m, 4), dtype=np.uint32)
        l4 = np.empty((m, 4), dtype=np.float32)
        self._check(self.lib.tqf_hip_lm_head_logits(self.ctx, w.handle, _ptr(x2), m, _ptr(y),
                                                    _ptr(t4), _ptr(l4)))
        return y, t4, l4

    def lm_head_logits_device(self, w: Q6KWeights, d_x: DeviceBuffer, m: int,
                              d_logits: DeviceBuffer, d_tokens4: DeviceBuffer,
                              d_logits4: DeviceBuffer) -> None:
        self._check(self.lib.tqf_hip_lm_head_logits_device(self.ctx, w.handle, d_x.ptr, m,
                                                           d_logits.ptr, d_tokens4.ptr,
                                                           d_logits4.ptr))

    # ---- MoE layer -------------------------------------------------------------
    def prepare_moe_layer(self, router: F32Tensor, shared_input_gate: F32Tensor,
                          shared: tuple[Q4Weights, Q4Weights, Q4Weights] | tuple[Q4KWeights, Q4KWeights, Q4KWeights],
                          routed_gate: Sequence[Q4Weights | Q4KWeights],
                          routed_up: Sequence[Q4Weights | Q4KWeights],
                          routed_down: Sequence[Q4Weights | Q4KWeights]) -> MoeLayer:
        """One layer's device handle.  Every expert matrix is Q4_0 or every
        one is Q4_K (the canonical checkpoint's experts); Q4_K layers run the
        Q8_K integer matvecs of the reference's Q4_K path."""
        E = len(routed_gate)
        g = (C.c_void_p * E)(*[w.handle for w in routed_gate])
        u = (C.c_void_p * E)(*[w.handle for w in routed_up])
        d = (C.c_void_p * E)(*[w.handle for w in routed_down])
        hidden, width = shared[0].cols, shared[0].rows
        mw = _lib.MoeWeights(router.handle, shared_input_gate.handle, shared[0].handle,
                             shared[1].handle, shared[2].handle,
                             C.cast(g, C.c_void_p), C.cast(u, C.c_void_p), C.cast(d, C.c_void_p),
                             E, hidden, width)
        h = C.c_void_p()
        self._check(self.lib.tqf_hip_moe_layer_prepare(self.ctx, C.byref(mw), C.byref(h)))
        return MoeLayer(h.value, hidden, width, E,
                        [router, shared_input_gate, *shared, *routed_gate, *routed_up, *routed_down])

    def free_moe_layer(self, layer: MoeLayer) -> None:
        self._check(self.lib.tqf_hip_moe_layer_free(self.ctx, layer.handle))

    def moe_forward_batch(self, layer: MoeLayer, x: np.ndarray):
        """x [m, hidden] f32 -> (y [m, hidden], ids [m, 8] u16, w [m, 8] f32)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim == 1:
            x = x.reshape(1, -1)
        m = x.shape[0]
        if x.shape[1] != layer.hidden:
            raise ValueError("x width does not match the layer's hidden size")
        y = np.empty((m, layer.hidden), dtype=np.float32)
        ids = np.empty((m, _lib.TOP_K), dtype=np.uint16)
        w = np.empty((m, _lib.TOP_K), dtype=np.float32)
        self._check(self.lib.tqf_hip_moe_layer(self.ctx, layer.handle, _ptr(x), m, _ptr(y),
                                               _ptr(ids), _ptr(w)))
        return y, ids, w

    def moe_layer_device(self, layer: MoeLayer, d_x: DeviceBuffer, m: int, d_y: DeviceBuffer,
                         d_ids: DeviceBuffer | None = None, d_w: DeviceBuffer | None = None,
                         d_status: DeviceBuffer | None = None) -> None:
        """Enqueues one layer on device buffers (d_x [m, hidden] f32 -> d_y)."""
        self._check(self.lib.tqf_hip_moe_layer_device(
            self.ctx, layer.handle, d_x.ptr, m, d_y.ptr, d_ids.ptr if d_ids else None,
            d_w.ptr if d_w else None, d_status.ptr if d_status else None))

    def moe_forward_batch_bf16(self, layer: MoeLayer, x_bf16: np.ndarray):
        x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
        if x.ndim == 1:
            x = x.reshape(1, -1)
        m = x.shape[0]
        y = np.empty((m, layer.hidden), dtype=np.float32)
        ids = np.empty((m, _lib.TOP_K), dtype=np.uint16)
        w = np.empty((m, _lib.TOP_K), dtype=np.float32)
        self._check(self.lib.tqf_hip_moe_layer_bf16(self.ctx, layer.handle, _ptr(x), m, _ptr(y),
                                                    _ptr(ids), _ptr(w)))
        return y, ids, w

    # ---- grouped expert GEMM (prefill) ---------------------------------------------
    def grouped_gemm(self, layer: MoeLayer, x_bf16: np.ndarray, ids: np.ndarray,
                     w: np.ndarray) -> np.ndarray:
        """x_bf16 [t, hidden] u16, ids [t, 8] u16, w [t, 8] f32 -> y [t, hidden] f32,
        the route-weighted sum of the routed experts (tqf_hip_grouped_gemm)."""
        x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
        ids = np.ascontiguousarray(ids, dtype=np.uint16)
        w = np.ascontiguousarray(w, dtype=np.float32)
        t = x.shape[0]
        if x.shape != (t, layer.hidden) or ids.shape != (t, _lib.TOP_K) or w.shape != ids.shape:
            raise ValueError("grouped_gemm: x [t, hidden], ids and w [t, 8]")
        y = np.empty((t, layer.hidden), dtype=np.float32)
        self._check(self.lib.tqf_hip_grouped_gemm(self.ctx, layer.handle, _ptr(x), t, _ptr(ids),
                                                  _ptr(w), _ptr(y)))
        return y

    def grouped_gemm_device(self, layer: MoeLayer, d_x: DeviceBuffer, t: int, d_ids: DeviceBuffer,
                            d_w: DeviceBuffer, d_y: DeviceBuffer,
                            d_status: DeviceBuffer | None = None) -> None:
        self._check(self.lib.tqf_hip_grouped_gemm_device(
            self.ctx, layer.handle, d_x.ptr, t, d_ids.ptr, d_w.ptr, d_y.ptr,
            d_status.ptr if d_status else None))

    # ---- stack / verify step -------------------------------------------------------
    def prepare_stack(self, layers: Sequence[MoeLayer], norms: Sequence[F32Tensor]) -> Stack:
        n = len(layers)
        la = (C.c_void_p * n)(*[l.handle for l in layers])
        na = (C.c_void_p * n)(*[t.handle for t in norms])
        h = C.c_void_p()
        self._check(self.lib.tqf_hip_stack_prepare(self.ctx, la, na, n, C.byref(h)))
        return Stack(h.value, list(layers), list(norms))

    def free_stack(self, st: Stack) -> None:
        self._check(self.lib.tqf_hip_stack_free(self.ctx, st.handle))

    def stack_forward_device(self, st: Stack, d_h: DeviceBuffer, m: int,
                             d_ids: DeviceBuffer | None = None, d_w: DeviceBuffer | None = None,
                             d_status: DeviceBuffer | None = None,
                             d_h_in: DeviceBuffer | None = None) -> None:
        """h <- stack(h_in) (in place when d_h_in is None)."""
        self._check(self.lib.tqf_hip_stack_forward_device(
            self.ctx, st.handle, d_h_in.ptr if d_h_in else None, d_h.ptr, m,
            d_ids.ptr if d_ids else None, d_w.ptr if d_w else None,
            d_status.ptr if d_status else None))

    def embed_rows_device(self, emb: Q4Weights, d_tokens: DeviceBuffer, n: int, d_out: DeviceBuffer,
                          d_add: DeviceBuffer | None = None,
                          d_status: DeviceBuffer | None = None) -> None:
        """d_out [n x cols] = Q4_0 rows d_tokens of emb (+ d_add)."""
        self._check(self.lib.tqf_hip_embed_rows_device(
            self.ctx, emb.handle, d_tokens.ptr, n, d_add.ptr if d_add else None, d_out.ptr,
            d_status.ptr if d_status else None))

    def rmsnorm_rows_device(self, d_x: DeviceBuffer, n: int, cols: int, w: F32Tensor,
                            d_out: DeviceBuffer) -> None:
        """d_out [n x cols] = qwen_rmsnorm of each row of d_x with weight w."""
        self._check(self.lib.tqf_hip_rmsnorm_rows_device(self.ctx, d_x.ptr, n, cols, w.handle,
                                                         d_out.ptr))

    def verify_step_device(self, st: Stack, d_h_in: DeviceBuffer | None, d_h: DeviceBuffer,
                           m: int, d_target: DeviceBuffer, d_draft: DeviceBuffer | None,
                           d_dtok: DeviceBuffer, vocab: int, temperature: float, greedy: bool,
                           d_u: DeviceBuffer | None, d_ures: DeviceBuffer | None,
                           d_accepted: DeviceBuffer, d_tokens: DeviceBuffer,
                           d_status: DeviceBuffer | None = None) -> None:
        """One verify step: h <- stack(h_in), then the acceptance.  d_status
        (device int32, caller-zeroed) receives the stack's device status."""
        self._check(self.lib.tqf_hip_verify_step_device(
            self.ctx, st.handle, d_h_in.ptr if d_h_in else None, d_h.ptr, m, d_target.ptr,
            d_draft.ptr if d_draft else None,
            d_dtok.ptr, vocab, temperature, 1 if greedy else 0, d_u.ptr if d_u else None,
            d_ures.ptr if d_ures else None, d_accepted.ptr, d_tokens.ptr,
            d_status.ptr if d_status else None))

    # ---- acceptance ------------------------------------------------------------------
    def accept(self, target: np.ndarray, draft: np.ndarray | None, draft_tokens: Sequence[int],
               temperature: float, greedy: bool, u: np.ndarray | None = None,
               u_resample: np.ndarray | None = None) -> tuple[int, list[int]]:
        """Returns (accepted, emitted tokens).  target [k+1, V], draft [k, V]."""
        target = np.ascontiguousarray(target, dtype=np.float32)
        kp1, vocab = target.shape
        k = kp1 - 1
        dt = np.ascontiguousarray(np.asarray(draft_tokens, dtype=np.int32).reshape(-1))
        if dt.size != k:
            raise ValueError("need k draft tokens for k+1 target rows")
        dr = None if draft is None else np.ascontiguousarray(draft, dtype=np.float32)
        uu = None if u is None else np.ascontiguousarray(u, dtype=np.float32)
        ur = None if u_resample is None else np.ascontiguousarray(u_resample, dtype=np.float32)
        acc = C.c_int32()
        toks = np.empty(k + 1, dtype=np.int32)
        self._check(self.lib.tqf_hip_accept(
            self.ctx, _ptr(target), None if dr is None else _ptr(dr), _ptr(dt) if k else None,
            k, vocab, float(temperature), 1 if greedy else 0,
            None if uu is None else _ptr(uu), None if ur is None else _ptr(ur),
            C.byref(acc), _ptr(toks)))
        a = acc.value
        return a, [int(t) for t in toks[: a + 1]]

    def accept_device(self, d_target: DeviceBuffer, d_draft: DeviceBuffer | None,
                      d_dtok: DeviceBuffer, k: int, vocab: int, temperature: float, greedy: bool,
                      d_u: DeviceBuffer | None, d_ures: DeviceBuffer | None,
                      d_accepted: DeviceBuffer, d_tokens: DeviceBuffer) -> None:
        self._check(self.lib.tqf_hip_accept_device(
            self.ctx, d_target.ptr, d_draft.ptr if d_draft else None, d_dtok.ptr, k, vocab,
            float(temperature), 1 if greedy else 0, d_u.ptr if d_u else None,
            d_ures.ptr if d_ures else None, d_accepted.ptr, d_tokens.ptr))

    def accept_device_noalloc(self, d_target: DeviceBuffer, d_draft: DeviceBuffer | None,
                              d_dtok: DeviceBuffer | None, k: int, vocab: int, temperature: float,
                              greedy: bool, d_u: DeviceBuffer | None, d_ures: DeviceBuffer | None,
                              d_accepted: DeviceBuffer, d_tokens: DeviceBuffer) -> None:
        """accept_device on the library's fixed per-GPU scratch (no allocation)."""
        self._check(self.lib.tqf_hip_accept_device_noalloc(
            self.ctx, d_target.ptr, d_draft.ptr if d_draft else None,
            d_dtok.ptr if d_dtok else None, k, vocab, float(temperature), 1 if greedy else 0,
            d_u.ptr if d_u else None, d_ures.ptr if d_ures else None, d_accepted.ptr,
            d_tokens.ptr))

    def sampler_select_device(self, d_logits: DeviceBuffer, rows: int, vocab: int,
                              temperature: float, d_u: DeviceBuffer | None,
                              d_tokens: DeviceBuffer, d_sums: DeviceBuffer | None = None) -> None:
        """Sampler::select on device rows (the reference's token for uniform
        d_u[row]); d_sums, if given, receives [rows x 2] (total, total2)."""
        self._check(self.lib.tqf_hip_sampler_select_device(
            self.ctx, d_logits.ptr, rows, vocab, float(temperature), d_u.ptr if d_u else None,
            d_tokens.ptr, d_sums.ptr if d_sums else None))

    def sampler_select(self, logits: np.ndarray, temperature: float, u, sums: bool = False):
        """Host form: [V] or [rows, V] logits and one uniform per row -> tokens,
        and with sums=True also the [rows, 2] f32 folds (total, total2)."""
        lg = np.ascontiguousarray(logits, dtype=np.float32)
        lg2 = lg.reshape(1, -1) if lg.ndim == 1 else lg
        rows, vocab = lg2.shape
        uu = np.ascontiguousarray(np.atleast_1d(np.asarray(u, dtype=np.float32)))
        if uu.size != rows:
            raise ValueError("one uniform per row")
        d_l, d_u, d_t = self.to_device(lg2), self.to_device(uu), self.alloc(4 * rows)
        d_s = self.alloc(8 * rows) if sums else None
        try:
            self.sampler_select_device(d_l, rows, vocab, temperature, d_u, d_t, d_s)
            toks = [int(t) for t in self.read(d_t, np.int32, (rows,))]
            return (toks, self.read(d_s, np.float32, (rows, 2))) if sums else toks
        finally:
            for b in (d_l, d_u, d_t, d_s):
                if b is not None:
                    self.free(b)

    def top_logit_candidates(self, logits: np.ndarray):
        """[V] or [rows, V] logits -> (tokens [rows, 4] u32, logits [rows, 4])."""
        lg = np.ascontiguousarray(logits, dtype=np.float32)
        squeeze = lg.ndim == 1
        lg2 = lg.reshape(1, -1) if squeeze else lg
        rows, vocab = lg2.shape
        toks = np.empty((rows, 4), dtype=np.uint32)
        vals = np.empty((rows, 4), dtype=np.float32)
        self._check(self.lib.tqf_hip_top_logit_candidates(self.ctx, _ptr(lg2), rows, vocab,
                                                          _ptr(toks), _ptr(vals)))
        return (toks[0], vals[0]) if squeeze else (toks, vals)

    # ---- kernel variants (GpuKernelKind) ------------------------------------------------
    def set_variant(self, variant: int, value: bool) -> None:
        self._check(self.lib.tqf_hip_set_variant(self.ctx, variant, 1 if value else 0))

    def get_variant(self, variant: int) -> bool:
        v = C.c_int32()
        self._check(self.lib.tqf_hip_get_variant(self.ctx, variant, C.byref(v)))
        return bool(v.value)

    @contextlib.contextmanager
    def variant(self, variant: int, value: bool):
        """Selects a kernel variant for the duration of a with-block."""
        old = self.get_variant(variant)
        self.set_variant(variant, value)
        try:
            yield
        finally:
            self.set_variant(variant, old)

    def recovery_counts(self) -> tuple[int, int]:
        """(stack re-runs, acceptance re-runs) after timed-out persistent launches."""
        st = C.c_uint64()
        ac = C.c_uint64()
        self._check(self.lib.tqf_hip_recovery_counts(self.ctx, C.byref(st), C.byref(ac)))
        return st.value, ac.value

    # ---- profiling ---------------------------------------------------------------------
    def profile_enable(self, enable: bool = True) -> None:
        self._check(self.lib.tqf_hip_profile_enable(self.ctx, 1 if enable else 0))

    def profile_read(self, kind: int) -> tuple[int, float, float]:
        """(launches, total kernel ms, total algorithmic bytes) of one kind."""
        n = C.c_uint64()
        ms = C.c_double()
        by = C.c_double()
        self._check(self.lib.tqf_hip_profile_read(self.ctx, kind, C.byref(n), C.byref(ms),
                                                  C.byref(by)))
        return n.value, ms.value, by.value
