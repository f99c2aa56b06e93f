"""ctypes binding of ``libtqf_hip.so`` (the C ABI in ``include/tqf_hip.h``).

This mirrors what the reference crate's Rust FFI module would declare.  The
library is required: importing the bindings without a built library raises,
there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libtqf_hip.so"

OK = 0
ERR_INVALID = 1
ERR_DEVICE = 2
ERR_NOMEM = 3
ERR_ROUTER = 4
TOP_K = 8
MAX_TOKENS = 8

KERNEL_ROUTE = 0
KERNEL_GATE_UP = 1
KERNEL_DOWN = 2
KERNEL_GEMV = 3
KERNEL_ACCEPT = 4
KERNEL_STACK = 5
KERNEL_GROUPED_GATE_UP = 6
KERNEL_GROUPED_DOWN = 7
KERNEL_GROUPED_AUX = 8
KERNEL_Q4K_GEMV = 9
KERNEL_Q4K_MATVEC = 10
KERNEL_Q6K_MATVEC = 11
KERNEL_SAMPLE = 12
KERNEL_KINDS = 13
VARIANT_PERSISTENT = 0
VARIANT_Q4K_FOLD = 1
VARIANT_GRAPHS = 2
VARIANT_RECOVER = 3
FORMAT_Q4_0 = 0
FORMAT_Q4_K = 1
FORMAT_Q6_K = 2
GROUPED_MAX_TOKENS = 4096

_vp = C.c_void_p
_i32 = C.c_int32
_u32 = C.c_uint32
_u64 = C.c_uint64
_sz = C.c_size_t
_f32 = C.c_float
_pp = C.POINTER(C.c_void_p)


class MoeWeights(C.Structure):
    """``tqf_hip_moe_weights`` (Qwen36ResidentMoe's tensors, experts/mod.rs:1454)."""

    _fields_ = [
        ("router", _vp),
        ("shared_input_gate", _vp),
        ("shared_gate", _vp),
        ("shared_up", _vp),
        ("shared_down", _vp),
        ("routed_gate", _vp),
        ("routed_up", _vp),
        ("routed_down", _vp),
        ("n_experts", _u32),
        ("hidden", _u32),
        ("width", _u32),
    ]


# name -> (restype, argtypes); every exported symbol of include/tqf_hip.h and
# include/tqf_hip_synth.h.
SIGNATURES = {
    "tqf_hip_create": (_i32, [_i32, _pp]),
    "tqf_hip_destroy": (_i32, [_vp]),
    "tqf_hip_last_error": (C.c_char_p, [_vp]),
    "tqf_hip_synchronize": (_i32, [_vp]),
    "tqf_hip_device_info": (_i32, [_vp, C.c_char_p, _sz, C.POINTER(_i32)]),
    "tqf_hip_buffer_alloc": (_i32, [_vp, _sz, _pp]),
    "tqf_hip_buffer_free": (_i32, [_vp, _vp]),
    "tqf_hip_memcpy_h2d": (_i32, [_vp, _vp, _vp, _sz]),
    "tqf_hip_memcpy_d2h": (_i32, [_vp, _vp, _vp, _sz]),
    "tqf_hip_memcpy_d2d": (_i32, [_vp, _vp, _vp, _sz]),
    "tqf_hip_weights_bytes_for": (_u64, [_u32, _u32]),
    "tqf_hip_weights_upload": (_i32, [_vp, _vp, _sz, _u32, _u32, _pp]),
    "tqf_hip_weights_upload_device": (_i32, [_vp, _vp, _sz, _u32, _u32, _pp]),
    "tqf_hip_weights_download": (_i32, [_vp, _vp, _vp, _sz]),
    "tqf_hip_weights_bytes": (_u64, [_vp]),
    "tqf_hip_weights_free": (_i32, [_vp, _vp]),
    "tqf_hip_tensor_upload": (_i32, [_vp, _vp, _sz, _pp]),
    "tqf_hip_tensor_free": (_i32, [_vp, _vp]),
    "tqf_hip_q4_gemv": (_i32, [_vp, _vp, _vp, _u32, _vp]),
    "tqf_hip_q4_gemv_device": (_i32, [_vp, _vp, _vp, _u32, _vp]),
    "tqf_hip_q4_gemv_batched_device": (_i32, [_vp, _vp, _u32, _vp, _vp]),
    "tqf_hip_expert_forward": (_i32, [_vp, _vp, _vp, _vp, _vp, _u32, _vp]),
    "tqf_hip_q4k_weights_bytes_for": (_u64, [_u32, _u32]),
    "tqf_hip_q4k_weights_upload": (_i32, [_vp, _vp, _sz, _u32, _u32, _pp]),
    "tqf_hip_q4k_weights_upload_device": (_i32, [_vp, _vp, _sz, _u32, _u32, _pp]),
    "tqf_hip_q4k_weights_download": (_i32, [_vp, _vp, _vp, _sz]),
    "tqf_hip_q4k_gemv": (_i32, [_vp, _vp, _vp, _u32, _vp]),
    "tqf_hip_q4k_gemv_device": (_i32, [_vp, _vp, _vp, _u32, _vp]),
    "tqf_hip_q4k_gemv_batched_device": (_i32, [_vp, _vp, _u32, _vp, _vp]),
    "tqf_hip_q4k_matvec": (_i32, [_vp, _vp, _vp, _u32, _vp]),
    "tqf_hip_q4k_matvec_device": (_i32, [_vp, _vp, _vp, _u32, _vp]),
    "tqf_hip_q4k_matvec_batched_device": (_i32, [_vp, _vp, _u32, _vp, _vp]),
    "tqf_hip_q4k_expert_forward": (_i32, [_vp, _vp, _vp, _vp, _vp, _u32, _vp]),
    "tqf_hip_q4k_expert_forward_device": (_i32, [_vp, _vp, _vp, _vp, _vp, _u32, _vp]),
    "tqf_hip_q6k_weights_bytes_for": (_u64, [_u32, _u32]),
    "tqf_hip_q6k_weights_upload": (_i32, [_vp, _vp, _sz, _u32, _u32, _pp]),
    "tqf_hip_q6k_weights_upload_device": (_i32, [_vp, _vp, _sz, _u32, _u32, _pp]),
    "tqf_hip_q6k_weights_download": (_i32, [_vp, _vp, _vp, _sz]),
    "tqf_hip_q6k_matvec": (_i32, [_vp, _vp, _vp, _u32, _vp]),
    "tqf_hip_q6k_matvec_device": (_i32, [_vp, _vp, _vp, _u32, _vp]),
    "tqf_hip_lm_head_logits": (_i32, [_vp, _vp, _vp, _u32, _vp, _vp, _vp]),
    "tqf_hip_lm_head_logits_device": (_i32, [_vp, _vp, _vp, _u32, _vp, _vp, _vp]),
    "tqf_hip_moe_layer_prepare": (_i32, [_vp, C.POINTER(MoeWeights), _pp]),
    "tqf_hip_moe_layer_free": (_i32, [_vp, _vp]),
    "tqf_hip_moe_layer": (_i32, [_vp, _vp, _vp, _u32, _vp, _vp, _vp]),
    "tqf_hip_moe_layer_bf16": (_i32, [_vp, _vp, _vp, _u32, _vp, _vp, _vp]),
    "tqf_hip_moe_layer_device": (_i32, [_vp, _vp, _vp, _u32, _vp, _vp, _vp, _vp]),
    "tqf_hip_stack_prepare": (_i32, [_vp, _vp, _vp, _u32, _pp]),
    "tqf_hip_stack_free": (_i32, [_vp, _vp]),
    "tqf_hip_stack_forward_device": (_i32, [_vp, _vp, _vp, _vp, _u32, _vp, _vp, _vp]),
    "tqf_hip_accept": (_i32, [_vp, _vp, _vp, _vp, _u32, _u32, _f32, _i32, _vp, _vp, _vp, _vp]),
    "tqf_hip_accept_device": (_i32, [_vp, _vp, _vp, _vp, _u32, _u32, _f32, _i32, _vp, _vp, _vp, _vp]),
    "tqf_hip_accept_device_noalloc": (
        _i32, [_vp, _vp, _vp, _vp, _u32, _u32, _f32, _i32, _vp, _vp, _vp, _vp]),
    "tqf_hip_top_logit_candidates": (_i32, [_vp, _vp, _u32, _u32, _vp, _vp]),
    "tqf_hip_grouped_gemm": (_i32, [_vp, _vp, _vp, _u32, _vp, _vp, _vp]),
    "tqf_hip_grouped_gemm_device": (_i32, [_vp, _vp, _vp, _u32, _vp, _vp, _vp, _vp]),
    "tqf_hip_embed_rows_device": (_i32, [_vp, _vp, _vp, _u32, _vp, _vp, _vp]),
    "tqf_hip_rmsnorm_rows_device": (_i32, [_vp, _vp, _u32, _u32, _vp, _vp]),
    "tqf_hip_verify_step_device": (
        _i32, [_vp, _vp, _vp, _vp, _u32, _vp, _vp, _vp, _u32, _f32, _i32, _vp, _vp, _vp, _vp,
               _vp]),
    "tqf_hip_set_variant": (_i32, [_vp, _i32, _i32]),
    "tqf_hip_get_variant": (_i32, [_vp, _i32, C.POINTER(_i32)]),
    "tqf_hip_recovery_counts": (_i32, [_vp, C.POINTER(_u64), C.POINTER(_u64)]),
    "tqf_hip_sampler_select_device": (_i32, [_vp, _vp, _u32, _u32, C.c_float, _vp, _vp, _vp]),
    "tqf_hip_expert_table_open": (_i32, [_vp, _vp, C.c_size_t, _u64, _u64, _u64, C.POINTER(_vp)]),
    "tqf_hip_expert_table_free": (_i32, [_vp, _vp]),
    "tqf_hip_expert_table_counts": (_i32, [_vp, C.POINTER(_u64), C.POINTER(_u64)]),
    "tqf_hip_expert_lookup": (_i32, [_vp, _vp, C.c_uint8, C.c_uint16, _vp, _vp, C.c_size_t,
                                     C.POINTER(C.c_size_t)]),
    "tqf_hip_expert_reserve_bytes": (_i32, [_vp, _vp, C.c_uint8, C.c_uint16, C.POINTER(_u64),
                                            C.POINTER(_u64)]),
    "tqf_hip_expert_upload": (_i32, [_vp, _vp, C.c_uint8, C.c_uint16, _vp, C.c_size_t,
                                     C.POINTER(_vp), C.POINTER(_vp), C.POINTER(_vp)]),
    "tqf_hip_profile_enable": (_i32, [_vp, _i32]),
    "tqf_hip_profile_read": (_i32, [_vp, _i32, C.POINTER(_u64), C.POINTER(C.c_double),
                                    C.POINTER(C.c_double)]),
    "tqf_hip_weights_synth": (_i32, [_vp, _u32, _u32, _u32, _u32, _pp]),
    "tqf_hip_weights_synth_recipe": (_i32, [_vp, _u32, _u32, _u32, _u32, _u32, _pp]),
}

_LIB = None


def load(path: Path | None = None) -> C.CDLL:
    """Loads the HIP backend once; raises if it has not been built."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise RuntimeError(
            f"{p} is missing: build the HIP backend first "
            "(python -c 'import __graft_entry__ as g; g.build()')")
    lib = C.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _LIB = lib
    return lib


class HipError(RuntimeError):
    """A non-zero status from the backend (BackendError::Gpu / ModelError)."""

    def __init__(self, status: int, message: str):
        super().__init__(f"status {status}: {message}")
        self.status = status
