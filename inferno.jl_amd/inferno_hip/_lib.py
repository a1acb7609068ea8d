"""ctypes binding of inferno.jl_amd/lib/libinferno_hip.so (include/inferno_hip.h).

The library is the product; this module only loads it and turns its status
codes into Python exceptions.  There is no CPU fallback: when the library is
missing, every call raises ``LibraryNotBuilt`` (build it with
``python -m inferno_hip.build`` or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

try:  # load torch's HIP runtime first so the process has exactly one
    import torch  # noqa: F401
except Exception:  # pragma: no cover - torch is optional for the host entry points
    torch = None

PKG = Path(__file__).resolve().parents[1]
LIB_PATH = PKG / "lib" / "libinferno_hip.so"

IHIP_OK = 0
IHIP_ERR_INVALID = -1
IHIP_ERR_HIP = -2
IHIP_ERR_NO_DEVICE = -3
IHIP_ERR_NONFINITE = -4
IHIP_ERR_DISABLED = -5
IHIP_ERR_NOMEM = -6
IHIP_ERR_EMPTY = -7

Q8_0, Q4_K, Q5_K, Q6_K, IQ4_NL = 8, 12, 13, 14, 20
FLAG_NAN, FLAG_POSINF, FLAG_ALL_NEGINF = 1, 2, 4
ARGMAX_WS_BYTES = 262144
Q8_K_BYTES = 292


class LibraryNotBuilt(RuntimeError):
    pass


class IHIPError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class IHIPArgumentError(IHIPError, ValueError):
    """Invalid arguments, NaN/+Inf logits, empty logits: the cases where the
    reference throws ArgumentError / AssertionError."""


_vp, _i, _i64, _sz, _u64 = C.c_void_p, C.c_int, C.c_int64, C.c_size_t, C.c_uint64

SIGNATURES = {
    "ihip_last_error": ([], C.c_char_p),
    "ihip_version": ([], _i),
    "ihip_available": ([], _i),
    "ihip_init": ([_i], _i),
    "ihip_shutdown": ([], _i),
    "ihip_weight_register": ([_vp, _sz, _i, _i, _i, C.POINTER(_u64)], _i),
    "ihip_weight_release": ([_u64], _i),
    "ihip_weight_forget": ([_vp], _i),
    "ihip_weight_device_ptr": ([_u64, C.POINTER(_vp)], _i),
    "ihip_weight_register_group": ([C.POINTER(_vp), C.POINTER(_i), _i, _i, _i, C.POINTER(_u64)], _i),
    "ihip_weight_bytes": ([_i, _i, _i], _sz),
    "ihip_weight_fingerprint": ([_vp, _sz, C.POINTER(_u64)], _i),
    "ihip_q4_k_gemv": ([_vp, _vp, _vp, _vp, _i, _i], _i),
    "ihip_q5_k_gemv": ([_vp, _vp, _vp, _vp, _i, _i], _i),
    "ihip_q6_k_gemv": ([_vp, _vp, _vp, _vp, _i, _i], _i),
    "ihip_q8_0_gemv": ([_vp, _vp, _vp, _i, _i], _i),
    "ihip_iq4_nl_gemv": ([_vp, _vp, _vp, _i, _i], _i),
    "ihip_gguf_open": ([C.c_char_p, C.POINTER(_u64)], _i),
    "ihip_gguf_close": ([_u64], _i),
    "ihip_gguf_info": ([_u64, C.POINTER(C.c_uint32), C.POINTER(_u64), C.POINTER(_u64),
                        C.POINTER(_i64)], _i),
    "ihip_gguf_tensor_info": ([_u64, _i64, C.c_char_p, _sz, C.POINTER(_i), C.POINTER(_i),
                               C.POINTER(_i64), C.POINTER(_u64), C.POINTER(_u64)], _i),
    "ihip_gguf_tensor_bytes": ([_u64, C.c_char_p, _vp, _sz], _i),
    "ihip_gguf_upload": ([_u64, C.c_char_p, C.POINTER(_u64)], _i),
    "ihip_gguf_upload_group": ([_u64, C.POINTER(C.c_char_p), _i, C.POINTER(_u64)], _i),
    "ihip_quantize_row_q8_k": ([_vp, _vp, _i64], _i),
    "ihip_vec_dot_q4_k_q8_k": ([_vp, _vp, _i, C.POINTER(C.c_float)], _i),
    "ihip_vec_dot_q5_k_q8_k": ([_vp, _vp, _i, C.POINTER(C.c_float)], _i),
    "ihip_vec_dot_q6_k_q8_k": ([_vp, _vp, _i, C.POINTER(C.c_float)], _i),
    "ihip_q4_k_gemv_q8k": ([_vp, _vp, _vp, _vp, _i, _i], _i),
    "ihip_q5_k_gemv_q8k": ([_vp, _vp, _vp, _vp, _i, _i], _i),
    "ihip_q6_k_gemv_q8k": ([_vp, _vp, _vp, _vp, _i, _i], _i),
    "ihip_dequantize": ([_i, _vp, _vp, _i64], _i),
    "ihip_ffn_swiglu": ([_i, _vp, _i, _vp, _i, _vp, _vp, _vp, _vp, _i, _i], _i),
    "ihip_lm_head_argmax": ([_i, _vp, _vp, _vp, C.POINTER(C.c_int32), _i, _i], _i),
    "ihip_prefill_q4_k": ([_vp, _vp, _vp, _i, _i, _i], _i),
    "ihip_ffn_block": ([_i, _vp, _i, _vp, _i, _vp, _vp, C.c_float, _vp, _i, _i], _i),
    "ihip_rmsnorm_dev": ([_vp, _vp, C.c_float, _vp, _i, _vp], _i),
    "ihip_ffn_block_dev": ([_i, _vp, _i, _vp, _i, _vp, _vp, C.c_float, _vp, _vp, _i, _i, _vp], _i),
    "ihip_lm_head_argmax_norm_dev": ([_i, _vp, _vp, C.c_float, _vp, _vp, _vp, _vp, _vp, _i, _i,
                                      _vp, _vp], _i),
    "ihip_gemv_dev": ([_i, _vp, _vp, _vp, _i, _i, _vp], _i),
    "ihip_gemv_add_dev": ([_i, _vp, _vp, _vp, _vp, _i, _i, _vp], _i),
    "ihip_gemv_norm_dev": ([_i, _vp, _vp, C.c_float, _vp, _vp, _vp, _i, _i, _vp], _i),
    "ihip_dequantize_dev": ([_i, _vp, _vp, _i64, _vp], _i),
    "ihip_gate_up_swiglu_dev": ([_i, _vp, _i, _vp, _vp, _vp, _i, _i, _vp], _i),
    "ihip_ffn_swiglu_dev": ([_i, _vp, _i, _vp, _i, _vp, _vp, _vp, _vp, _i, _i, _vp], _i),
    "ihip_lm_head_argmax_dev": ([_i, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp, _vp], _i),
    "ihip_lm_head_argmax_noalloc_dev": ([_i, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp], _i),
    "ihip_lm_head_fused": ([_i, _vp, _vp, _i, _i], _i),
    "ihip_ffn_block_scratch_floats": ([_i, _i, _i, _i], _sz),
    "ihip_argmax_dev": ([_vp, _i64, _vp, _vp, _vp, _vp], _i),
    "ihip_fused_mlp_gate_mul_dev": ([_vp, _vp, _i64, _vp], _i),
    "ihip_fused_silu_gate_mul_dev": ([_vp, _vp, _vp, _i64, _vp], _i),
    "ihip_prefill_q4_k_dev": ([_vp, _vp, _vp, _vp, _i, _i, _i, _vp], _i),
    "ihip_prefill_scratch_bytes": ([_i, _i], _sz),
    "ihip_prefill_q4_k_f32_dev": ([_vp, _vp, _vp, _i, _i, _i, _vp], _i),
    "ihip_prefill_convert_dev": ([_vp, _vp, _i, _i, _vp], _i),
    "ihip_prefill_q4_k_xh_dev": ([_vp, _vp, _vp, _i, _i, _i, _vp], _i),
    "ihip_quantize_row_q8_k_dev": ([_vp, _vp, _i64, _vp], _i),
    "ihip_gemv_q8k_dev": ([_i, _vp, _vp, _vp, _i, _i, _vp], _i),
    "ihip_gemv_q8k_x_dev": ([_i, _vp, _vp, _vp, _vp, _i, _i, _vp], _i),
}

_lib = None


def lib():
    """The loaded library (raises LibraryNotBuilt when it is absent)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise LibraryNotBuilt(f"{LIB_PATH} is missing: run python -m inferno_hip.build")
        L = C.CDLL(str(LIB_PATH))
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc == IHIP_OK:
        return
    msg = lib().ihip_last_error().decode(errors="replace")
    if rc in (IHIP_ERR_INVALID, IHIP_ERR_NONFINITE, IHIP_ERR_EMPTY):
        raise IHIPArgumentError(rc, msg)
    raise IHIPError(rc, msg)


def available() -> bool:
    try:
        return bool(lib().ihip_available())
    except LibraryNotBuilt:
        return False


