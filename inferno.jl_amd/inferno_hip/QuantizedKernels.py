"""Drop-in mirror of Inferno.jl's ``QuantizedKernels`` module
(src/QuantizedKernels.jl:14-16) running on the MI355X library.

Julia's ``q4_k_gemv!(out, weight_data, x, inner_dim, outer_dim)`` becomes
``q4_k_gemv_(out, weight_data, x, inner_dim, outer_dim)`` (trailing ``_`` for
the in-place ``!``).  Arguments have the reference's meaning: host arrays,
``weight_data`` the raw GGML block bytes of an ``outer_dim x inner_dim``
row-major matrix, ``out`` filled in place and returned.  Activations stay
fp32 on the GPU (the reference C path re-quantizes them to int8 first,
src/kernels/quant_kernels.c:608; see the fp32-activation note in
inferno_hip.synth / the oracle).

Errors: the reference raises ``ErrorException("Quantized C kernel not
available")`` when the library is missing (src/QuantizedKernels.jl:86); here
that is ``inferno_hip._lib.LibraryNotBuilt`` / ``IHIPError``.  Shape checks
that the reference makes with ``@assert`` (src/QuantsCPU.jl:46-49,
src/QuantizedKernels.jl:64) raise ``IHIPArgumentError`` (a ValueError).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import IQ4_NL, Q4_K, Q5_K, Q6_K, Q8_0, IHIPArgumentError, check, lib
from .synth import BLOCK_BYTES, BLOCK_ELEMS

__all__ = ["quant_kernels_available", "q4_k_gemv_", "q5_k_gemv_", "q6_k_gemv_", "q8_0_gemv_",
           "quantize_q8_k_", "vec_dot_q4_k_q8_k", "vec_dot_q5_k_q8_k", "vec_dot_q6_k_q8_k",
           "q4_k_gemv_q8k_", "q5_k_gemv_q8k_", "q6_k_gemv_q8k_"]


def quant_kernels_available() -> bool:
    """src/QuantizedKernels.jl:50-51: true when the kernels can run (a gfx950
    device is present and IHIP_DISABLE is unset)."""
    return _lib.available()


def _args(ggml_type, out, weight_data, x, inner_dim, outer_dim):
    if inner_dim <= 0 or outer_dim <= 0 or inner_dim % BLOCK_ELEMS[ggml_type]:
        raise IHIPArgumentError(_lib.IHIP_ERR_INVALID,
                                f"inner_dim={inner_dim} must be a positive multiple of "
                                f"{BLOCK_ELEMS[ggml_type]}")
    need = outer_dim * (inner_dim // BLOCK_ELEMS[ggml_type]) * BLOCK_BYTES[ggml_type]
    for name, a, dt, n in (("out", out, np.float32, outer_dim), ("x", x, np.float32, inner_dim),
                           ("weight_data", weight_data, np.uint8, need)):
        if not isinstance(a, np.ndarray) or a.dtype != dt or not a.flags.c_contiguous:
            raise IHIPArgumentError(_lib.IHIP_ERR_INVALID, f"{name} must be a contiguous {dt.__name__} array")
        if a.size < n:
            raise IHIPArgumentError(_lib.IHIP_ERR_INVALID, f"{name} has {a.size} elements, needs {n}")
    return weight_data.ctypes.data, x.ctypes.data, out.ctypes.data


def q4_k_gemv_(out, weight_data, x, inner_dim, outer_dim):
    w, xp, op = _args(Q4_K, out, weight_data, x, inner_dim, outer_dim)
    check(lib().ihip_q4_k_gemv(w, xp, op, None, inner_dim, outer_dim))
    return out


def q5_k_gemv_(out, weight_data, x, inner_dim, outer_dim):
    w, xp, op = _args(Q5_K, out, weight_data, x, inner_dim, outer_dim)
    check(lib().ihip_q5_k_gemv(w, xp, op, None, inner_dim, outer_dim))
    return out


def q6_k_gemv_(out, weight_data, x, inner_dim, outer_dim):
    w, xp, op = _args(Q6_K, out, weight_data, x, inner_dim, outer_dim)
    check(lib().ihip_q6_k_gemv(w, xp, op, None, inner_dim, outer_dim))
    return out


def q8_0_gemv_(out, weight_data, x, inner_dim, outer_dim):
    w, xp, op = _args(Q8_0, out, weight_data, x, inner_dim, outer_dim)
    check(lib().ihip_q8_0_gemv(w, xp, op, inner_dim, outer_dim))
    return out


def iq4_nl_gemv_(out, weight_data, x, inner_dim, outer_dim):
    """mul_quant_mat_vec(::IQ4NL_Matrix, x, out) (src/ModelCPU.jl:381-408)."""
    w, xp, op = _args(IQ4_NL, out, weight_data, x, inner_dim, outer_dim)
    check(lib().ihip_iq4_nl_gemv(w, xp, op, inner_dim, outer_dim))
    return out


# ---- the int8-activation variant: the reference C numerics, bit for bit ----

Q8_K_BYTES = _lib.Q8_K_BYTES


def _u8(name, a, n):
    if not isinstance(a, np.ndarray) or a.dtype != np.uint8 or not a.flags.c_contiguous:
        raise IHIPArgumentError(_lib.IHIP_ERR_INVALID, f"{name} must be a contiguous uint8 array")
    if a.size < n:
        raise IHIPArgumentError(_lib.IHIP_ERR_INVALID, f"{name} has {a.size} bytes, needs {n}")
    return a.ctypes.data


def quantize_q8_k_(q8_buf, x, inner_dim):
    """quantize_q8_k!(q8_buf, x, inner_dim) (src/QuantizedKernels.jl:151-156):
    x (fp32, inner_dim a multiple of 256) into inner_dim/256 Q8_K blocks of
    292 bytes in q8_buf, exactly as quantize_row_q8_K
    (src/kernels/quant_kernels.c:166-194).  The reference's ccall passes the
    two pointers in swapped order; this mirror keeps the meaning of its Julia
    arguments and calls the C-order entry point."""
    if inner_dim <= 0 or inner_dim % 256:
        raise IHIPArgumentError(_lib.IHIP_ERR_INVALID, f"inner_dim={inner_dim} must be a positive multiple of 256")
    if not isinstance(x, np.ndarray) or x.dtype != np.float32 or not x.flags.c_contiguous or x.size < inner_dim:
        raise IHIPArgumentError(_lib.IHIP_ERR_INVALID, "x must be a contiguous float32 array of inner_dim")
    yp = _u8("q8_buf", q8_buf, inner_dim // 256 * Q8_K_BYTES)
    check(lib().ihip_quantize_row_q8_k(x.ctypes.data, yp, inner_dim))
    return q8_buf


def _vec_dot(fn, ggml_type, weight, q8, nb):
    if nb <= 0:
        raise IHIPArgumentError(_lib.IHIP_ERR_INVALID, f"nb={nb} must be positive")
    wp = _u8("weight", weight, nb * BLOCK_BYTES[ggml_type])
    qp = _u8("q8", q8, nb * Q8_K_BYTES)
    s = ctypes.c_float(0.0)
    check(fn(wp, qp, nb, ctypes.byref(s)))
    return np.float32(s.value)


def vec_dot_q4_k_q8_k(weight, q8, nb):
    """vec_dot_q4_k_q8_k(weight_ptr, q8_ptr, nb) (src/QuantizedKernels.jl:159-164):
    one row of nb Q4_K blocks against nb Q8_K blocks, as vec_dot_q4_K_q8_K
    (src/kernels/quant_kernels.c:204-277) computes it."""
    return _vec_dot(lib().ihip_vec_dot_q4_k_q8_k, Q4_K, weight, q8, nb)


def vec_dot_q5_k_q8_k(weight, q8, nb):
    """src/QuantizedKernels.jl:166-171 / quant_kernels.c:311-397."""
    return _vec_dot(lib().ihip_vec_dot_q5_k_q8_k, Q5_K, weight, q8, nb)


def vec_dot_q6_k_q8_k(weight, q8, nb):
    """src/QuantizedKernels.jl:173-178 / quant_kernels.c:440-521."""
    return _vec_dot(lib().ihip_vec_dot_q6_k_q8_k, Q6_K, weight, q8, nb)


def _gemv_q8k(fn, ggml_type, out, weight_data, x, inner_dim, outer_dim, q8_buf):
    w, xp, op = _args(ggml_type, out, weight_data, x, inner_dim, outer_dim)
    qp = None if q8_buf is None else _u8("q8_buf", q8_buf, inner_dim // 256 * Q8_K_BYTES)
    check(fn(w, xp, op, qp, inner_dim, outer_dim))
    return out


def q4_k_gemv_q8k_(out, weight_data, x, inner_dim, outer_dim, q8_buf=None):
    """q4_k_gemv! with the reference C numerics (x re-quantized to Q8_K,
    src/kernels/quant_kernels.c:602-614): bit-identical to the C library."""
    return _gemv_q8k(lib().ihip_q4_k_gemv_q8k, Q4_K, out, weight_data, x, inner_dim, outer_dim, q8_buf)


def q5_k_gemv_q8k_(out, weight_data, x, inner_dim, outer_dim, q8_buf=None):
    """quant_kernels.c:620-632 numerics."""
    return _gemv_q8k(lib().ihip_q5_k_gemv_q8k, Q5_K, out, weight_data, x, inner_dim, outer_dim, q8_buf)


def q6_k_gemv_q8k_(out, weight_data, x, inner_dim, outer_dim, q8_buf=None):
    """quant_kernels.c:638-650 numerics."""
    return _gemv_q8k(lib().ihip_q6_k_gemv_q8k, Q6_K, out, weight_data, x, inner_dim, outer_dim, q8_buf)


def forget(weight_data) -> None:
    """Drop the cached device copy of a host weight (call before reusing the
    host buffer for different bytes)."""
    check(lib().ihip_weight_forget(weight_data.ctypes.data))
