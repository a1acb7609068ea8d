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

import numpy as np

from . import _lib
from ._lib import Q4_K, Q5_K, Q6_K, Q8_0, IHIPArgumentError, check, lib
from .synth import BLOCK_BYTES, BLOCK_ELEMS

__all__ = ["quant_kernels_available", "q4_k_gemv_", "q5_k_gemv_", "q6_k_gemv_", "q8_0_gemv_"]


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


def forget(weight_data) -> None:
    """Drop the cached device copy of a host weight (call before reusing the
    host buffer for different bytes)."""
    check(lib().ihip_weight_forget(weight_data.ctypes.data))
