"""Drop-in mirror of Inferno.jl's ``Dequant`` exports (src/Dequant.jl:5-6):
``dequantize_q4_k(data, num_elements) -> float32 vector`` and friends, run
bit-exactly on the MI355X (src/Dequant.jl:304-601 semantics)."""
from __future__ import annotations

import numpy as np

from . import _lib
from ._lib import IQ4_NL, Q4_K, Q5_K, Q6_K, Q8_0, IHIPArgumentError, check, lib
from .synth import BLOCK_BYTES, BLOCK_ELEMS

__all__ = ["dequantize_q4_k", "dequantize_q5_k", "dequantize_q6_k", "dequantize_q8_0",
           "dequantize_iq4_nl", "dequantize"]


def dequantize(ggml_type: int, data: np.ndarray, num_elements: int) -> np.ndarray:
    be = BLOCK_ELEMS[ggml_type]
    if num_elements < 0 or num_elements % be:
        raise IHIPArgumentError(_lib.IHIP_ERR_INVALID, f"num_elements={num_elements} not a multiple of {be}")
    data = np.ascontiguousarray(data, dtype=np.uint8)
    if data.size < num_elements // be * BLOCK_BYTES[ggml_type]:
        raise IHIPArgumentError(_lib.IHIP_ERR_INVALID, "data too short")
    out = np.empty(num_elements, dtype=np.float32)
    if num_elements:
        check(lib().ihip_dequantize(ggml_type, data.ctypes.data, out.ctypes.data, num_elements))
    return out


def dequantize_q4_k(data, num_elements):
    return dequantize(Q4_K, data, num_elements)


def dequantize_q5_k(data, num_elements):
    return dequantize(Q5_K, data, num_elements)


def dequantize_q6_k(data, num_elements):
    return dequantize(Q6_K, data, num_elements)


def dequantize_q8_0(data, num_elements):
    return dequantize(Q8_0, data, num_elements)


def dequantize_iq4_nl(data, num_elements):
    """src/Dequant.jl:655-693: d * KVALUES_IQ4NL[nibble], 32 per 18-byte block."""
    return dequantize(IQ4_NL, data, num_elements)
