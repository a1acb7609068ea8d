"""Seeded synthetic GGML blocks and activations.

The block fields follow the distributions of the decode workloads this
library is measured on:

* Q4_K / Q5_K (144 / 176 B): fp16 ``d`` and ``dmin`` drawn as |N(0,1)|*0.01,
  12 packed scale bytes uniform 0..255 (the 12-byte -> 16 six-bit-field
  unpack is a bijection on bits, so uniform bytes give uniform 0..63 scales
  and mins), ``qh`` and ``qs`` bytes uniform.
* Q6_K (210 B): ``ql``/``qh`` bytes uniform, 16 int8 scales uniform -32..31,
  fp16 ``d`` drawn as |N(0,1)|*0.005.
* Q8_0 (34 B): fp16 ``d`` drawn as |N(0,1)|*0.01, 32 int8 quants uniform
  -127..127.
* activations: fp32 N(0,1).

Block byte layouts are those of src/kernels/quant_kernels.c:24-62 and
src/Dequant.jl:311-316, 336-341, 392-400, 570-574 (Inferno.jl).
"""
from __future__ import annotations

import numpy as np

Q8_0, Q4_K, Q5_K, Q6_K, IQ4_NL = 8, 12, 13, 14, 20
BLOCK_BYTES = {Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210, IQ4_NL: 18}
BLOCK_ELEMS = {Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256, IQ4_NL: 32}
TYPE_NAMES = {Q8_0: "Q8_0", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K", IQ4_NL: "IQ4_NL"}


def rng_for(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def _half_bytes(values: np.ndarray) -> np.ndarray:
    """fp32/fp64 -> fp16 (round to nearest even) -> little-endian byte pairs."""
    h = np.asarray(values, dtype=np.float64).astype(np.float16)
    return h.view(np.uint8).reshape(-1, 2)


def q4_k_blocks(rng: np.random.Generator, nblocks: int) -> np.ndarray:
    b = np.empty((nblocks, 144), dtype=np.uint8)
    b[:, 0:2] = _half_bytes(np.abs(rng.standard_normal(nblocks)) * 0.01)
    b[:, 2:4] = _half_bytes(np.abs(rng.standard_normal(nblocks)) * 0.01)
    b[:, 4:144] = rng.integers(0, 256, size=(nblocks, 140), dtype=np.uint8)
    return b.reshape(-1)


def q5_k_blocks(rng: np.random.Generator, nblocks: int) -> np.ndarray:
    b = np.empty((nblocks, 176), dtype=np.uint8)
    b[:, 0:2] = _half_bytes(np.abs(rng.standard_normal(nblocks)) * 0.01)
    b[:, 2:4] = _half_bytes(np.abs(rng.standard_normal(nblocks)) * 0.01)
    b[:, 4:176] = rng.integers(0, 256, size=(nblocks, 172), dtype=np.uint8)
    return b.reshape(-1)


def q6_k_blocks(rng: np.random.Generator, nblocks: int) -> np.ndarray:
    b = np.empty((nblocks, 210), dtype=np.uint8)
    b[:, 0:192] = rng.integers(0, 256, size=(nblocks, 192), dtype=np.uint8)
    b[:, 192:208] = rng.integers(-32, 32, size=(nblocks, 16), dtype=np.int8).view(np.uint8)
    b[:, 208:210] = _half_bytes(np.abs(rng.standard_normal(nblocks)) * 0.005)
    return b.reshape(-1)


def q8_0_blocks(rng: np.random.Generator, nblocks: int) -> np.ndarray:
    b = np.empty((nblocks, 34), dtype=np.uint8)
    b[:, 0:2] = _half_bytes(np.abs(rng.standard_normal(nblocks)) * 0.01)
    b[:, 2:34] = rng.integers(-127, 128, size=(nblocks, 32), dtype=np.int8).view(np.uint8)
    return b.reshape(-1)


def iq4_nl_blocks(rng: np.random.Generator, nblocks: int) -> np.ndarray:
    b = np.empty((nblocks, 18), dtype=np.uint8)
    b[:, 0:2] = _half_bytes(np.abs(rng.standard_normal(nblocks)) * 0.0005)
    b[:, 2:18] = rng.integers(0, 256, size=(nblocks, 16), dtype=np.uint8)
    return b.reshape(-1)


_GEN = {Q4_K: q4_k_blocks, Q5_K: q5_k_blocks, Q6_K: q6_k_blocks, Q8_0: q8_0_blocks,
        IQ4_NL: iq4_nl_blocks}


def weight(rng: np.random.Generator, ggml_type: int, outer: int, inner: int) -> np.ndarray:
    """Row-major quantized matrix: `outer` rows of `inner` elements."""
    be = BLOCK_ELEMS[ggml_type]
    if inner % be:
        raise ValueError(f"inner={inner} not a multiple of {be}")
    return _GEN[ggml_type](rng, outer * (inner // be))


def activations(rng: np.random.Generator, n: int) -> np.ndarray:
    return rng.standard_normal(n).astype(np.float32)


def nbytes(ggml_type: int, outer: int, inner: int) -> int:
    return outer * (inner // BLOCK_ELEMS[ggml_type]) * BLOCK_BYTES[ggml_type]
