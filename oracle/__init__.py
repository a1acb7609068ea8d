"""ctypes view of the CPU parity checker (test infrastructure only).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this package, and only as the checker or the timed CPU baseline.
The product library never calls it.

* ``lib()``      -- oracle/_build/libkquant_oracle.so, the C restatement in
                    kquant_oracle.c (every function cites the reference line
                    it restates).
* ``ref_lib()``  -- oracle/_ref/libquant_ref.so, the reference's own
                    src/kernels/quant_kernels.c compiled from source by
                    oracle/Makefile, or None when it has not been built.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libkquant_oracle.so"
REF_PATH = HERE / "_ref" / "libquant_ref.so"

Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14
Q8K_BYTES = 292

_lib = None
_ref = None

_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")


def build() -> None:
    """Compile the oracle (and oracle/_ref where the reference source exists)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        L.orc_half_to_float.argtypes = [C.c_uint16]
        L.orc_half_to_float.restype = C.c_float
        L.orc_float_to_half_rne.argtypes = [C.c_float]
        L.orc_float_to_half_rne.restype = C.c_uint16
        L.orc_dequant.argtypes = [C.c_int, _u8p, _f32p, C.c_int64]
        L.orc_gemv_f64.argtypes = [C.c_int, _u8p, _f32p, _f64p, C.c_int, C.c_int]
        L.orc_row_norms.argtypes = [C.c_int, _u8p, _f64p, C.c_int, C.c_int]
        L.orc_gemm_f64.argtypes = [C.c_int, _u8p, _f32p, _f64p, C.c_int, C.c_int, C.c_int]
        L.orc_gemv_f32_serial.argtypes = [C.c_int, _u8p, _f32p, _f32p, C.c_int, C.c_int]
        L.orc_argmax.argtypes = [_f32p, C.c_int64, C.POINTER(C.c_int64), C.POINTER(C.c_int)]
        L.orc_ffn_swiglu_f64.argtypes = [C.c_int, _u8p, C.c_int, _u8p, C.c_int, _u8p, _f32p,
                                         C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p,
                                         _f64p]
        L.orc_rmsnorm_f64.argtypes = [_f32p, _f32p, C.c_float, C.c_int, _f64p]
        L.orc_ffn_block_f64.argtypes = [C.c_int, _u8p, C.c_int, _u8p, C.c_int, _u8p, _f32p, _f32p,
                                        C.c_float, C.c_int, C.c_int, _f64p, _f64p, _f64p, _f64p,
                                        _f64p]
        L.orc_quantize_row_q8k.argtypes = [_f32p, _u8p, C.c_int64]
        L.orc_gemv_q8k.argtypes = [C.c_int, _u8p, _f32p, _f32p, _u8p, C.c_int, C.c_int]
        L.orc_gemv_q8_0_lanes.argtypes = [_u8p, _f32p, _f32p, C.c_int, C.c_int]
        for name in ("orc_dequant", "orc_gemv_f64", "orc_gemm_f64", "orc_row_norms", "orc_gemv_f32_serial",
                     "orc_argmax", "orc_ffn_swiglu_f64", "orc_rmsnorm_f64", "orc_ffn_block_f64",
                     "orc_quantize_row_q8k",
                     "orc_gemv_q8k", "orc_gemv_q8_0_lanes"):
            getattr(L, name).restype = C.c_int
        _lib = L
    return _lib


def ref_lib():
    """The reference's quant_kernels.c compiled from source, or None."""
    global _ref
    if _ref is None and REF_PATH.exists():
        R = C.CDLL(str(REF_PATH))
        for n in ("q4_k_gemv", "q5_k_gemv", "q6_k_gemv"):
            getattr(R, n).argtypes = [_u8p, _f32p, _f32p, _u8p, C.c_int, C.c_int]
            getattr(R, n).restype = None
        R.q8_0_gemv.argtypes = [_u8p, _f32p, _f32p, C.c_int, C.c_int]
        R.q8_0_gemv.restype = None
        R.quantize_row_q8_K.argtypes = [_f32p, _u8p, C.c_int64]
        R.quantize_row_q8_K.restype = None
        _ref = R
    return _ref


def _chk(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"oracle {what} failed ({rc})")


def half_to_float(h: int) -> float:
    return lib().orc_half_to_float(h)


def float_to_half(f: float) -> int:
    return lib().orc_float_to_half_rne(f)


def dequant(ggml_type: int, data: np.ndarray, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    _chk(lib().orc_dequant(ggml_type, np.ascontiguousarray(data, np.uint8), out, n), "dequant")
    return out


def gemv_f64(ggml_type: int, w: np.ndarray, x: np.ndarray, inner: int, outer: int) -> np.ndarray:
    out = np.empty(outer, dtype=np.float64)
    _chk(lib().orc_gemv_f64(ggml_type, w, np.ascontiguousarray(x, np.float32), out, inner, outer),
         "gemv_f64")
    return out


def gemm_f64(ggml_type: int, w: np.ndarray, X: np.ndarray, inner: int,
             outer: int) -> np.ndarray:
    """T x outer fp64 outputs of the per-token loop (row t = gemv_f64 of X[t])."""
    X = np.ascontiguousarray(X, np.float32)
    T = X.shape[0]
    Y = np.empty((T, outer), dtype=np.float64)
    _chk(lib().orc_gemm_f64(ggml_type, w, X.reshape(-1), Y.reshape(-1), T, inner, outer),
         "gemm_f64")
    return Y


def row_norms(ggml_type: int, w: np.ndarray, inner: int, outer: int) -> np.ndarray:
    out = np.empty(outer, dtype=np.float64)
    _chk(lib().orc_row_norms(ggml_type, w, out, inner, outer), "row_norms")
    return out


def gemv_f32_serial(ggml_type: int, w: np.ndarray, x: np.ndarray, inner: int,
                    outer: int) -> np.ndarray:
    out = np.empty(outer, dtype=np.float32)
    _chk(lib().orc_gemv_f32_serial(ggml_type, w, np.ascontiguousarray(x, np.float32), out,
                                   inner, outer), "gemv_f32_serial")
    return out


def argmax(logits: np.ndarray):
    """(index, all_neg_inf) with 0-based index, or raises ValueError like
    src/CommonOps.jl:149-152 raises ArgumentError."""
    idx = C.c_int64(0)
    ani = C.c_int(0)
    rc = lib().orc_argmax(np.ascontiguousarray(logits, np.float32), len(logits),
                          C.byref(idx), C.byref(ani))
    if rc == -1:
        raise ValueError("logits must not contain NaN")
    if rc == -2:
        raise ValueError("logits must not contain +Inf")
    if rc == -3:
        raise ValueError("logits must not be empty")
    return int(idx.value), bool(ani.value)


def ffn_swiglu_f64(gtype, wg, utype, wu, dtype_, wd, x, hidden, inter):
    g = np.empty(inter, np.float64)
    u = np.empty(inter, np.float64)
    h = np.empty(inter, np.float64)
    y = np.empty(hidden, np.float64)
    _chk(lib().orc_ffn_swiglu_f64(gtype, wg, utype, wu, dtype_, wd,
                                  np.ascontiguousarray(x, np.float32), hidden, inter,
                                  g.ctypes.data, u.ctypes.data, h.ctypes.data, y), "ffn")
    return g, u, h, y


def rmsnorm_f64(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    out = np.empty(len(x), np.float64)
    _chk(lib().orc_rmsnorm_f64(np.ascontiguousarray(x, np.float32), np.ascontiguousarray(w, np.float32),
                               eps, len(x), out), "rmsnorm")
    return out


def ffn_block_f64(gtype, wg, utype, wu, dtype_, wd, x, nw, eps, hidden, inter):
    n = np.empty(hidden, np.float64)
    g, u, h = (np.empty(inter, np.float64) for _ in range(3))
    y = np.empty(hidden, np.float64)
    _chk(lib().orc_ffn_block_f64(gtype, wg, utype, wu, dtype_, wd, np.ascontiguousarray(x, np.float32),
                                 np.ascontiguousarray(nw, np.float32), eps, hidden, inter,
                                 n, g, u, h, y), "ffn_block")
    return n, g, u, h, y


def quantize_row_q8k(x: np.ndarray) -> np.ndarray:
    out = np.zeros(len(x) // 256 * Q8K_BYTES, dtype=np.uint8)
    _chk(lib().orc_quantize_row_q8k(np.ascontiguousarray(x, np.float32), out, len(x)), "q8k")
    return out


def gemv_q8k(ggml_type: int, w: np.ndarray, x: np.ndarray, inner: int, outer: int) -> np.ndarray:
    out = np.empty(outer, dtype=np.float32)
    q8 = np.zeros(inner // 256 * Q8K_BYTES, dtype=np.uint8)
    _chk(lib().orc_gemv_q8k(ggml_type, w, np.ascontiguousarray(x, np.float32), out, q8,
                            inner, outer), "gemv_q8k")
    return out


def gemv_q8_0_lanes(w: np.ndarray, x: np.ndarray, inner: int, outer: int) -> np.ndarray:
    out = np.empty(outer, dtype=np.float32)
    _chk(lib().orc_gemv_q8_0_lanes(w, np.ascontiguousarray(x, np.float32), out, inner, outer),
         "q8_0_lanes")
    return out


def ref_gemv(ggml_type: int, w: np.ndarray, x: np.ndarray, inner: int, outer: int) -> np.ndarray:
    """Run the compiled reference C GEMV (the path QuantizedKernels.q*_gemv!
    calls, src/QuantizedKernels.jl:84-148)."""
    R = ref_lib()
    if R is None:
        raise FileNotFoundError(str(REF_PATH))
    out = np.empty(outer, dtype=np.float32)
    x = np.ascontiguousarray(x, np.float32)
    if ggml_type == Q8_0:
        R.q8_0_gemv(w, x, out, inner, outer)
    else:
        q8 = np.zeros(inner // 256 * Q8K_BYTES, dtype=np.uint8)
        fn = {Q4_K: R.q4_k_gemv, Q5_K: R.q5_k_gemv, Q6_K: R.q6_k_gemv}[ggml_type]
        fn(w, x, out, q8, inner, outer)
    return out


def ref_quantize_row_q8k(x: np.ndarray) -> np.ndarray:
    R = ref_lib()
    if R is None:
        raise FileNotFoundError(str(REF_PATH))
    out = np.zeros(len(x) // 256 * Q8K_BYTES, dtype=np.uint8)
    R.quantize_row_q8_K(np.ascontiguousarray(x, np.float32), out, len(x))
    return out


def tolerance(norms: np.ndarray, x: np.ndarray) -> np.ndarray:
    """The parity bound for fp32-accumulated outputs: 1e-4 * ||w_row|| * ||x||."""
    return 1e-4 * norms * float(np.linalg.norm(np.asarray(x, np.float64)))

