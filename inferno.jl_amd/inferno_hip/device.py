"""Device-resident entry points over torch CUDA(HIP) tensors.

torch only provides device memory and the stream here; all computation runs
in libinferno_hip.so.  Each function takes device tensors, launches on
torch's current stream (or ``stream``) and returns without synchronizing.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import Q4_K, IHIPArgumentError, check, lib
from .synth import BLOCK_BYTES, BLOCK_ELEMS


# torch's current-stream handle without building a Stream object (2-3 us of
# host time per call otherwise); the public API where torch lacks it.
_raw_current_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(stream=None) -> int:
    if stream is not None:
        return stream.cuda_stream
    if _raw_current_stream is not None:
        return _raw_current_stream(torch.cuda.current_device())
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor, dtype=None, what="tensor") -> int:
    if not t.is_cuda:
        raise IHIPArgumentError(_lib.IHIP_ERR_INVALID, f"{what} must be a device tensor")
    if dtype is not None and t.dtype != dtype:
        raise IHIPArgumentError(_lib.IHIP_ERR_INVALID, f"{what} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise IHIPArgumentError(_lib.IHIP_ERR_INVALID, f"{what} must be contiguous")
    return t.data_ptr()


@dataclass
class DeviceWeight:
    """GGML blocks of an ``outer x inner`` row-major matrix in device memory."""
    data: torch.Tensor        # uint8, device
    ggml_type: int
    inner: int
    outer: int

    @classmethod
    def upload(cls, host_bytes, ggml_type: int, inner: int, outer: int, device="cuda"):
        t = torch.as_tensor(host_bytes, dtype=torch.uint8).to(device)
        w = cls(t, ggml_type, inner, outer)
        w.validate()
        return w

    def validate(self):
        be = BLOCK_ELEMS[self.ggml_type]
        need = self.outer * (self.inner // be) * BLOCK_BYTES[self.ggml_type]
        if self.inner % be or self.data.numel() < need:
            raise IHIPArgumentError(_lib.IHIP_ERR_INVALID, "weight bytes do not match the shape")

    @property
    def nbytes(self) -> int:
        return self.outer * (self.inner // BLOCK_ELEMS[self.ggml_type]) * BLOCK_BYTES[self.ggml_type]


class ArgmaxWorkspace:
    """IHIP_ARGMAX_WS_BYTES of device memory for the per-workgroup partial
    maxima, plus the token/flags outputs.  Calls sharing one workspace must
    not overlap on the GPU."""

    def __init__(self, device="cuda"):
        self.ws = torch.zeros(_lib.ARGMAX_WS_BYTES, dtype=torch.uint8, device=device)
        self.token = torch.zeros(1, dtype=torch.int32, device=device)
        self.flags = torch.zeros(1, dtype=torch.int32, device=device)

    def result(self) -> int:
        """Synchronize and return the 0-based token, raising like
        src/CommonOps.jl:149-152 on NaN/+Inf."""
        torch.cuda.synchronize()
        fl = int(self.flags.item())
        if fl & _lib.FLAG_NAN:
            raise IHIPArgumentError(_lib.IHIP_ERR_NONFINITE, "logits must not contain NaN")
        if fl & _lib.FLAG_POSINF:
            raise IHIPArgumentError(_lib.IHIP_ERR_NONFINITE, "logits must not contain +Inf")
        return int(self.token.item())


class WeightGroup:
    """Host weights of one GGML type and row length uploaded back to back as
    one registered weight (ihip_weight_register_group), e.g. wq, wk and wv:
    `whole` is the group as one DeviceWeight of the summed rows, `members[i]`
    member i's rows inside it, `offsets[i]` its first output row.  Freed by
    release()."""

    def __init__(self, hosts, ggml_type: int, inner: int, outers):
        import numpy as np
        src = [np.ascontiguousarray(h, dtype=np.uint8) for h in hosts]  # alive through the upload
        n = len(src)
        ptrs = (C.c_void_p * n)(*[a.ctypes.data for a in src])
        rows = (C.c_int * n)(*outers)
        h = C.c_uint64(0)
        check(lib().ihip_weight_register_group(ptrs, rows, n, ggml_type, inner, C.byref(h)))
        del src
        self.handle = h.value
        p = C.c_void_p(0)
        check(lib().ihip_weight_device_ptr(self.handle, C.byref(p)))
        self.ptr = p.value
        self.ggml_type, self.inner, self.outers = ggml_type, inner, list(outers)
        self.offsets = [sum(outers[:i]) for i in range(n)]

    def member_ptr(self, i: int) -> int:
        return self.ptr + lib().ihip_weight_bytes(self.ggml_type, self.inner, self.offsets[i])

    def gemv_norm(self, norm_w: torch.Tensor, eps: float, x: torch.Tensor, out: torch.Tensor = None,
                  xn: torch.Tensor = None, stream=None) -> torch.Tensor:
        """Every member's outputs of the normed x in one launch where the norm
        folds (ihip_gemv_norm_dev over the group)."""
        total = sum(self.outers)
        if out is None:
            out = torch.empty(total, dtype=torch.float32, device=x.device)
        if xn is None:
            xn = torch.empty(self.inner, dtype=torch.float32, device=x.device)
        check(lib().ihip_gemv_norm_dev(self.ggml_type, self.ptr, _ptr(norm_w, torch.float32, "norm_w"), eps,
                                       _ptr(x, torch.float32, "x"), _ptr(xn, torch.float32, "xn"),
                                       _ptr(out, torch.float32, "out"), self.inner, total, _stream(stream)))
        return out

    def gemv(self, x: torch.Tensor, out: torch.Tensor = None, stream=None) -> torch.Tensor:
        """Every member's outputs in one launch: out[offsets[i]:][:outers[i]]."""
        total = sum(self.outers)
        if out is None:
            out = torch.empty(total, dtype=torch.float32, device=x.device)
        check(lib().ihip_gemv_dev(self.ggml_type, self.ptr, _ptr(x, torch.float32, "x"),
                                  _ptr(out, torch.float32, "out"), self.inner, total, _stream(stream)))
        return out

    def release(self):
        if self.handle:
            check(lib().ihip_weight_release(self.handle))
            self.handle = 0


def gemv(w: DeviceWeight, x: torch.Tensor, out: torch.Tensor = None, stream=None):
    if out is None:
        out = torch.empty(w.outer, dtype=torch.float32, device=x.device)
    check(lib().ihip_gemv_dev(w.ggml_type, _ptr(w.data, torch.uint8, "w"), _ptr(x, torch.float32, "x"),
                              _ptr(out, torch.float32, "out"), w.inner, w.outer, _stream(stream)))
    return out


def gemv_add(w: DeviceWeight, x: torch.Tensor, resid: torch.Tensor, out: torch.Tensor = None,
             stream=None) -> torch.Tensor:
    """out = resid + W x in one launch (ihip_gemv_add_dev); out defaults to
    resid (in place), as the layer's x .+= residual (src/ModelCPU.jl:909)."""
    if out is None:
        out = resid
    check(lib().ihip_gemv_add_dev(w.ggml_type, _ptr(w.data), _ptr(x, torch.float32, "x"),
                                  _ptr(resid, torch.float32, "resid"), _ptr(out, torch.float32, "out"),
                                  w.inner, w.outer, _stream(stream)))
    return out


def gemv_norm(w: DeviceWeight, norm_w: torch.Tensor, eps: float, x: torch.Tensor,
              out: torch.Tensor = None, xn: torch.Tensor = None, stream=None) -> torch.Tensor:
    """out = W (rmsnorm(x) .* norm_w) (ihip_gemv_norm_dev): one launch where
    the norm folds into the GEMV, else the norm into xn (allocated here when
    not given) and the plain GEMV."""
    if out is None:
        out = torch.empty(w.outer, dtype=torch.float32, device=x.device)
    if xn is None:
        xn = torch.empty(w.inner, dtype=torch.float32, device=x.device)
    check(lib().ihip_gemv_norm_dev(w.ggml_type, _ptr(w.data), _ptr(norm_w, torch.float32, "norm_w"),
                                   eps, _ptr(x, torch.float32, "x"), _ptr(xn, torch.float32, "xn"),
                                   _ptr(out, torch.float32, "out"), w.inner, w.outer, _stream(stream)))
    return out


def dequantize(w: DeviceWeight, out: torch.Tensor = None, stream=None):
    n = w.inner * w.outer
    if out is None:
        out = torch.empty(n, dtype=torch.float32, device=w.data.device)
    check(lib().ihip_dequantize_dev(w.ggml_type, _ptr(w.data, torch.uint8, "w"),
                                    _ptr(out, torch.float32, "out"), n, _stream(stream)))
    return out


def gate_up_swiglu(wg: DeviceWeight, wu: DeviceWeight, x, h=None, stream=None):
    if h is None:
        h = torch.empty(wg.outer, dtype=torch.float32, device=x.device)
    check(lib().ihip_gate_up_swiglu_dev(wg.ggml_type, _ptr(wg.data), wu.ggml_type, _ptr(wu.data),
                                        _ptr(x, torch.float32, "x"), _ptr(h, torch.float32, "h"),
                                        wg.inner, wg.outer, _stream(stream)))
    return h


def ffn_swiglu(wg: DeviceWeight, wu: DeviceWeight, wd: DeviceWeight, x, h=None, y=None, stream=None):
    if h is None:
        h = torch.empty(wg.outer, dtype=torch.float32, device=x.device)
    if y is None:
        y = torch.empty(wd.outer, dtype=torch.float32, device=x.device)
    check(lib().ihip_ffn_swiglu_dev(wg.ggml_type, _ptr(wg.data), wu.ggml_type, _ptr(wu.data),
                                    wd.ggml_type, _ptr(wd.data), _ptr(x, torch.float32, "x"),
                                    _ptr(h, torch.float32, "h"), _ptr(y, torch.float32, "y"),
                                    wg.inner, wg.outer, _stream(stream)))
    return y


def lm_head_argmax(w: DeviceWeight, x, ws: ArgmaxWorkspace, logits=None, stream=None):
    """logits may be None; where the argmax is not fused into the GEMV (other
    types or shapes) a logits buffer is allocated for the call."""
    if logits is None and not lib().ihip_lm_head_fused(w.ggml_type, _ptr(w.data), _ptr(x, torch.float32, "x"),
                                                       w.inner, w.outer):
        logits = torch.empty(w.outer, dtype=torch.float32, device=x.device)
    lp = _ptr(logits, torch.float32, "logits") if logits is not None else None
    check(lib().ihip_lm_head_argmax_dev(w.ggml_type, _ptr(w.data), _ptr(x, torch.float32, "x"), lp,
                                        ws.token.data_ptr(), ws.flags.data_ptr(), w.inner, w.outer,
                                        ws.ws.data_ptr(), _stream(stream)))
    return logits


def argmax(logits: torch.Tensor, ws: ArgmaxWorkspace, stream=None):
    check(lib().ihip_argmax_dev(_ptr(logits, torch.float32, "logits"), logits.numel(),
                                ws.token.data_ptr(), ws.flags.data_ptr(), ws.ws.data_ptr(),
                                _stream(stream)))


def prefill_scratch(T: int, inner: int, device="cuda") -> torch.Tensor:
    """Caller scratch of ihip_prefill_q4_k_dev: the fp16 activations, one
    scale exponent per token and the partial sums of a split over K
    (ihip_prefill_scratch_bytes bytes)."""
    return torch.empty(lib().ihip_prefill_scratch_bytes(T, inner), dtype=torch.uint8, device=device)


def prefill_q4_k(w: DeviceWeight, X: torch.Tensor, Y: torch.Tensor = None, xh: torch.Tensor = None,
                 stream=None):
    if w.ggml_type != Q4_K:
        raise IHIPArgumentError(_lib.IHIP_ERR_INVALID, "prefill takes a Q4_K weight")
    T = X.shape[0]
    if xh is None:
        xh = prefill_scratch(T, w.inner, X.device)
    if Y is None:
        Y = torch.empty(T, w.outer, dtype=torch.float32, device=X.device)
    check(lib().ihip_prefill_q4_k_dev(_ptr(w.data), _ptr(X, torch.float32, "X"), _ptr(xh), _ptr(Y, torch.float32, "Y"),
                                      T, w.inner, w.outer, _stream(stream)))
    return Y


def prefill_convert(X: torch.Tensor, xh: torch.Tensor = None, stream=None) -> torch.Tensor:
    """The rounding half of prefill_q4_k (ihip_prefill_convert_dev): X (T x
    inner, inner > 512) into xh, which prefill_q4_k_xh then multiplies by any
    number of weights."""
    T, inner = X.shape
    if xh is None:
        xh = prefill_scratch(T, inner, device=X.device)
    check(lib().ihip_prefill_convert_dev(_ptr(X, torch.float32, "X"), _ptr(xh, torch.uint8, "xh"),
                                         T, inner, _stream(stream)))
    return xh


def prefill_q4_k_xh(w: DeviceWeight, xh: torch.Tensor, T: int, Y: torch.Tensor = None,
                    stream=None) -> torch.Tensor:
    """The product half (ihip_prefill_q4_k_xh_dev): Y = W X from rows that
    prefill_convert rounded into xh; bit-identical to prefill_q4_k."""
    if w.ggml_type != Q4_K:
        raise IHIPArgumentError(_lib.IHIP_ERR_INVALID, "prefill takes a Q4_K weight")
    if Y is None:
        Y = torch.empty(T, w.outer, dtype=torch.float32, device=xh.device)
    check(lib().ihip_prefill_q4_k_xh_dev(_ptr(w.data), _ptr(xh, torch.uint8, "xh"),
                                         _ptr(Y, torch.float32, "Y"), T, w.inner, w.outer,
                                         _stream(stream)))
    return Y


def prefill_q4_k_f32(w: DeviceWeight, X: torch.Tensor, Y: torch.Tensor = None, stream=None):
    """The prefill on fp32 operands (ihip_prefill_q4_k_f32_dev): within the row
    bound for any finite X, slower than prefill_q4_k on long rows."""
    if w.ggml_type != Q4_K:
        raise IHIPArgumentError(_lib.IHIP_ERR_INVALID, "prefill takes a Q4_K weight")
    T = X.shape[0]
    if Y is None:
        Y = torch.empty(T, w.outer, dtype=torch.float32, device=X.device)
    check(lib().ihip_prefill_q4_k_f32_dev(_ptr(w.data), _ptr(X, torch.float32, "X"),
                                          _ptr(Y, torch.float32, "Y"), T, w.inner, w.outer,
                                          _stream(stream)))
    return Y


def quantize_row_q8k(x: torch.Tensor, y: torch.Tensor = None, stream=None) -> torch.Tensor:
    """x (fp32, a multiple of 256 elements) -> Q8_K blocks (uint8, 292 bytes
    per 256 elements), as quantize_row_q8_K (src/kernels/quant_kernels.c:166-194)."""
    k = x.numel()
    if y is None:
        y = torch.empty(k // 256 * _lib.Q8_K_BYTES, dtype=torch.uint8, device=x.device)
    check(lib().ihip_quantize_row_q8_k_dev(_ptr(x, torch.float32, "x"), _ptr(y, torch.uint8, "y"), k,
                                           _stream(stream)))
    return y


def gemv_q8k(w: DeviceWeight, q8: torch.Tensor, out: torch.Tensor = None, stream=None) -> torch.Tensor:
    """out = W x with x given as Q8_K blocks: the reference C path's numerics
    (vec_dot_q{4,5,6}_K_q8_K per row, src/kernels/quant_kernels.c:204-521)."""
    if out is None:
        out = torch.empty(w.outer, dtype=torch.float32, device=q8.device)
    check(lib().ihip_gemv_q8k_dev(w.ggml_type, _ptr(w.data), _ptr(q8, torch.uint8, "q8"),
                                  _ptr(out, torch.float32, "out"), w.inner, w.outer, _stream(stream)))
    return out


def gemv_q8k_x(w: DeviceWeight, x: torch.Tensor, out: torch.Tensor = None, q8: torch.Tensor = None,
               stream=None) -> torch.Tensor:
    """out = W x in the reference C path's numerics with x given as fp32 (the
    reference's q{4,5,6}_k_gemv, src/kernels/quant_kernels.c:602-650): x is
    quantized to Q8_K inside the call; q8, when given (inner/256 * 292 bytes),
    receives the blocks."""
    if out is None:
        out = torch.empty(w.outer, dtype=torch.float32, device=x.device)
    check(lib().ihip_gemv_q8k_x_dev(w.ggml_type, _ptr(w.data), _ptr(x, torch.float32, "x"),
                                    _ptr(out, torch.float32, "out"),
                                    None if q8 is None else _ptr(q8, torch.uint8, "q8"),
                                    w.inner, w.outer, _stream(stream)))
    return out


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, out: torch.Tensor = None,
            stream=None) -> torch.Tensor:
    """rmsnorm_cpu! (src/ModelCPU.jl:111-123): x * (1/sqrt(mean(x^2) + eps)) .* w."""
    if out is None:
        out = torch.empty_like(x)
    check(lib().ihip_rmsnorm_dev(_ptr(x, torch.float32, "x"), _ptr(w, torch.float32, "w"), eps,
                                 _ptr(out, torch.float32, "out"), x.numel(), _stream(stream)))
    return out


def ffn_block(wg: DeviceWeight, wu: DeviceWeight, wd: DeviceWeight, norm_w: torch.Tensor,
              eps: float, x: torch.Tensor, h: torch.Tensor = None, stream=None) -> torch.Tensor:
    """The MLP half of a decoder layer (src/ModelCPU.jl:913-920), in place on x:
    x += Wd (silu(Wg n) * (Wu n)), n = rmsnorm(x) .* norm_w."""
    if h is None:
        n = lib().ihip_ffn_block_scratch_floats(wg.ggml_type, wu.ggml_type, wg.inner, wg.outer)
        h = torch.empty(n, dtype=torch.float32, device=x.device)
    check(lib().ihip_ffn_block_dev(wg.ggml_type, _ptr(wg.data), wu.ggml_type, _ptr(wu.data),
                                   wd.ggml_type, _ptr(wd.data), _ptr(norm_w, torch.float32, "norm_w"),
                                   eps, _ptr(x, torch.float32, "x"), _ptr(h, torch.float32, "h"),
                                   wg.inner, wg.outer, _stream(stream)))
    return x


def lm_head_argmax_norm(w: DeviceWeight, norm_w: torch.Tensor, eps: float, x: torch.Tensor,
                        ws: "ArgmaxWorkspace", xn: torch.Tensor = None, logits: torch.Tensor = None,
                        stream=None):
    """Final norm + lm_head + greedy token (src/ModelCPU.jl:1014-1015); the
    token and flags land in ws.token / ws.flags (device)."""
    if xn is None:
        xn = torch.empty_like(x)
    if logits is None and not lib().ihip_lm_head_fused(w.ggml_type, _ptr(w.data), _ptr(xn, torch.float32, "xn"),
                                                       w.inner, w.outer):
        logits = torch.empty(w.outer, dtype=torch.float32, device=x.device)
    check(lib().ihip_lm_head_argmax_norm_dev(
        w.ggml_type, _ptr(w.data), _ptr(norm_w, torch.float32, "norm_w"), eps,
        _ptr(x, torch.float32, "x"), _ptr(xn, torch.float32, "xn"),
        None if logits is None else _ptr(logits, torch.float32, "logits"),
        ws.token.data_ptr(), ws.flags.data_ptr(), w.inner, w.outer, ws.ws.data_ptr(), _stream(stream)))
    return xn
