"""Drop-in mirror of the element-wise fusions of Inferno.jl's
``FusedKernels`` module on the MI355X (device tensors):

* ``fused_mlp_gate_mul_(gate, up)``  -- src/FusedKernels.jl:203-214,
  gate <- gate / (1 + exp(-gate)) * up, in place;
* ``fused_silu_gate_mul_(out, x, gate)`` -- src/FusedKernels.jl:219-230;
* ``gpu_argmax(logits)`` -- src/FusedKernels.jl:271-311 with the checks of
  src/CommonOps.jl:142-163: the lowest index of the maximum, 0-based (the
  Julia binding adds 1), NaN/+Inf raise, all -Inf gives 0.
"""
from __future__ import annotations

import torch

from . import _lib
from ._lib import IHIPArgumentError, check, lib
from .device import ArgmaxWorkspace, _ptr, _stream, argmax

__all__ = ["fused_mlp_gate_mul_", "fused_silu_gate_mul_", "gpu_argmax"]


def fused_mlp_gate_mul_(gate: torch.Tensor, up: torch.Tensor, stream=None):
    if gate.numel() != up.numel():
        raise IHIPArgumentError(_lib.IHIP_ERR_INVALID, "gate and up differ in length")
    check(lib().ihip_fused_mlp_gate_mul_dev(_ptr(gate, torch.float32, "gate"),
                                            _ptr(up, torch.float32, "up"), gate.numel(),
                                            _stream(stream)))
    return gate


def fused_silu_gate_mul_(out: torch.Tensor, x: torch.Tensor, gate: torch.Tensor, stream=None):
    if not (out.numel() == x.numel() == gate.numel()):
        raise IHIPArgumentError(_lib.IHIP_ERR_INVALID, "length mismatch")
    check(lib().ihip_fused_silu_gate_mul_dev(_ptr(out, torch.float32, "out"),
                                             _ptr(x, torch.float32, "x"),
                                             _ptr(gate, torch.float32, "gate"), out.numel(),
                                             _stream(stream)))
    return out


_ws = None


def gpu_argmax(logits: torch.Tensor, ws: ArgmaxWorkspace = None) -> int:
    global _ws
    if logits.numel() == 0:
        raise IHIPArgumentError(_lib.IHIP_ERR_EMPTY, "logits must not be empty")
    if ws is None:
        if _ws is None:
            _ws = ArgmaxWorkspace(logits.device)
        ws = _ws
    argmax(logits, ws)
    return ws.result()
