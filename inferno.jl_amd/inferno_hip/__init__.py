"""inferno_hip -- host side of the MI355X K-quant matvec library.

The compute lives in ``inferno.jl_amd/lib/libinferno_hip.so`` (hand-written
gfx950 HIP kernels behind the C ABI in ``include/inferno_hip.h``).  This
package mirrors the call surface of Inferno.jl's QuantizedKernels,
FusedKernels and Dequant modules over that library:

* ``inferno_hip.QuantizedKernels`` -- q4_k_gemv_ / q5_k_gemv_ / q6_k_gemv_ /
  q8_0_gemv_ on host arrays (src/QuantizedKernels.jl:84-148);
* ``inferno_hip.Dequant``          -- dequantize_q4_k ... (src/Dequant.jl);
* ``inferno_hip.FusedKernels``     -- fused_mlp_gate_mul_, fused_silu_gate_mul_,
  gpu_argmax on device tensors (src/FusedKernels.jl:203-311);
* ``inferno_hip.device``           -- device-resident GEMV, SwiGLU FFN,
  lm_head + argmax and prefill entry points;
* ``inferno_hip.synth``            -- seeded synthetic GGML blocks.

There is no CPU fallback: without the built library the calls raise.
"""
from ._lib import (IHIPArgumentError, IHIPError, LibraryNotBuilt, Q4_K, Q5_K, Q6_K, Q8_0,  # noqa: F401
                   available, lib)
