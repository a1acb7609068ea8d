"""
    InfernoHIP

Drop-in for Inferno.jl's quantized-kernel call surface on the MI355X (gfx950)
library `libinferno_hip.so` (C ABI: `include/inferno_hip.h`).  Three
submodules carry the reference's module names, function names and argument
meaning, so a caller switches by changing what it `using`s:

* `InfernoHIP.QuantizedKernels` -- `src/QuantizedKernels.jl:14-16, 50-177`:
  `quant_kernels_available`, `q4_k_gemv!`, `q5_k_gemv!`, `q6_k_gemv!`,
  `q8_0_gemv!`, `quantize_q8_k!`, `vec_dot_q{4,5,6}_k_q8_k` on host
  `Vector`s, plus `forget_weight!` for the device weight cache;
* `InfernoHIP.Dequant` -- `src/Dequant.jl:5-6, 304-601, 655-693`:
  `dequantize_q8_0`, `dequantize_q4_k`, `dequantize_q5_k`, `dequantize_q6_k`,
  `dequantize_iq4_nl`;
* `InfernoHIP.FusedKernels` -- `src/FusedKernels.jl:14-16, 203-311`:
  `fused_mlp_gate_mul!`, `fused_silu_gate_mul!`, `gpu_argmax!` on DEVICE
  vectors (AMDGPU.jl `ROCArray`s or anything `pointer` maps to device
  memory), plus the fused decode calls the GPU forward makes
  (`ffn_swiglu!`, `ffn_block!`, `lm_head_argmax!`) and the batched prefill
  (`prefill_q4_k!`, `prefill_q4_k_f32!`, and `prefill_convert!` with
  `prefill_q4_k_xh!` for weights that share an input).

Beyond the reference's three modules, `QuantizedKernels` also has
`iq4_nl_gemv!` and the batched prefill `q4_k_gemm!` on host arrays;
`InfernoHIP.Device` has the unfused device calls of a device-resident forward
(`gemv!`, `gemv_add!`, `gemv_norm!`, `dequantize!`, `rmsnorm!`,
`gate_up_swiglu!`, `lm_head_argmax_norm!`, and `register_group` for weights
that share an input); `InfernoHIP.GGUF` loads GGUF tensors straight into device memory
(`open_gguf`, `tensor_count`, `tensor_info`, `upload`, `upload_group`,
`release`, `close_gguf`).

Errors: every library call returns a status; a non-zero status becomes an
`ArgumentError` for bad arguments and NaN/+Inf/empty logits (the reference's
`@assert` / `_validate_logits` cases, `src/CommonOps.jl:142-163`) and an
`ErrorException` otherwise.  With the library missing, or `IHIP_DISABLE` set
(the reference's `INFERNO_NO_QUANT_KERNELS`, `src/QuantizedKernels.jl:26-32`),
`quant_kernels_available()` is `false` and every call throws
`ErrorException("Quantized C kernel not available")`
(`src/QuantizedKernels.jl:86`); there is no silent CPU fallback inside
this module.

Token ids come back 1-based, like the rest of the engine (the library's are
0-based).
"""
module InfernoHIP

const LIBIHIP = get(ENV, "INFERNO_HIP_LIB",
                    joinpath(@__DIR__, "..", "inferno.jl_amd", "lib", "libinferno_hip.so"))
const LIBHIP = "libamdhip64"

const IHIP_ARGMAX_WS_BYTES = 262144
const FLAG_NAN = UInt32(1)
const FLAG_POSINF = UInt32(2)

# GGML type ids (src/GGUF.jl:25-60)
const GGML_Q8_0 = 8
const GGML_Q4_K = 12
const GGML_Q5_K = 13
const GGML_Q6_K = 14
const GGML_IQ4_NL = 20

function available()
    isfile(LIBIHIP) || return false
    return ccall((:ihip_available, LIBIHIP), Cint, ()) == 1
end

function require()
    available() || error("Quantized C kernel not available")
    return nothing
end

function check(rc::Cint)
    rc == 0 && return nothing
    msg = unsafe_string(ccall((:ihip_last_error, LIBIHIP), Cstring, ()))
    # -1 invalid argument, -4 NaN/+Inf logits, -7 empty logits
    (rc == -1 || rc == -4 || rc == -7) && throw(ArgumentError(msg))
    error("libinferno_hip: " * msg)
end

# ---- device memory for the argmax workspace (HIP runtime, no AMDGPU.jl) -----

"""
    ArgmaxWorkspace()

`IHIP_ARGMAX_WS_BYTES` of device memory for the per-workgroup partial maxima
plus the device token and flags.  Calls that share one must not overlap on
the GPU; the memory is freed by the finalizer.
"""
mutable struct ArgmaxWorkspace
    ptr::Ptr{Cvoid}
    function ArgmaxWorkspace()
        p = Ref{Ptr{Cvoid}}(C_NULL)
        rc = ccall((:hipMalloc, LIBHIP), Cint, (Ref{Ptr{Cvoid}}, Csize_t), p, IHIP_ARGMAX_WS_BYTES + 64)
        rc == 0 || error("hipMalloc of the argmax workspace failed ($rc)")
        ws = new(p[])
        finalizer(w -> ccall((:hipFree, LIBHIP), Cint, (Ptr{Cvoid},), w.ptr), ws)
        return ws
    end
end
token_ptr(ws::ArgmaxWorkspace) = Ptr{Int32}(ws.ptr + IHIP_ARGMAX_WS_BYTES)
flags_ptr(ws::ArgmaxWorkspace) = Ptr{UInt32}(ws.ptr + IHIP_ARGMAX_WS_BYTES + 32)

"""Wait for `stream`, read the token and flags back, return the 1-based token."""
function read_token(ws::ArgmaxWorkspace, stream::Ptr{Cvoid})
    ccall((:hipStreamSynchronize, LIBHIP), Cint, (Ptr{Cvoid},), stream) == 0 ||
        error("hipStreamSynchronize failed")
    tok = Ref{Int32}(0)
    fl = Ref{UInt32}(0)
    ccall((:hipMemcpy, LIBHIP), Cint, (Ref{Int32}, Ptr{Int32}, Csize_t, Cint), tok, token_ptr(ws), 4, 2) == 0 ||
        error("hipMemcpy of the token failed")
    ccall((:hipMemcpy, LIBHIP), Cint, (Ref{UInt32}, Ptr{UInt32}, Csize_t, Cint), fl, flags_ptr(ws), 4, 2) == 0 ||
        error("hipMemcpy of the flags failed")
    (fl[] & FLAG_NAN) != 0 && throw(ArgumentError("logits must not contain NaN"))
    (fl[] & FLAG_POSINF) != 0 && throw(ArgumentError("logits must not contain +Inf"))
    return Int(tok[]) + 1
end

# ============================================================================
module QuantizedKernels
# src/QuantizedKernels.jl:14-16
export quant_kernels_available
export q4_k_gemv!, q5_k_gemv!, q6_k_gemv!, q8_0_gemv!
export quantize_q8_k!, vec_dot_q4_k_q8_k, vec_dot_q5_k_q8_k, vec_dot_q6_k_q8_k
export q4_k_gemv_q8k!, q5_k_gemv_q8k!, q6_k_gemv_q8k!, EXACT_C_NUMERICS
export q4_k_gemm!, iq4_nl_gemv!

import ..InfernoHIP: LIBIHIP, check, require, available

"""src/QuantizedKernels.jl:50-51: the kernels can run (a gfx950 device, IHIP_DISABLE unset)."""
quant_kernels_available() = available()

function check_dims(out, weight_data, x, inner_dim, outer_dim, elems, bytes)
    inner_dim > 0 && outer_dim > 0 && inner_dim % elems == 0 ||
        throw(ArgumentError("inner_dim=$inner_dim must be a positive multiple of $elems"))
    length(out) >= outer_dim || throw(ArgumentError("out is shorter than outer_dim"))
    length(x) >= inner_dim || throw(ArgumentError("x is shorter than inner_dim"))
    length(weight_data) >= outer_dim * (inner_dim ÷ elems) * bytes ||
        throw(ArgumentError("weight_data is too short for $outer_dim x $inner_dim"))
    return nothing
end

"""
    EXACT_C_NUMERICS[] = true

Routes `q4_k_gemv!`, `q5_k_gemv!` and `q6_k_gemv!` through the int8-activation
kernels (`q*_k_gemv_q8k!`): x quantized to Q8_K per 256 values and integer
dot products, bit-identical to the reference's C kernels
(src/kernels/quant_kernels.c:602-650), which is what the reference's
`q*_k_gemv!` computes.  Default `false`: fp32 activations, within
1e-4 ||w_row|| ||x|| of the exact sum.  Initialised from the environment
variable IHIP_EXACT_C_NUMERICS=1.
"""
const EXACT_C_NUMERICS = Ref(get(ENV, "IHIP_EXACT_C_NUMERICS", "0") == "1")

"""
    q4_k_gemv_q8k!(out, weight_data, x, inner_dim, outer_dim)

src/kernels/quant_kernels.c:602-614 on the GPU, bit-identical: x quantized to
Q8_K (quantize_row_q8_K), then the integer Q4_K x Q8_K dot products.
"""
function q4_k_gemv_q8k!(out::Vector{Float32}, weight_data::Vector{UInt8},
                        x::Vector{Float32}, inner_dim::Int, outer_dim::Int)
    require()
    check_dims(out, weight_data, x, inner_dim, outer_dim, 256, 144)
    check(ccall((:ihip_q4_k_gemv_q8k, LIBIHIP), Cint,
                (Ptr{UInt8}, Ptr{Float32}, Ptr{Float32}, Ptr{Cvoid}, Cint, Cint),
                weight_data, x, out, C_NULL, inner_dim, outer_dim))
    return out
end

"""src/kernels/quant_kernels.c:620-632 on the GPU, bit-identical (Q5_K)."""
function q5_k_gemv_q8k!(out::Vector{Float32}, weight_data::Vector{UInt8},
                        x::Vector{Float32}, inner_dim::Int, outer_dim::Int)
    require()
    check_dims(out, weight_data, x, inner_dim, outer_dim, 256, 176)
    check(ccall((:ihip_q5_k_gemv_q8k, LIBIHIP), Cint,
                (Ptr{UInt8}, Ptr{Float32}, Ptr{Float32}, Ptr{Cvoid}, Cint, Cint),
                weight_data, x, out, C_NULL, inner_dim, outer_dim))
    return out
end

"""src/kernels/quant_kernels.c:638-650 on the GPU, bit-identical (Q6_K)."""
function q6_k_gemv_q8k!(out::Vector{Float32}, weight_data::Vector{UInt8},
                        x::Vector{Float32}, inner_dim::Int, outer_dim::Int)
    require()
    check_dims(out, weight_data, x, inner_dim, outer_dim, 256, 210)
    check(ccall((:ihip_q6_k_gemv_q8k, LIBIHIP), Cint,
                (Ptr{UInt8}, Ptr{Float32}, Ptr{Float32}, Ptr{Cvoid}, Cint, Cint),
                weight_data, x, out, C_NULL, inner_dim, outer_dim))
    return out
end

"""
    q4_k_gemv!(out, weight_data, x, inner_dim, outer_dim)

src/QuantizedKernels.jl:84-96 on the GPU: `out = W x` for the Q4_K blocks of an
`outer_dim x inner_dim` matrix, fp32 activations (within 1e-4 ||w_row|| ||x||
of the exact sum), or the reference C numerics when `EXACT_C_NUMERICS[]`.
The weight is uploaded on first use and cached.
"""
function q4_k_gemv!(out::Vector{Float32}, weight_data::Vector{UInt8},
                    x::Vector{Float32}, inner_dim::Int, outer_dim::Int)
    EXACT_C_NUMERICS[] && return q4_k_gemv_q8k!(out, weight_data, x, inner_dim, outer_dim)
    require()
    check_dims(out, weight_data, x, inner_dim, outer_dim, 256, 144)
    check(ccall((:ihip_q4_k_gemv, LIBIHIP), Cint,
                (Ptr{UInt8}, Ptr{Float32}, Ptr{Float32}, Ptr{Cvoid}, Cint, Cint),
                weight_data, x, out, C_NULL, inner_dim, outer_dim))
    return out
end

"""src/QuantizedKernels.jl:103-115 on the GPU (Q5_K; `EXACT_C_NUMERICS` as q4_k_gemv!)."""
function q5_k_gemv!(out::Vector{Float32}, weight_data::Vector{UInt8},
                    x::Vector{Float32}, inner_dim::Int, outer_dim::Int)
    EXACT_C_NUMERICS[] && return q5_k_gemv_q8k!(out, weight_data, x, inner_dim, outer_dim)
    require()
    check_dims(out, weight_data, x, inner_dim, outer_dim, 256, 176)
    check(ccall((:ihip_q5_k_gemv, LIBIHIP), Cint,
                (Ptr{UInt8}, Ptr{Float32}, Ptr{Float32}, Ptr{Cvoid}, Cint, Cint),
                weight_data, x, out, C_NULL, inner_dim, outer_dim))
    return out
end

"""src/QuantizedKernels.jl:122-134 on the GPU (Q6_K; `EXACT_C_NUMERICS` as q4_k_gemv!)."""
function q6_k_gemv!(out::Vector{Float32}, weight_data::Vector{UInt8},
                    x::Vector{Float32}, inner_dim::Int, outer_dim::Int)
    EXACT_C_NUMERICS[] && return q6_k_gemv_q8k!(out, weight_data, x, inner_dim, outer_dim)
    require()
    check_dims(out, weight_data, x, inner_dim, outer_dim, 256, 210)
    check(ccall((:ihip_q6_k_gemv, LIBIHIP), Cint,
                (Ptr{UInt8}, Ptr{Float32}, Ptr{Float32}, Ptr{Cvoid}, Cint, Cint),
                weight_data, x, out, C_NULL, inner_dim, outer_dim))
    return out
end

"""src/QuantizedKernels.jl:141-150 on the GPU (Q8_0, fp32 x)."""
function q8_0_gemv!(out::Vector{Float32}, weight_data::Vector{UInt8},
                    x::Vector{Float32}, inner_dim::Int, outer_dim::Int)
    require()
    check_dims(out, weight_data, x, inner_dim, outer_dim, 32, 34)
    check(ccall((:ihip_q8_0_gemv, LIBIHIP), Cint,
                (Ptr{UInt8}, Ptr{Float32}, Ptr{Float32}, Cint, Cint),
                weight_data, x, out, inner_dim, outer_dim))
    return out
end

"""
    iq4_nl_gemv!(out, weight_data, x, inner_dim, outer_dim)

mul_quant_mat_vec(::IQ4NL_Matrix) (src/ModelCPU.jl:381-408) on the GPU: 18-byte
blocks of 32 (fp16 d, 16 bytes of 4-bit indices into the IQ4_NL grid), fp32 x,
within 1e-4 ||w_row|| ||x|| of the exact sum.
"""
function iq4_nl_gemv!(out::Vector{Float32}, weight_data::Vector{UInt8},
                      x::Vector{Float32}, inner_dim::Int, outer_dim::Int)
    require()
    check_dims(out, weight_data, x, inner_dim, outer_dim, 32, 18)
    check(ccall((:ihip_iq4_nl_gemv, LIBIHIP), Cint,
                (Ptr{UInt8}, Ptr{Float32}, Ptr{Float32}, Cint, Cint),
                weight_data, x, out, inner_dim, outer_dim))
    return out
end

"""
    q4_k_gemm!(Y, weight_data, X, inner_dim, outer_dim)

The prefill's per-token loop (src/ModelCPU.jl:1001-1017: `q4_k_gemv!` of every
token column) as one batched product on the matrix cores:
`Y[:, t] = W X[:, t]` for the `T = size(X, 2)` token columns.  Julia's
column-major `X` (inner_dim x T) and `Y` (outer_dim x T) are the library's
row-major T x inner and T x outer.  Within 1e-4 ||w_row|| ||x_t|| of the
exact sum for any finite X (ihip_prefill_q4_k); the weight is uploaded on
first use and cached, like `q4_k_gemv!`'s.
"""
function q4_k_gemm!(Y::Matrix{Float32}, weight_data::Vector{UInt8}, X::Matrix{Float32},
                    inner_dim::Int, outer_dim::Int)
    require()
    T = size(X, 2)
    T > 0 || throw(ArgumentError("X has no token columns"))
    size(X, 1) == inner_dim || throw(DimensionMismatch("X has $(size(X, 1)) rows, inner_dim is $inner_dim"))
    size(Y) == (outer_dim, T) || throw(DimensionMismatch("Y must be $outer_dim x $T"))
    check_dims(view(Y, :, 1), weight_data, view(X, :, 1), inner_dim, outer_dim, 256, 144)
    check(ccall((:ihip_prefill_q4_k, LIBIHIP), Cint,
                (Ptr{UInt8}, Ptr{Float32}, Ptr{Float32}, Cint, Cint, Cint),
                weight_data, X, Y, T, inner_dim, outer_dim))
    return Y
end

"""
    quantize_q8_k!(q8_buf, x, inner_dim)

src/QuantizedKernels.jl:153-158 with the reference's argument order, passed to
the C function in ITS order (x, y, k): the reference's ccall hands
`quantize_row_q8_K` the two pointers swapped and a 32-bit count.
"""
function quantize_q8_k!(q8_buf::Vector{UInt8}, x::Vector{Float32}, inner_dim::Int)
    require()
    inner_dim > 0 && inner_dim % 256 == 0 ||
        throw(ArgumentError("inner_dim=$inner_dim must be a positive multiple of 256"))
    length(q8_buf) >= (inner_dim ÷ 256) * 292 || throw(ArgumentError("q8_buf is too short"))
    check(ccall((:ihip_quantize_row_q8_k, LIBIHIP), Cint,
                (Ptr{Float32}, Ptr{UInt8}, Int64), x, q8_buf, inner_dim))
    return q8_buf
end

"""src/QuantizedKernels.jl:161-165: one Q4_K row of nb blocks against nb Q8_K blocks."""
function vec_dot_q4_k_q8_k(weight_ptr::Ptr{UInt8}, q8_ptr::Ptr{UInt8}, nb::Cint)
    require()
    s = Ref{Cfloat}(0)
    check(ccall((:ihip_vec_dot_q4_k_q8_k, LIBIHIP), Cint,
                (Ptr{UInt8}, Ptr{UInt8}, Cint, Ref{Cfloat}), weight_ptr, q8_ptr, nb, s))
    return s[]
end

"""src/QuantizedKernels.jl:168-172 (Q5_K)."""
function vec_dot_q5_k_q8_k(weight_ptr::Ptr{UInt8}, q8_ptr::Ptr{UInt8}, nb::Cint)
    require()
    s = Ref{Cfloat}(0)
    check(ccall((:ihip_vec_dot_q5_k_q8_k, LIBIHIP), Cint,
                (Ptr{UInt8}, Ptr{UInt8}, Cint, Ref{Cfloat}), weight_ptr, q8_ptr, nb, s))
    return s[]
end

"""src/QuantizedKernels.jl:175-179 (Q6_K)."""
function vec_dot_q6_k_q8_k(weight_ptr::Ptr{UInt8}, q8_ptr::Ptr{UInt8}, nb::Cint)
    require()
    s = Ref{Cfloat}(0)
    check(ccall((:ihip_vec_dot_q6_k_q8_k, LIBIHIP), Cint,
                (Ptr{UInt8}, Ptr{UInt8}, Cint, Ref{Cfloat}), weight_ptr, q8_ptr, nb, s))
    return s[]
end

"""
    forget_weight!(weight_data)

Drop the cached device copy of a host weight (a `Q*_Matrix`'s `data`).  The
cache already re-uploads a buffer whose sampled content changed; call this
when a weight is freed, or after an in-place rewrite that might leave every
sampled window unchanged.  Attach it as a finalizer to keep-quantized
matrices (src/LoaderCPU.jl:134-163).
"""
function forget_weight!(weight_data::Vector{UInt8})
    check(ccall((:ihip_weight_forget, LIBIHIP), Cint, (Ptr{UInt8},), weight_data))
    return nothing
end

end # module QuantizedKernels

# ============================================================================
module Dequant
# src/Dequant.jl:5-6 (the K-quant, Q8_0 and IQ4_NL exports)
export dequantize_q8_0, dequantize_q4_k, dequantize_q5_k, dequantize_q6_k, dequantize_iq4_nl

import ..InfernoHIP: LIBIHIP, check, require, GGML_Q8_0, GGML_Q4_K, GGML_Q5_K, GGML_Q6_K, GGML_IQ4_NL

function dequant(t::Int, data::Vector{UInt8}, n::Int, elems::Int, bytes::Int)
    require()
    n >= 0 && n % elems == 0 || throw(ArgumentError("n=$n is not a multiple of $elems"))
    length(data) >= (n ÷ elems) * bytes || throw(ArgumentError("data is too short for $n elements"))
    out = Vector{Float32}(undef, n)
    check(ccall((:ihip_dequantize, LIBIHIP), Cint,
                (Cint, Ptr{UInt8}, Ptr{Float32}, Int64), t, data, out, n))
    return out
end

"""src/Dequant.jl:304-321, bit-exact."""
dequantize_q8_0(data::Vector{UInt8}, n::Int) = dequant(GGML_Q8_0, data, n, 32, 34)
"""src/Dequant.jl:325-375, bit-exact."""
dequantize_q4_k(data::Vector{UInt8}, n::Int) = dequant(GGML_Q4_K, data, n, 256, 144)
"""src/Dequant.jl:379-441, bit-exact."""
dequantize_q5_k(data::Vector{UInt8}, n::Int) = dequant(GGML_Q5_K, data, n, 256, 176)
"""src/Dequant.jl:558-601, bit-exact."""
dequantize_q6_k(data::Vector{UInt8}, n::Int) = dequant(GGML_Q6_K, data, n, 256, 210)
"""src/Dequant.jl:655-693, bit-exact."""
dequantize_iq4_nl(data::Vector{UInt8}, n::Int) = dequant(GGML_IQ4_NL, data, n, 32, 18)

end # module Dequant

# ============================================================================
module FusedKernels
# src/FusedKernels.jl:14-16 (the element-wise fusions and the greedy argmax of
# the decode path) and the fused decode calls of a device-resident forward.
export fused_mlp_gate_mul!, fused_silu_gate_mul!, gpu_argmax!
export ffn_swiglu!, ffn_block!, lm_head_argmax!
export prefill_scratch_bytes, prefill_q4_k!, prefill_q4_k_f32!, prefill_convert!, prefill_q4_k_xh!

import ..InfernoHIP: LIBIHIP, check, require, ArgmaxWorkspace, token_ptr, flags_ptr, read_token

"""
    fused_mlp_gate_mul!(gate, up; stream = C_NULL)

src/FusedKernels.jl:203-214: `gate .= gate / (1 + exp(-gate)) .* up` in place,
on device vectors, asynchronous on `stream` (a hipStream_t).
"""
function fused_mlp_gate_mul!(gate::AbstractVector{Float32}, up::AbstractVector{Float32};
                             stream::Ptr{Cvoid} = C_NULL)
    require()
    n = length(gate)
    length(up) == n || throw(DimensionMismatch("gate and up differ in length"))
    n == 0 && return gate
    check(ccall((:ihip_fused_mlp_gate_mul_dev, LIBIHIP), Cint,
                (Ptr{Float32}, Ptr{Float32}, Int64, Ptr{Cvoid}), gate, up, n, stream))
    return gate
end

"""
    fused_silu_gate_mul!(out, x, gate; stream = C_NULL)

src/FusedKernels.jl:219-230: `out .= x / (1 + exp(-x)) .* gate`.
"""
function fused_silu_gate_mul!(out::AbstractVector{Float32}, x::AbstractVector{Float32},
                              gate::AbstractVector{Float32}; stream::Ptr{Cvoid} = C_NULL)
    require()
    n = length(out)
    length(x) == n && length(gate) == n || throw(DimensionMismatch("lengths differ"))
    n == 0 && return out
    check(ccall((:ihip_fused_silu_gate_mul_dev, LIBIHIP), Cint,
                (Ptr{Float32}, Ptr{Float32}, Ptr{Float32}, Int64, Ptr{Cvoid}), out, x, gate, n, stream))
    return out
end

"""
    gpu_argmax!(logits; ws = ArgmaxWorkspace(), stream = C_NULL) -> Int

src/FusedKernels.jl:271-311: the 1-based index of the largest logit, the
lowest index among equal maxima, reduced on the device (no per-chunk host
pass).  Empty logits return 1 as the reference does; NaN or +Inf logits
throw ArgumentError (`_validate_logits`, src/CommonOps.jl:142-163).
"""
function gpu_argmax!(logits::AbstractVector{Float32}; ws::ArgmaxWorkspace = ArgmaxWorkspace(),
                     stream::Ptr{Cvoid} = C_NULL)
    require()
    n = length(logits)
    n == 0 && return 1
    check(ccall((:ihip_argmax_dev, LIBIHIP), Cint,
                (Ptr{Float32}, Int64, Ptr{Int32}, Ptr{UInt32}, Ptr{Cvoid}, Ptr{Cvoid}),
                logits, n, token_ptr(ws), flags_ptr(ws), ws.ptr, stream))
    return read_token(ws, stream)
end

"""
    ffn_swiglu!(y, h, gate_type, wg, up_type, wu, down_type, wd, x, hidden, inter; stream)

mlp_forward (src/ModelCPU.jl:482-508) on device memory: `h = silu(Wg x) .* (Wu x)`,
`y = Wd h`.  wg, wu, wd are device weight pointers (16-byte aligned GGML
blocks, e.g. from ihip_gguf_upload + ihip_weight_device_ptr); h holds
`inter` floats.
"""
function ffn_swiglu!(y::AbstractVector{Float32}, h::AbstractVector{Float32}, gate_type::Integer,
                     wg::Ptr{Cvoid}, up_type::Integer, wu::Ptr{Cvoid}, down_type::Integer,
                     wd::Ptr{Cvoid}, x::AbstractVector{Float32}, hidden::Integer, inter::Integer;
                     stream::Ptr{Cvoid} = C_NULL)
    require()
    length(h) >= inter && length(y) >= hidden && length(x) >= hidden ||
        throw(DimensionMismatch("x, h or y too short"))
    check(ccall((:ihip_ffn_swiglu_dev, LIBIHIP), Cint,
                (Cint, Ptr{Cvoid}, Cint, Ptr{Cvoid}, Cint, Ptr{Cvoid}, Ptr{Float32}, Ptr{Float32},
                 Ptr{Float32}, Cint, Cint, Ptr{Cvoid}),
                gate_type, wg, up_type, wu, down_type, wd, x, h, y, hidden, inter, stream))
    return y
end

"""
    ffn_block!(x, h, gate_type, wg, up_type, wu, down_type, wd, norm_w, eps, hidden, inter; stream)

The MLP half of a decoder layer (src/ModelCPU.jl:913-920) in place on x:
`x += Wd (silu(Wg n) .* (Wu n))`, `n = rmsnorm_cpu!(x) .* norm_w`.  h is caller
scratch of `ihip_ffn_block_scratch_floats` floats.
"""
function ffn_block!(x::AbstractVector{Float32}, h::AbstractVector{Float32}, gate_type::Integer,
                    wg::Ptr{Cvoid}, up_type::Integer, wu::Ptr{Cvoid}, down_type::Integer,
                    wd::Ptr{Cvoid}, norm_w::AbstractVector{Float32}, eps::Real, hidden::Integer,
                    inter::Integer; stream::Ptr{Cvoid} = C_NULL)
    require()
    need = ccall((:ihip_ffn_block_scratch_floats, LIBIHIP), Csize_t, (Cint, Cint, Cint, Cint),
                 gate_type, up_type, hidden, inter)
    length(h) >= need || throw(DimensionMismatch("h needs $need floats"))
    check(ccall((:ihip_ffn_block_dev, LIBIHIP), Cint,
                (Cint, Ptr{Cvoid}, Cint, Ptr{Cvoid}, Cint, Ptr{Cvoid}, Ptr{Float32}, Cfloat,
                 Ptr{Float32}, Ptr{Float32}, Cint, Cint, Ptr{Cvoid}),
                gate_type, wg, up_type, wu, down_type, wd, norm_w, Float32(eps), x, h, hidden,
                inter, stream))
    return x
end

"""
    lm_head_argmax!(logits, w_type, w, x, hidden, vocab; ws, stream) -> Int

lm_head_project! + greedy token (src/ModelCPU.jl:1091-1123, src/CommonOps.jl:142-163)
with the argmax fused into the GEMV where the library fuses it: the 1-based
token.  `logits` (device, vocab floats) may be `nothing` when
`ihip_lm_head_fused` says so.
"""
function lm_head_argmax!(logits::Union{Nothing,AbstractVector{Float32}}, w_type::Integer,
                         w::Ptr{Cvoid}, x::AbstractVector{Float32}, hidden::Integer, vocab::Integer;
                         ws::ArgmaxWorkspace = ArgmaxWorkspace(), stream::Ptr{Cvoid} = C_NULL)
    require()
    lp = logits === nothing ? Ptr{Float32}(C_NULL) : Base.unsafe_convert(Ptr{Float32}, logits)
    check(ccall((:ihip_lm_head_argmax_dev, LIBIHIP), Cint,
                (Cint, Ptr{Cvoid}, Ptr{Float32}, Ptr{Float32}, Ptr{Int32}, Ptr{UInt32}, Cint, Cint,
                 Ptr{Cvoid}, Ptr{Cvoid}),
                w_type, w, x, lp, token_ptr(ws), flags_ptr(ws), hidden, vocab, ws.ptr, stream))
    return read_token(ws, stream)
end

"""
    prefill_scratch_bytes(T, inner) -> Int

Bytes of device scratch `prefill_q4_k!` takes for T tokens of `inner`
columns (the rounded activations, one scale per token, the partial sums of a
split over K); independent of the weight's row count.
"""
prefill_scratch_bytes(T::Integer, inner::Integer) =
    Int(ccall((:ihip_prefill_scratch_bytes, LIBIHIP), Csize_t, (Cint, Cint), T, inner))

"""
    prefill_q4_k!(Y, w, X, xh, T, inner, outer; stream)

The prefill's per-token loop (src/ModelCPU.jl:1001-1017) on device memory:
`Y[:, t] = W X[:, t]` for T token columns (X: inner x T, Y: outer x T,
column-major), W a device Q4_K weight pointer.  Rows of more than 512 columns
multiply fp16 operands (each token column scaled by a power of two first):
any finite X, every dequantized weight below 65504 in magnitude.  `xh` is
scratch of `prefill_scratch_bytes(T, inner)` bytes; calls sharing it must not
overlap on the GPU.  Pointers 16-byte aligned.
"""
function prefill_q4_k!(Y::AbstractMatrix{Float32}, w::Ptr{Cvoid}, X::AbstractMatrix{Float32},
                       xh::Ptr{Cvoid}, T::Integer, inner::Integer, outer::Integer;
                       stream::Ptr{Cvoid} = C_NULL)
    require()
    size(X, 1) == inner && size(X, 2) >= T && size(Y, 1) == outer && size(Y, 2) >= T ||
        throw(DimensionMismatch("X must be $inner x $T and Y $outer x $T"))
    check(ccall((:ihip_prefill_q4_k_dev, LIBIHIP), Cint,
                (Ptr{Cvoid}, Ptr{Float32}, Ptr{Cvoid}, Ptr{Float32}, Cint, Cint, Cint, Ptr{Cvoid}),
                w, X, xh, Y, T, inner, outer, stream))
    return Y
end

"""
    prefill_convert!(xh, X, T, inner; stream)

The rounding half of `prefill_q4_k!` (rows of more than 512 columns): X
(inner x T) into the scratch `xh`, which `prefill_q4_k_xh!` then multiplies by
every weight that shares this input -- wq, wk and wv
(src/ModelCPU.jl:789-791), gate and up (:490, 498).
"""
function prefill_convert!(xh::Ptr{Cvoid}, X::AbstractMatrix{Float32}, T::Integer, inner::Integer;
                          stream::Ptr{Cvoid} = C_NULL)
    require()
    size(X, 1) == inner && size(X, 2) >= T || throw(DimensionMismatch("X must be $inner x $T"))
    check(ccall((:ihip_prefill_convert_dev, LIBIHIP), Cint,
                (Ptr{Float32}, Ptr{Cvoid}, Cint, Cint, Ptr{Cvoid}), X, xh, T, inner, stream))
    return xh
end

"""
    prefill_q4_k_xh!(Y, w, xh, T, inner, outer; stream)

The product half: `Y[:, t] = W X[:, t]` from the rows `prefill_convert!`
rounded into `xh`, bit-identical to `prefill_q4_k!`; any number of products
may follow one conversion.
"""
function prefill_q4_k_xh!(Y::AbstractMatrix{Float32}, w::Ptr{Cvoid}, xh::Ptr{Cvoid}, T::Integer,
                          inner::Integer, outer::Integer; stream::Ptr{Cvoid} = C_NULL)
    require()
    size(Y, 1) == outer && size(Y, 2) >= T || throw(DimensionMismatch("Y must be $outer x $T"))
    check(ccall((:ihip_prefill_q4_k_xh_dev, LIBIHIP), Cint,
                (Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Float32}, Cint, Cint, Cint, Ptr{Cvoid}),
                w, xh, Y, T, inner, outer, stream))
    return Y
end

"""
    prefill_q4_k_f32!(Y, w, X, T, inner, outer; stream)

`prefill_q4_k!` on fp32 operands at every row length (no scratch): within
1e-4 ||w_row|| ||x_t|| for any finite X and any weight, several times slower
on long rows.
"""
function prefill_q4_k_f32!(Y::AbstractMatrix{Float32}, w::Ptr{Cvoid}, X::AbstractMatrix{Float32},
                           T::Integer, inner::Integer, outer::Integer; stream::Ptr{Cvoid} = C_NULL)
    require()
    size(X, 1) == inner && size(X, 2) >= T && size(Y, 1) == outer && size(Y, 2) >= T ||
        throw(DimensionMismatch("X must be $inner x $T and Y $outer x $T"))
    check(ccall((:ihip_prefill_q4_k_f32_dev, LIBIHIP), Cint,
                (Ptr{Cvoid}, Ptr{Float32}, Ptr{Float32}, Cint, Cint, Cint, Ptr{Cvoid}),
                w, X, Y, T, inner, outer, stream))
    return Y
end

end # module FusedKernels

# ============================================================================
module Device
# The unfused device calls of a device-resident forward (the role
# src/Qwen35GPU.jl plays for oneAPI): mul_quant_mat_vec, dequantization,
# rmsnorm_cpu!, the gate/up pair and the final norm + lm_head on device
# vectors, asynchronous on `stream` (a hipStream_t).  Weights are device
# pointers to GGML blocks (e.g. `GGUF.upload`).
export gemv!, gemv_add!, gemv_norm!, dequantize!, rmsnorm!, gate_up_swiglu!, lm_head_argmax_norm!
export register_group, weight_bytes

import ..InfernoHIP: LIBIHIP, check, require, ArgmaxWorkspace, token_ptr, flags_ptr, read_token

"""
    gemv!(out, w_type, w, x, inner, outer; stream)

mul_quant_mat_vec (src/ModelCPU.jl:285-408) on device memory for GGML type
`w_type` (Q4_K, Q5_K, Q6_K, Q8_0, IQ4_NL): `out = W x`, within
1e-4 ||w_row|| ||x|| of the exact sum.
"""
function gemv!(out::AbstractVector{Float32}, w_type::Integer, w::Ptr{Cvoid},
               x::AbstractVector{Float32}, inner::Integer, outer::Integer; stream::Ptr{Cvoid} = C_NULL)
    require()
    length(out) >= outer && length(x) >= inner || throw(DimensionMismatch("x or out too short"))
    check(ccall((:ihip_gemv_dev, LIBIHIP), Cint,
                (Cint, Ptr{Cvoid}, Ptr{Float32}, Ptr{Float32}, Cint, Cint, Ptr{Cvoid}),
                w_type, w, x, out, inner, outer, stream))
    return out
end

"""
    gemv_add!(out, w_type, w, x, resid, inner, outer; stream)

`out = resid + W x` in one launch: the attention's output projection
(src/ModelCPU.jl:885) with the layer's `x .+= residual` (:909) folded into the
GEMV's epilogue.  `resid` may be `out` (in place); x may not overlap out.
"""
function gemv_add!(out::AbstractVector{Float32}, w_type::Integer, w::Ptr{Cvoid},
                   x::AbstractVector{Float32}, resid::AbstractVector{Float32}, inner::Integer,
                   outer::Integer; stream::Ptr{Cvoid} = C_NULL)
    require()
    length(out) >= outer && length(resid) >= outer && length(x) >= inner ||
        throw(DimensionMismatch("x, resid or out too short"))
    check(ccall((:ihip_gemv_add_dev, LIBIHIP), Cint,
                (Cint, Ptr{Cvoid}, Ptr{Float32}, Ptr{Float32}, Ptr{Float32}, Cint, Cint, Ptr{Cvoid}),
                w_type, w, x, resid, out, inner, outer, stream))
    return out
end

"""
    gemv_norm!(out, w_type, w, norm_w, eps, x, xn, inner, outer; stream)

`out = W (rmsnorm(x) .* norm_w)`: a layer's input norm (src/ModelCPU.jl:903)
folded into the GEMV that consumes it, e.g. a `register_group` of wq, wk and
wv (:789-791).  One launch for aligned Q4_K / Q5_K rows of at most 4096
columns; otherwise `xn` (inner floats, may be
`nothing` where the norm folds) receives the normed x first.
"""
function gemv_norm!(out::AbstractVector{Float32}, w_type::Integer, w::Ptr{Cvoid},
                    norm_w::AbstractVector{Float32}, eps::Real, x::AbstractVector{Float32},
                    xn::Union{Nothing,AbstractVector{Float32}}, inner::Integer, outer::Integer;
                    stream::Ptr{Cvoid} = C_NULL)
    require()
    length(out) >= outer && length(x) >= inner && length(norm_w) >= inner ||
        throw(DimensionMismatch("x, norm_w or out too short"))
    xp = xn === nothing ? Ptr{Float32}(C_NULL) : Base.unsafe_convert(Ptr{Float32}, xn)
    check(ccall((:ihip_gemv_norm_dev, LIBIHIP), Cint,
                (Cint, Ptr{Cvoid}, Ptr{Float32}, Cfloat, Ptr{Float32}, Ptr{Float32}, Ptr{Float32}, Cint,
                 Cint, Ptr{Cvoid}),
                w_type, w, norm_w, Float32(eps), x, xp, out, inner, outer, stream))
    return out
end

"""
    dequantize!(dst, w_type, src, n; stream)

The Dequant.jl routines (src/Dequant.jl:304-693) on device memory: n weights
of GGML type `w_type` to fp32, bit-exact.
"""
function dequantize!(dst::AbstractVector{Float32}, w_type::Integer, src::Ptr{Cvoid}, n::Integer;
                     stream::Ptr{Cvoid} = C_NULL)
    require()
    length(dst) >= n || throw(DimensionMismatch("dst holds fewer than $n floats"))
    check(ccall((:ihip_dequantize_dev, LIBIHIP), Cint,
                (Cint, Ptr{Cvoid}, Ptr{Float32}, Int64, Ptr{Cvoid}), w_type, src, dst, n, stream))
    return dst
end

"""
    rmsnorm!(out, x, w, eps; stream)

rmsnorm_cpu! (src/ModelCPU.jl:111-123): `out = x * (1/sqrt(mean(x^2) + eps)) .* w`
(out may be x).
"""
function rmsnorm!(out::AbstractVector{Float32}, x::AbstractVector{Float32},
                  w::AbstractVector{Float32}, eps::Real; stream::Ptr{Cvoid} = C_NULL)
    require()
    n = length(x)
    length(out) >= n && length(w) >= n || throw(DimensionMismatch("out or w too short"))
    check(ccall((:ihip_rmsnorm_dev, LIBIHIP), Cint,
                (Ptr{Float32}, Ptr{Float32}, Cfloat, Ptr{Float32}, Cint, Ptr{Cvoid}),
                x, w, Float32(eps), out, n, stream))
    return out
end

"""
    gate_up_swiglu!(h, gate_type, wg, up_type, wu, x, hidden, inter; stream)

The first half of mlp_forward (src/ModelCPU.jl:482-505):
`h = silu(Wg x) .* (Wu x)`, one pass over both weights for a matching
16-byte aligned Q4_K or Q5_K pair.
"""
function gate_up_swiglu!(h::AbstractVector{Float32}, gate_type::Integer, wg::Ptr{Cvoid},
                         up_type::Integer, wu::Ptr{Cvoid}, x::AbstractVector{Float32},
                         hidden::Integer, inter::Integer; stream::Ptr{Cvoid} = C_NULL)
    require()
    length(h) >= inter && length(x) >= hidden || throw(DimensionMismatch("x or h too short"))
    check(ccall((:ihip_gate_up_swiglu_dev, LIBIHIP), Cint,
                (Cint, Ptr{Cvoid}, Cint, Ptr{Cvoid}, Ptr{Float32}, Ptr{Float32}, Cint, Cint, Ptr{Cvoid}),
                gate_type, wg, up_type, wu, x, h, hidden, inter, stream))
    return h
end

"""
    lm_head_argmax_norm!(xn, logits, w_type, w, norm_w, eps, x, hidden, vocab; ws, stream) -> Int

The last step of the forward (src/ModelCPU.jl:1014-1015, src/CommonOps.jl:142-163):
`xn = rmsnorm(x) .* norm_w`, then the lm_head and the greedy token, 1-based.
`logits` may be `nothing` where the argmax is fused into the GEMV.
"""
function lm_head_argmax_norm!(xn::AbstractVector{Float32}, logits::Union{Nothing,AbstractVector{Float32}},
                              w_type::Integer, w::Ptr{Cvoid}, norm_w::AbstractVector{Float32},
                              eps::Real, x::AbstractVector{Float32}, hidden::Integer, vocab::Integer;
                              ws::ArgmaxWorkspace = ArgmaxWorkspace(), stream::Ptr{Cvoid} = C_NULL)
    require()
    lp = logits === nothing ? Ptr{Float32}(C_NULL) : Base.unsafe_convert(Ptr{Float32}, logits)
    check(ccall((:ihip_lm_head_argmax_norm_dev, LIBIHIP), Cint,
                (Cint, Ptr{Cvoid}, Ptr{Float32}, Cfloat, Ptr{Float32}, Ptr{Float32}, Ptr{Float32},
                 Ptr{Int32}, Ptr{UInt32}, Cint, Cint, Ptr{Cvoid}, Ptr{Cvoid}),
                w_type, w, norm_w, Float32(eps), x, xn, lp, token_ptr(ws), flags_ptr(ws), hidden,
                vocab, ws.ptr, stream))
    return read_token(ws, stream)
end

"""`weight_bytes(w_type, inner, outer) -> Int`: bytes of an outer x inner weight."""
weight_bytes(w_type::Integer, inner::Integer, outer::Integer) =
    Int(ccall((:ihip_weight_bytes, LIBIHIP), Csize_t, (Cint, Cint, Cint), w_type, inner, outer))

"""
    register_group(datas, w_type, inner, outers) -> (handle, device_pointer)

Host weights that share an input -- wq, wk and wv (src/ModelCPU.jl:789-791)
-- uploaded back to back as one weight of `sum(outers)` rows: `gemv!` over it
with `outer = sum(outers)` computes every member's outputs in one launch
(member i's rows follow the rows of the members before it, and its blocks
start `weight_bytes(w_type, inner, rows before it)` into the group).
Free it with `GGUF.release(handle)`.
"""
function register_group(datas::Vector{Vector{UInt8}}, w_type::Integer, inner::Integer,
                        outers::Vector{<:Integer})
    require()
    n = length(datas)
    n == length(outers) || throw(DimensionMismatch("one row count per weight"))
    for (d, o) in zip(datas, outers)
        length(d) >= weight_bytes(w_type, inner, o) || throw(ArgumentError("a weight is too short"))
    end
    ptrs = [pointer(d) for d in datas]
    rows = Cint.(outers)
    h = Ref{UInt64}(0)
    GC.@preserve datas begin
        check(ccall((:ihip_weight_register_group, LIBIHIP), Cint,
                    (Ptr{Ptr{UInt8}}, Ptr{Cint}, Cint, Cint, Cint, Ref{UInt64}),
                    ptrs, rows, n, w_type, inner, h))
    end
    p = Ref{Ptr{Cvoid}}(C_NULL)
    check(ccall((:ihip_weight_device_ptr, LIBIHIP), Cint, (UInt64, Ref{Ptr{Cvoid}}), h[], p))
    return h[], p[]
end

end # module Device

# ============================================================================
module GGUF
# read_gguf (src/GGUF.jl:119-165) and the keep-quantized load
# (src/LoaderCPU.jl:125-163) straight into device memory: the file is
# memory-mapped and parsed by the library, and each quantized tensor is
# uploaded once into the weight registry.
export open_gguf, close_gguf, tensor_count, tensor_info, upload, upload_group, release

import ..InfernoHIP: LIBIHIP, check

"""`open_gguf(path) -> UInt64`: parse the header and tensor table (no GPU needed)."""
function open_gguf(path::AbstractString)
    fh = Ref{UInt64}(0)
    check(ccall((:ihip_gguf_open, LIBIHIP), Cint, (Cstring, Ref{UInt64}), path, fh))
    return fh[]
end

close_gguf(fh::UInt64) = check(ccall((:ihip_gguf_close, LIBIHIP), Cint, (UInt64,), fh))

"""`tensor_count(fh) -> Int`, from the header (src/GGUF.jl:125-130)."""
function tensor_count(fh::UInt64)
    version = Ref{UInt32}(0)
    alignment = Ref{UInt64}(0)
    data_offset = Ref{UInt64}(0)
    n = Ref{Int64}(0)
    check(ccall((:ihip_gguf_info, LIBIHIP), Cint,
                (UInt64, Ref{UInt32}, Ref{UInt64}, Ref{UInt64}, Ref{Int64}),
                fh, version, alignment, data_offset, n))
    return Int(n[])
end

"""
    tensor_info(fh, i) -> (name, ggml_type, dims, offset, nbytes)

Tensor `i` (1-based) of the table: dims with ne0 first, the offset relative
to the data section, and the byte count its type's blocks take.
"""
function tensor_info(fh::UInt64, i::Integer)
    name = Vector{UInt8}(undef, 1024)
    t = Ref{Cint}(0)
    nd = Ref{Cint}(0)
    dims = zeros(Int64, 4)
    off = Ref{UInt64}(0)
    nb = Ref{UInt64}(0)
    check(ccall((:ihip_gguf_tensor_info, LIBIHIP), Cint,
                (UInt64, Int64, Ptr{UInt8}, Csize_t, Ref{Cint}, Ref{Cint}, Ptr{Int64}, Ref{UInt64},
                 Ref{UInt64}),
                fh, i - 1, name, length(name), t, nd, dims, off, nb))
    s = unsafe_string(pointer(name))
    return s, Int(t[]), dims[1:nd[]], off[], nb[]
end

"""
    upload(fh, name) -> (handle, device_pointer)

Upload a Q4_K / Q5_K / Q6_K / Q8_0 / IQ4_NL tensor into the registry; the
pointer feeds the `Device` and `FusedKernels` calls until `release(handle)`.
"""
function upload(fh::UInt64, name::AbstractString)
    h = Ref{UInt64}(0)
    check(ccall((:ihip_gguf_upload, LIBIHIP), Cint, (UInt64, Cstring, Ref{UInt64}), fh, name, h))
    p = Ref{Ptr{Cvoid}}(C_NULL)
    check(ccall((:ihip_weight_device_ptr, LIBIHIP), Cint, (UInt64, Ref{Ptr{Cvoid}}), h[], p))
    return h[], p[]
end

"""
    upload_group(fh, names) -> (handle, device_pointer)

The named tensors (one type, one ne0), e.g. a layer's attn_q, attn_k and
attn_v, uploaded back to back as one weight (see `Device.register_group`).
"""
function upload_group(fh::UInt64, names::Vector{String})
    h = Ref{UInt64}(0)
    ptrs = [pointer(n) for n in names]  # Julia strings end in a NUL byte
    GC.@preserve names begin
        check(ccall((:ihip_gguf_upload_group, LIBIHIP), Cint,
                    (UInt64, Ptr{Ptr{UInt8}}, Cint, Ref{UInt64}), fh, ptrs, length(names), h))
    end
    p = Ref{Ptr{Cvoid}}(C_NULL)
    check(ccall((:ihip_weight_device_ptr, LIBIHIP), Cint, (UInt64, Ref{Ptr{Cvoid}}), h[], p))
    return h[], p[]
end

release(h::UInt64) = check(ccall((:ihip_weight_release, LIBIHIP), Cint, (UInt64,), h))

end # module GGUF

end # module InfernoHIP
