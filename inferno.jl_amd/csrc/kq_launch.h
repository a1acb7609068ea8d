// kq_launch.h -- internal launchers shared by the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ihip {

// kq_gemv.hip
// resid != nullptr: y = epi_apply(resid, W x, epi) per row (kq_common.h: the
// residual add, or the SwiGLU of an unfused gate/up pair); resid may be y.
hipError_t launch_gemv(int type, const void *w, const float *x, float *y, int inner, int outer,
                       hipStream_t s, const float *resid = nullptr, int epi = 0);
bool gate_up_fusable(int gate_type, int up_type);
// norm_w != nullptr: the input is rmsnorm(x) .* norm_w (eps inside the root).
hipError_t launch_gate_up_swiglu(int type, const void *wg, const void *wu, const float *x,
                                 float *h, int hidden, int inter, hipStream_t s,
                                 const float *norm_w = nullptr, float eps = 0.0f);
// Whether the argmax can be fused into the lm_head GEMV: Q6_K / Q8_0 rows of
// at most 16 segments of 2048 columns (any vocabulary: the grid is capped at
// kArgMaxParts workgroups, one partial each).
bool lm_head_fusable(int type, int hidden);
// Argmax partials (16 bytes each) one lm_head call writes: fused into the
// streamed GEMV, or the standalone argmax after the GEMV.
int lm_head_argmax_parts(int type, int hidden, int vocab, bool fused);
hipError_t launch_lm_head_argmax(int type, const void *w, const float *x, float *logits,
                                 int32_t *token, uint32_t *flags, int hidden, int vocab,
                                 void *ws, hipStream_t s);
hipError_t launch_argmax(const float *v, int64_t n, int32_t *token, uint32_t *flags, void *ws,
                         hipStream_t s);

// kq_dequant.hip
hipError_t launch_gemv_generic(int type, const void *w, const float *x, float *y, int inner,
                               int outer, hipStream_t s, const float *resid = nullptr, int epi = 0);
// rmsnorm_cpu! (src/ModelCPU.jl:111-123): out = x * (1/sqrt(mean(x^2) + eps)) .* w
hipError_t launch_rmsnorm(const float *x, const float *w, float eps, float *out, int n,
                          hipStream_t s);
hipError_t launch_dequant(int type, const void *src, float *dst, int64_t n, bool aligned,
                          hipStream_t s);
hipError_t launch_mlp_gate_mul(float *gate, const float *up, int64_t n, hipStream_t s);
hipError_t launch_silu_gate_mul(float *out, const float *x, const float *gate, int64_t n,
                                hipStream_t s);

// kq_prefill.hip
// The prefill GEMM addresses its operands as 32-bit byte offsets from the
// start of Xh (T x inner fp16) and W (outer Q4_K rows).
inline bool prefill_fits(int T, int inner, int outer)
{
    return 2 * (int64_t)T * inner <= (int64_t)UINT32_MAX &&
           (int64_t)outer * (inner / 256) * 144 <= (int64_t)UINT32_MAX;
}
// The caller's scratch xh: the fp16 activations (T x inner), then one int
// per token (its power-of-two scale) from the next 16-byte boundary.
inline size_t prefill_scale_offset(int T, int inner)
{
    return ((size_t)2 * (size_t)T * (size_t)inner + 15) & ~(size_t)15;
}
inline size_t prefill_scratch_bytes(int T, int inner)
{
    return prefill_scale_offset(T, inner) + (size_t)4 * (size_t)T;
}
hipError_t launch_prefill_q4k(const void *w, const float *X, void *xh, float *Y, int T,
                              int inner, int outer, hipStream_t s);

// kq_q8k.hip
hipError_t launch_quantize_q8k(const float *x, void *y, int64_t k, hipStream_t s);
hipError_t launch_gemv_q8k(int type, const void *w, const void *q8, float *out, int inner,
                           int outer, hipStream_t s);
// x as fp32, quantized to Q8_K inside the launch where the kernel takes the
// shape (Q4_K / Q5_K, at most 32768 columns, 16-byte aligned w and x); q8out
// (optional) receives the Q8_K blocks; otherwise x is quantized into q8out or,
// without it, into q8tmp (inner / 256 blocks) first.
hipError_t launch_gemv_q8k_x(int type, const void *w, const float *x, void *q8out, void *q8tmp,
                             float *out, int inner, int outer, hipStream_t s);

} // namespace ihip
