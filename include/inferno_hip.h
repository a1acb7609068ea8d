/*
 * inferno_hip.h -- C ABI of the MI355X (gfx950) K-quant matvec library.
 *
 * This is the whole boundary: plain pointers, sizes and status codes, no
 * HIP or torch types.  It replaces the native library behind Inferno.jl's
 * QuantizedKernels / FusedKernels / Dequant call surface (paths relative to
 * the Inferno.jl checkout):
 *
 *   src/QuantizedKernels.jl:84-148  ccall((:q4_k_gemv,...)), q5_k, q6_k, q8_0
 *   src/kernels/quant_kernels.c:602-697  the C functions those ccalls bind
 *   src/Dequant.jl:304-601          dequantize_q8_0/_q4_k/_q5_k/_q6_k
 *   src/FusedKernels.jl:203-311     fused_mlp_gate_mul!, fused_silu_gate_mul!,
 *                                   gpu_argmax!
 *   src/ModelCPU.jl:482-508         mlp_forward (gate/up/SwiGLU/down)
 *   src/ModelCPU.jl:1091-1123 + src/CommonOps.jl:142-163
 *                                   lm_head_project! + greedy argmax
 *   src/ModelCPU.jl:1001-1017       per-token prefill loop
 *
 * Conventions
 *   - Every function returns int: IHIP_OK (0) or a negative IHIP_ERR_*.
 *     ihip_last_error() returns a message for the calling thread's last
 *     failure.  (The reference C returns void and only asserts.)
 *   - Weights are GGML blocks, row-major: output row r owns blocks
 *     [r*nb, (r+1)*nb) with nb = inner/256 (K-quants) or inner/32 (Q8_0);
 *     `inner` is GGUF ne0 = length of x (src/ModelCPU.jl:296-297).
 *   - Functions without a suffix take HOST pointers and are synchronous,
 *     like the reference.  Weights passed by host pointer are uploaded once
 *     and cached by address (they are immutable after load in the
 *     reference).  Every call checks the cached entry against the buffer's
 *     size, type, shape and sampled content fingerprint
 *     (ihip_weight_fingerprint) and uploads again on a mismatch, so a freed
 *     buffer whose address returns with other bytes, or a weight rewritten in
 *     place, is not served stale.  A rewrite that leaves every sampled
 *     window unchanged is not seen: call ihip_weight_forget after changing
 *     a weight in place.
 *   - *_dev functions take DEVICE pointers and an `ihip_stream` (a
 *     hipStream_t passed as void*, NULL = the null stream) and are
 *     asynchronous.  Device weight pointers must be 16-byte aligned.
 *   - Token ids are 0-based (Julia callers add 1).
 *   - Calls from several threads are serialized inside the library; two
 *     *_dev calls that share a workspace must not overlap on the GPU.
 *   - *_dev functions use no library-owned device memory: scratch, where a
 *     path needs it, is the caller's (h, xn, workspace arguments), so calls
 *     on different streams never share a buffer.  The host-pointer entry
 *     points stage through library buffers on the library's own stream and
 *     are synchronous.
 */
#ifndef INFERNO_HIP_H
#define INFERNO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IHIP_OK 0
#define IHIP_ERR_INVALID (-1)     /* bad argument: type, shape, pointer, alignment */
#define IHIP_ERR_HIP (-2)         /* a HIP runtime call failed */
#define IHIP_ERR_NO_DEVICE (-3)   /* no usable gfx950 device */
#define IHIP_ERR_NONFINITE (-4)   /* argmax saw NaN or +Inf (CommonOps.jl:149-152) */
#define IHIP_ERR_DISABLED (-5)    /* IHIP_DISABLE is set in the environment */
#define IHIP_ERR_NOMEM (-6)
#define IHIP_ERR_EMPTY (-7)       /* argmax of an empty vector (CommonOps.jl:177) */

/* GGML type ids (src/GGUF.jl:25-60) */
#define IHIP_Q8_0 8
#define IHIP_Q4_K 12
#define IHIP_Q5_K 13
#define IHIP_Q6_K 14

/* argmax flag bits written to *flags */
#define IHIP_FLAG_NAN 1u
#define IHIP_FLAG_POSINF 2u
#define IHIP_FLAG_ALL_NEGINF 4u

typedef void *ihip_stream;

/* ---- status / lifecycle ------------------------------------------------ */
const char *ihip_last_error(void);
int ihip_version(void);
/* 1 when a gfx950 device is usable and IHIP_DISABLE is unset, else 0.
 * Replaces quant_kernels_available (src/QuantizedKernels.jl:50-51). */
int ihip_available(void);
/* Select the device and create the library's stream (optional: the host
 * entry points initialise device 0 on first use). */
int ihip_init(int device);
/* Free every cached weight and buffer. */
int ihip_shutdown(void);

/* ---- weight registry (host entry points use it implicitly) ------------ */
/* Upload `bytes` of GGML blocks once; *handle names the device copy. */
int ihip_weight_register(const void *host, size_t bytes, int ggml_type, int inner,
                         int outer, uint64_t *handle);
int ihip_weight_release(uint64_t handle);
/* Release the cache entry of a host pointer (no-op if not cached). */
int ihip_weight_forget(const void *host);
/* The fingerprint the host-pointer cache checks: the size and 64 windows of
 * 16 bytes at evenly spaced offsets (first and last included), hashed.
 * Needs no device. */
int ihip_weight_fingerprint(const void *host, size_t bytes, uint64_t *fp);
/* Device address of a registered weight (for the *_dev entry points). */
int ihip_weight_device_ptr(uint64_t handle, const void **dev);
/* Weights that multiply the same input -- the attention's wq, wk and wv
 * (src/ModelCPU.jl:789-791), the SSM's in and gate projections (:570-571) --
 * uploaded back to back as ONE registered weight of outers[0] + ... +
 * outers[n-1] rows (1 <= n <= 64, one GGML type, one row length inner).
 * ihip_gemv_dev over it computes every member's outputs in one launch:
 * member i's are out[o_i .. o_i + outers[i] - 1] with o_i the rows before it,
 * and its blocks start ihip_weight_bytes(type, inner, o_i) bytes into the
 * group (Q4_K 4096 + 1024 + 1024 rows x 4096 columns: 5.3 us as one launch
 * against 10.3 us as three). */
int ihip_weight_register_group(const void *const *hosts, const int *outers, int n, int ggml_type,
                               int inner, uint64_t *handle);
/* Bytes of an outer x inner weight of a GGML type (0 for an unknown type or
 * an inner that is not a whole number of blocks). */
size_t ihip_weight_bytes(int ggml_type, int inner, int outer);

/* ---- drop-in mirrors of src/kernels/quant_kernels.c ------------------- */
/* Same arguments as q{4,5,6}_k_gemv (quant_kernels.c:602, 620, 638); the
 * Q8_K scratch argument is accepted and ignored (activations stay fp32). */
int ihip_q4_k_gemv(const uint8_t *weight, const float *x, float *out, void *q8_buf_unused,
                   int inner_dim, int outer_dim);
int ihip_q5_k_gemv(const uint8_t *weight, const float *x, float *out, void *q8_buf_unused,
                   int inner_dim, int outer_dim);
int ihip_q6_k_gemv(const uint8_t *weight, const float *x, float *out, void *q8_buf_unused,
                   int inner_dim, int outer_dim);
/* Same arguments as q8_0_gemv (quant_kernels.c:657). */
int ihip_q8_0_gemv(const uint8_t *weight, const float *x, float *out, int inner_dim,
                   int outer_dim);
/* mul_quant_mat_vec(::IQ4NL_Matrix) (src/ModelCPU.jl:381-408): 18-byte
 * blocks of 32 (f16 d, 16 bytes of 4-bit indices into the grid of
 * src/QuantsData.jl:384); GGML type 20.  The same arguments as
 * ihip_q8_0_gemv. */
int ihip_iq4_nl_gemv(const uint8_t *weight, const float *x, float *out, int inner_dim,
                     int outer_dim);

/* ---- GGUF files feeding the weight registry ------------------------------
 * read_gguf (src/GGUF.jl:119-165) and the keep-quantized load
 * (src/LoaderCPU.jl:125-163): the file is memory-mapped and parsed (no GPU
 * needed); tensors are listed by index (from 0); a Q4_K, Q5_K, Q6_K, Q8_0 or
 * IQ4_NL tensor uploads into the registry (inner = ne0, outer = ne1) for
 * ihip_weight_device_ptr and the *_dev entry points. */
int ihip_gguf_open(const char *path, uint64_t *file_handle);
int ihip_gguf_close(uint64_t file_handle);
int ihip_gguf_info(uint64_t file_handle, uint32_t *version, uint64_t *alignment,
                   uint64_t *data_offset, int64_t *tensor_count);
/* name is NUL-terminated into name[name_cap]; dims[0] = ne0 (unused dims 1);
 * offset is relative to the data section; nbytes = blocks x block size of the
 * type (0 for a type without a known block size). */
int ihip_gguf_tensor_info(uint64_t file_handle, int64_t index, char *name, size_t name_cap,
                          int *ggml_type, int *ndim, int64_t dims[4], uint64_t *offset,
                          uint64_t *nbytes);
/* get_tensor_raw_bytes (src/GGUF.jl:186-205) sized by the tensor's type
 * rather than 4 bytes per element: copies nbytes into dst. */
int ihip_gguf_tensor_bytes(uint64_t file_handle, const char *name, void *dst, size_t dst_bytes);
int ihip_gguf_upload(uint64_t file_handle, const char *name, uint64_t *weight_handle);
/* ihip_weight_register_group from the file: the named tensors (one type, one
 * ne0) back to back as one registered weight, in the order given. */
int ihip_gguf_upload_group(uint64_t file_handle, const char *const *names, int n,
                           uint64_t *weight_handle);

/* ---- int8-activation variant: the reference C numerics, bit for bit ---- */
/* Q8_K block: float d, int8 qs[256], int16 bsums[16] (292 bytes,
 * block_q8_K, quant_kernels.c:51-56). */
#define IHIP_Q8_K_BYTES 292
/* quantize_row_q8_K(x, y, k) (quant_kernels.c:166-194): k % 256 == 0, y gets
 * k/256 Q8_K blocks.  Replaces the binding of quantize_q8_k!
 * (src/QuantizedKernels.jl:151-156), whose ccall passes (y, x, Cint): here
 * the arguments are in the C order. */
int ihip_quantize_row_q8_k(const float *x, void *y, int64_t k);
/* vec_dot_q{4,5,6}_K_q8_K(x, y, nb) (quant_kernels.c:204, 311, 440), bound
 * by vec_dot_q{4,5,6}_k_q8_k (src/QuantizedKernels.jl:159-178): one weight
 * row of nb blocks against nb Q8_K blocks; the float result goes to *s. */
int ihip_vec_dot_q4_k_q8_k(const void *x, const void *y, int nb, float *s);
int ihip_vec_dot_q5_k_q8_k(const void *x, const void *y, int nb, float *s);
int ihip_vec_dot_q6_k_q8_k(const void *x, const void *y, int nb, float *s);
/* q{4,5,6}_k_gemv with the reference C numerics (quant_kernels.c:602-650:
 * x re-quantized to Q8_K, integer dots): the same arguments as
 * ihip_q{4,5,6}_k_gemv; when q8_buf is not NULL it receives the Q8_K blocks
 * of x (inner/256 * IHIP_Q8_K_BYTES), as the reference's scratch does. */
int ihip_q4_k_gemv_q8k(const uint8_t *weight, const float *x, float *out, void *q8_buf,
                       int inner_dim, int outer_dim);
int ihip_q5_k_gemv_q8k(const uint8_t *weight, const float *x, float *out, void *q8_buf,
                       int inner_dim, int outer_dim);
int ihip_q6_k_gemv_q8k(const uint8_t *weight, const float *x, float *out, void *q8_buf,
                       int inner_dim, int outer_dim);

/* ---- Dequant (src/Dequant.jl:304-601): bit-exact blocks -> fp32 -------- */
/* n = number of elements; src holds n/256 (or n/32) blocks. */
int ihip_dequantize(int ggml_type, const uint8_t *src, float *dst, int64_t n);

/* ---- fused calls (host pointers, synchronous) ---------------------------- */
/* mlp_forward, src/ModelCPU.jl:482-508: h = silu(Wg x) .* (Wu x), y = Wd h.
 * wg, wu: inter x hidden; wd: hidden x inter. h may be NULL. */
int ihip_ffn_swiglu(int gate_type, const uint8_t *wg, int up_type, const uint8_t *wu,
                    int down_type, const uint8_t *wd, const float *x, float *h, float *y,
                    int hidden, int inter);
/* lm_head_project! + greedy token (ModelCPU.jl:1091-1123, CommonOps.jl:142-163):
 * logits = W x (W: vocab x hidden), *token = lowest index of the max.
 * logits may be NULL.  Returns IHIP_ERR_NONFINITE on NaN/+Inf logits. */
int ihip_lm_head_argmax(int ggml_type, const uint8_t *w, const float *x, float *logits,
                        int32_t *token, int hidden, int vocab);
/* The MLP half of a decoder layer (src/ModelCPU.jl:913-920): x <- x + Wd h,
 * h = silu(Wg n) .* (Wu n), n = rmsnorm_cpu!(x, norm_w, eps)
 * (src/ModelCPU.jl:111-123: x * (1/sqrt(mean(x^2) + eps)) .* norm_w).  x is
 * updated in place. */
int ihip_ffn_block(int gate_type, const uint8_t *wg, int up_type, const uint8_t *wu,
                   int down_type, const uint8_t *wd, const float *norm_w, float eps, float *x,
                   int hidden, int inter);
/* Batched prefill: Y[t,:] = W X[t,:] for t < T (W: outer x inner Q4_K), for
 * any finite fp32 X.  The activations are rounded to fp16 for the matrix
 * cores, each token row first scaled by a power of two that puts its largest
 * magnitude in [2^14, 2^15) (undone exactly on the outputs), so no finite
 * value overflows and small ones keep fp16's 11 significant bits down to
 * 2^-29 of their row's maximum. */
int ihip_prefill_q4_k(const uint8_t *w, const float *X, float *Y, int T, int inner,
                      int outer);

/* ---- device-pointer entry points (asynchronous on `stream`) -------------- */
/* out = W x on device pointers.  Device entry points refuse, with
 * IHIP_ERR_INVALID, inputs that overlap the outputs their kernels write while
 * every workgroup reads the inputs (x and out here; x and h of the gate/up
 * pair; x and logits; src and dst of a dequantization; X, xh and Y of the
 * prefill). */
int ihip_gemv_dev(int ggml_type, const void *w, const float *x, float *out, int inner,
                  int outer, ihip_stream stream);
/* out = resid + W x, the residual add folded into the GEMV's epilogue: the
 * attention's output projection (src/ModelCPU.jl:885) and the layer's
 * x .+= residual (:909) as one launch.  resid may be out (in place) but not
 * overlap it otherwise; x may not overlap out. */
int ihip_gemv_add_dev(int ggml_type, const void *w, const float *x, const float *resid,
                      float *out, int inner, int outer, ihip_stream stream);
/* out = W (rmsnorm(x) .* norm_w): a layer's input norm (src/ModelCPU.jl:903,
 * rmsnorm_cpu! at :111-123) folded into the GEMV that consumes it, e.g. the
 * grouped wq/wk/wv (:789-791).  One launch for 16-byte aligned Q4_K / Q5_K
 * rows of at most 4096 columns.  Otherwise xn
 * (inner floats of caller scratch) receives the normed input and the plain
 * GEMV follows; xn may be NULL only where the norm folds. */
int ihip_gemv_norm_dev(int ggml_type, const void *w, const float *norm_w, float eps,
                       const float *x, float *xn, float *out, int inner, int outer,
                       ihip_stream stream);
int ihip_dequantize_dev(int ggml_type, const void *src, float *dst, int64_t n,
                        ihip_stream stream);
/* h = silu(Wg x) .* (Wu x) (h: inter floats).  A matching Q4_K or Q5_K pair
 * (16-byte aligned) runs as one pass over both weights; any other pair writes
 * Wg x into h and the up GEMV turns it into silu(h) * (Wu x) in place. */
int ihip_gate_up_swiglu_dev(int gate_type, const void *wg, int up_type, const void *wu,
                            const float *x, float *h, int hidden, int inter,
                            ihip_stream stream);
/* gate/up/SwiGLU then down: y = Wd h; h is caller-provided (inter floats). */
int ihip_ffn_swiglu_dev(int gate_type, const void *wg, int up_type, const void *wu,
                        int down_type, const void *wd, const float *x, float *h, float *y,
                        int hidden, int inter, ihip_stream stream);
/* Workspace for the argmax entry points: IHIP_ARGMAX_WS_BYTES of device
 * memory (per-workgroup partial maxima; no initialisation needed).  Calls
 * that share a workspace must not overlap on the GPU. */
#define IHIP_ARGMAX_WS_BYTES 262144
/* GEMV + fused greedy argmax.  *token and *flags are device int32s (flags:
 * IHIP_FLAG_* bits; the token is meaningless when NAN or POSINF is set).
 * logits may be NULL when the argmax is fused into the GEMV, which
 * ihip_lm_head_fused reports: a Q6_K or Q8_0 weight, 16-byte aligned w and x,
 * and hidden a whole number of blocks of at most 32768 columns.  Otherwise
 * the GEMV writes logits and a second kernel reduces them, and NULL logits is
 * IHIP_ERR_INVALID. */
int ihip_lm_head_argmax_dev(int ggml_type, const void *w, const float *x, float *logits,
                            int32_t *token, uint32_t *flags, int hidden, int vocab,
                            void *workspace, ihip_stream stream);
/* ihip_lm_head_argmax_dev without the workspace argument.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation).  The argmax partials go to a library array of
 * IHIP_ARGMAX_WS_BYTES in each device's memory (one 16-byte partial per
 * workgroup, at most 16384; a call that would need more is IHIP_ERR_INVALID),
 * resolved once per device -- at ihip_init or at the first call on that
 * device -- and never allocated per call.  Every call on a device shares its
 * array: calls that overlap on one GPU race.  Same arguments, outputs and
 * errors as ihip_lm_head_argmax_dev otherwise. */
int ihip_lm_head_argmax_noalloc_dev(int ggml_type, const void *w, const float *x, float *logits,
                                    int32_t *token, uint32_t *flags, int hidden, int vocab,
                                    ihip_stream stream);
/* 1 when ihip_lm_head_argmax_dev with these arguments fuses the argmax into
 * the GEMV (logits may then be NULL), else 0. */
int ihip_lm_head_fused(int ggml_type, const void *w, const float *x, int hidden, int vocab);
/* gpu_argmax! (FusedKernels.jl:271-311) with _validate_logits semantics. */
int ihip_argmax_dev(const float *logits, int64_t n, int32_t *token, uint32_t *flags,
                    void *workspace, ihip_stream stream);
/* fused_mlp_gate_mul! (FusedKernels.jl:203-214): gate = gate/(1+exp(-gate))*up */
int ihip_fused_mlp_gate_mul_dev(float *gate, const float *up, int64_t n, ihip_stream stream);
/* fused_silu_gate_mul! (FusedKernels.jl:219-230): out = x/(1+exp(-x))*gate */
int ihip_fused_silu_gate_mul_dev(float *out, const float *x, const float *gate, int64_t n,
                                 ihip_stream stream);
/* X: T x inner fp32 (row-major), Y: T x outer fp32.  `xh` is caller scratch
 * of ihip_prefill_scratch_bytes(T, inner) bytes: the rounded activations
 * (T*inner fp16 values), one scale exponent per token and room for the
 * partial sums of a weight of few rows, whose K is split over several
 * workgroups (the size does not depend on outer).  Rows of more than 512
 * columns multiply fp16 operands: any finite X (each token row is scaled by
 * a power of two), but every dequantized weight below 65504 in magnitude.
 * w, X, xh and Y are 16-byte aligned; calls that share xh must not overlap
 * on the GPU. */
int ihip_prefill_q4_k_dev(const void *w, const float *X, void *xh, float *Y, int T,
                          int inner, int outer, ihip_stream stream);
size_t ihip_prefill_scratch_bytes(int T, int inner);
/* ihip_prefill_q4_k_dev in two halves, for weights that multiply the same
 * activations: the attention's wq, wk and wv (src/ModelCPU.jl:789-791), the
 * MLP's gate and up (:490, 498), the SSM's in and gate projections
 * (:570-571).  ihip_prefill_convert_dev rounds X into xh (as
 * ihip_prefill_q4_k_dev does); each ihip_prefill_q4_k_xh_dev then multiplies
 * one weight by the rounded rows, with outputs bit-identical to
 * ihip_prefill_q4_k_dev's for that weight.  The product reuses xh's
 * partial-sum area and leaves the rounded rows as they were, so any number
 * of products (same T and inner) may follow one conversion; none of them may
 * overlap another call that uses xh on the GPU.  Rows of at most 512 columns
 * are IHIP_ERR_INVALID here: ihip_prefill_q4_k_dev multiplies them on fp32
 * operands straight from X. */
int ihip_prefill_convert_dev(const float *X, void *xh, int T, int inner, ihip_stream stream);
int ihip_prefill_q4_k_xh_dev(const void *w, void *xh, float *Y, int T, int inner, int outer,
                             ihip_stream stream);
/* The per-token prefill loop (src/ModelCPU.jl:1001-1017 over
 * mul_quant_mat_vec, :285-307) on fp32 operands: the weights dequantized to
 * fp32 exactly and X as given, multiplied on the fp32 matrix cores.  The
 * error is fp32 rounding, within 1e-4 * ||w_row|| * ||x|| for any finite X;
 * ihip_prefill_q4_k_dev (which takes this path for rows of at most 512
 * columns) rounds both operands of longer rows to fp16, which meets that
 * bound for the benchmark's data but not for every X (a token equal to a
 * weight row reaches 2-3x it) and needs every dequantized weight below
 * 65504 in magnitude.  Several times slower than the fp16 path on long rows;
 * no scratch.  w, X and Y are 16-byte aligned; T * outer < 2^31. */
int ihip_prefill_q4_k_f32_dev(const void *w, const float *X, float *Y, int T, int inner,
                              int outer, ihip_stream stream);

/* rmsnorm_cpu! (src/ModelCPU.jl:111-123): out = x * (1/sqrt(mean(x^2) + eps))
 * .* w over n values (out may alias x). */
int ihip_rmsnorm_dev(const float *x, const float *w, float eps, float *out, int n,
                     ihip_stream stream);
/* ihip_ffn_block on device pointers: the norm is folded into the fused gate/up
 * pass (its scale multiplies the row sums) and the residual add into the down
 * projection's epilogue.  h: caller scratch of ihip_ffn_block_scratch_floats()
 * floats, inter + hidden for every pair: h receives silu(g) .* u, and a pair
 * that does not run as one fused pass (not a matching Q4_K or Q5_K pair, or
 * wg, wu, x or norm_w off 16-byte alignment) puts the normed input in
 * h + inter. */
int ihip_ffn_block_dev(int gate_type, const void *wg, int up_type, const void *wu, int down_type,
                       const void *wd, const float *norm_w, float eps, float *x, float *h,
                       int hidden, int inter, ihip_stream stream);
size_t ihip_ffn_block_scratch_floats(int gate_type, int up_type, int hidden, int inter);
/* Final norm + lm_head + greedy token (src/ModelCPU.jl:1014-1015): xn
 * (hidden floats of caller scratch) receives rmsnorm(x) .* norm_w; the rest
 * is ihip_lm_head_argmax_dev on xn. */
int ihip_lm_head_argmax_norm_dev(int ggml_type, const void *w, const float *norm_w, float eps,
                                 const float *x, float *xn, float *logits, int32_t *token,
                                 uint32_t *flags, int hidden, int vocab, void *workspace,
                                 ihip_stream stream);

/* Device twins of the int8-activation variant.  x: 4-byte aligned fp32,
 * y / q8: 4-byte aligned Q8_K blocks; w: 16-byte aligned (Q4_K, Q5_K) or
 * 2-byte aligned (Q6_K). */
int ihip_quantize_row_q8_k_dev(const float *x, void *y, int64_t k, ihip_stream stream);
int ihip_gemv_q8k_dev(int ggml_type, const void *w, const void *q8, float *out, int inner,
                      int outer, ihip_stream stream);
/* The same with x as fp32, quantized to Q8_K as ihip_quantize_row_q8_k_dev
 * does -- the reference's q{4,5,6}_k_gemv (src/kernels/quant_kernels.c:602-650)
 * as one device call.  Q4_K / Q5_K rows of at most 32768 columns with a
 * 16-byte aligned x run as one launch, and q8 (when not NULL) receives the
 * Q8_K blocks of x; other cases quantize x into q8 first, which they then
 * require (inner/256 * IHIP_Q8_K_BYTES, 4-byte aligned). */
int ihip_gemv_q8k_x_dev(int ggml_type, const void *w, const float *x, float *out, void *q8,
                        int inner, int outer, ihip_stream stream);

#ifdef __cplusplus
}
#endif
#endif /* INFERNO_HIP_H */
