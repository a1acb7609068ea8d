/*
 * kquant_oracle.h -- CPU restatement of Inferno.jl's K-quant matvec path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * kernels.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it, and only as the checker (or the timed CPU baseline), never
 * as the product path.  The product (inferno.jl_amd/lib/libinferno_hip.so)
 * never links or calls it.
 *
 * Every function cites the reference file:line it restates.  Paths are
 * relative to the Inferno.jl checkout.
 *
 * Numerics:
 *   - dequant functions are bit-exact restatements of src/Dequant.jl
 *     (every product there is exact in fp32, see kquant_oracle.c);
 *   - orc_gemv_f64 accumulates the bit-exact fp32 weights times fp32 x in
 *     fp64: the "truth" the 1e-4*||w_row||*||x|| tolerance is measured from;
 *   - orc_gemv_f32_serial restates the Julia fallback loop
 *     (src/ModelCPU.jl:290-306): serial fp32 sum, no FMA contraction;
 *   - orc_quantize_row_q8k + orc_gemv_q8k_* restate the reference C path
 *     (src/kernels/quant_kernels.c), reproducing its 8-lane AVX2 summation
 *     order so results are bit-identical to the compiled reference.
 */
#ifndef KQUANT_ORACLE_H
#define KQUANT_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (src/GGUF.jl:25-60). */
enum {
    ORC_Q8_0 = 8,
    ORC_Q4_K = 12,
    ORC_Q5_K = 13,
    ORC_Q6_K = 14,
    ORC_IQ4_NL = 20,
};

float    orc_half_to_float(uint16_t h);
uint16_t orc_float_to_half_rne(float f);

/* bytes per block and elements per block for a type id; 0 if unknown */
int orc_block_bytes(int type);
int orc_block_elems(int type);

/* Standalone dequant, src/Dequant.jl:304-601.  n = number of elements. */
int orc_dequant(int type, const uint8_t *src, float *dst, int64_t n);

/* fp64-accumulated GEMV over the exact fp32 dequantized weights. */
int orc_gemv_f64(int type, const uint8_t *w, const float *x, double *out,
                 int inner, int outer);
/* The per-token prefill loop (src/ModelCPU.jl:1001-1017) over T tokens:
 * Y[t*outer + r] = orc_gemv_f64 of X[t*inner ...] at row r, bit for bit. */
int orc_gemm_f64(int type, const uint8_t *w, const float *X, double *Y, int T,
                 int inner, int outer);
/* ||w_row||_2 of each dequantized row (fp64). */
int orc_row_norms(int type, const uint8_t *w, double *norms, int inner, int outer);
/* Julia fallback semantics: serial fp32 accumulation per row. */
int orc_gemv_f32_serial(int type, const uint8_t *w, const float *x, float *out,
                        int inner, int outer);

/* Greedy argmax, src/CommonOps.jl:142-163 (0-based index).
 * returns 0 on success, -1 if a NaN is present, -2 if +Inf is present,
 * -3 if n == 0.  *all_neg_inf is set when every logit is -Inf. */
int orc_argmax(const float *logits, int64_t n, int64_t *index, int *all_neg_inf);

/* SwiGLU decode FFN, src/ModelCPU.jl:482-508, all in fp64.
 * g,u,h are length `inter`, y length `hidden`. Any of g/u/h may be NULL. */
int orc_ffn_swiglu_f64(int gate_type, const uint8_t *wg, int up_type,
                       const uint8_t *wu, int down_type, const uint8_t *wd,
                       const float *x, int hidden, int inter,
                       double *g, double *u, double *h, double *y);

/* rmsnorm_cpu!, src/ModelCPU.jl:111-123, in fp64. */
int orc_rmsnorm_f64(const float *x, const float *w, float eps, int n, double *out);
/* Decoder MLP half, src/ModelCPU.jl:913-920, in fp64: n = rmsnorm(x) .* nw,
 * h = silu(Wg n) * (Wu n), y = x + Wd h (n, g, u, h: hidden/inter/inter/inter). */
int orc_ffn_block_f64(int gate_type, const uint8_t *wg, int up_type, const uint8_t *wu,
                      int down_type, const uint8_t *wd, const float *x, const float *nw,
                      float eps, int hidden, int inter, double *n, double *g, double *u,
                      double *h, double *y);

/* Reference C int8-activation path, src/kernels/quant_kernels.c:166-194. */
int orc_quantize_row_q8k(const float *x, uint8_t *q8, int64_t k);
/* q{4,5,6}_k_gemv with the AVX2 lane order, quant_kernels.c:204-277,
 * 311-397, 440-521, 602-650.  q8 scratch is provided by the caller
 * (inner/256 * 292 bytes). */
int orc_gemv_q8k(int type, const uint8_t *w, const float *x, float *out,
                 uint8_t *q8, int inner, int outer);
/* q8_0_gemv, quant_kernels.c:657-683 (AVX2 branch, 8-lane fp32 FMA). */
int orc_gemv_q8_0_lanes(const uint8_t *w, const float *x, float *out,
                        int inner, int outer);

#ifdef __cplusplus
}
#endif
#endif
