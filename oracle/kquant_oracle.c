/*
 * kquant_oracle.c -- CPU restatement of Inferno.jl's K-quant matvec path.
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker; see kquant_oracle.h).
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off; no -ffast-math, so
 * fp16 subnormals, NaN and Inf behave as IEEE says).
 *
 * Reference files restated (paths relative to the Inferno.jl checkout):
 *   src/Dequant.jl:304-321   dequantize_q8_0
 *   src/Dequant.jl:325-375   dequantize_q4_k
 *   src/Dequant.jl:379-441   dequantize_q5_k
 *   src/Dequant.jl:558-601   dequantize_q6_k
 *   src/ModelCPU.jl:285-379  mul_quant_mat_vec (fp32-activation fallback)
 *   src/ModelCPU.jl:482-508  mlp_forward (SwiGLU)
 *   src/CommonOps.jl:142-163 _validate_logits (greedy argmax)
 *   src/kernels/quant_kernels.c:166-194, 204-277, 311-397, 440-521,
 *                               602-697 (int8-activation C path)
 *
 * Exactness of the dequant restatement (why "bit-exact" is well defined):
 *   Q4_K/Q5_K: d*sc has <= 11+6 significant bits and (d*sc)*q <= 11+6+5,
 *   dmin*m <= 17 bits, all exact in fp32; only the final subtraction rounds.
 *   Q6_K: d*sc*q <= 11+6+6 bits, exact.  Q8_0: d*q <= 11+8 bits, exact.
 *   So any implementation that forms the same products and one subtraction
 *   produces identical bits, with or without FMA.
 */
#include "kquant_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* fp16 <-> fp32                                                        */
/* ------------------------------------------------------------------ */

/* Float32(reinterpret(Float16, bits)) as used at src/Dequant.jl:313, 337-338,
 * 574: exact widening.  Subnormal halves are m * 2^-24, which is an exact
 * fp32 normal number; the rest is a re-bias of the exponent. */
float orc_half_to_float(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    float f;
    if (e == 0) {
        f = (float)m * 0x1p-24f;
        return sign ? -f : f;
    }
    uint32_t bits;
    if (e == 31)
        bits = sign | 0x7f800000u | (m << 13);
    else
        bits = sign | ((e + 112u) << 23) | (m << 13);
    memcpy(&f, &bits, 4);
    return f;
}

/* IEEE round-to-nearest-even fp32 -> fp16 (used for the prefill operands:
 * the MFMA path feeds fp16 activations, so the oracle rounds x the same
 * way before its fp64 sum). */
uint16_t orc_float_to_half_rne(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u)
        return (uint16_t)(sign | 0x7e00u);          /* NaN */
    if (ax >= 0x477ff000u)
        return (uint16_t)(sign | 0x7c00u);          /* >= 65520 rounds to Inf */
    const int E = (int)(ax >> 23) - 127;
    if (E >= -14) {
        const uint32_t mant = ax & 0x7fffffu;
        uint32_t hb = ((uint32_t)(E + 15) << 10) | (mant >> 13);
        const uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (hb & 1u)))
            hb += 1u;
        return (uint16_t)(sign | hb);
    }
    if (E < -25)
        return (uint16_t)sign;
    const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    const int shift = -(E + 1);                      /* 14..24 */
    uint32_t q = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u)))
        q += 1u;
    return (uint16_t)(sign | q);
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

int orc_block_bytes(int type)
{
    switch (type) {
    case ORC_Q8_0: return 34;
    case ORC_Q4_K: return 144;
    case ORC_Q5_K: return 176;
    case ORC_Q6_K: return 210;
    case ORC_IQ4_NL: return 18;
    default: return 0;
    }
}

int orc_block_elems(int type)
{
    switch (type) {
    case ORC_Q8_0: case ORC_IQ4_NL: return 32;
    case ORC_Q4_K: case ORC_Q5_K: case ORC_Q6_K: return 256;
    default: return 0;
    }
}

/* ------------------------------------------------------------------ */
/* Per-block dequant                                                    */
/* ------------------------------------------------------------------ */

/* 6-bit scale/min of sub-block i (0..7) from the 12 packed bytes,
 * src/Dequant.jl:345-362. */
static inline void k_scale_min(const uint8_t *s, int i, unsigned *sc, unsigned *m)
{
    if (i < 4) {
        *sc = s[i] & 63u;
        *m = s[i + 4] & 63u;
    } else {
        *sc = (s[i + 4] & 0x0fu) | ((unsigned)(s[i - 4] >> 6) << 4);
        *m = (unsigned)(s[i + 4] >> 4) | ((unsigned)(s[i] >> 6) << 4);
    }
}

/* src/Dequant.jl:325-375 */
static void deq_q4_k_block(const uint8_t *b, float *y)
{
    const float d = orc_half_to_float(rd16(b));
    const float dmin = orc_half_to_float(rd16(b + 2));
    const uint8_t *s = b + 4;
    const uint8_t *qs = b + 16;
    for (int j = 0; j < 4; ++j) {
        unsigned sc1, m1, sc2, m2;
        k_scale_min(s, 2 * j, &sc1, &m1);
        k_scale_min(s, 2 * j + 1, &sc2, &m2);
        const float d1 = d * (float)sc1, min1 = dmin * (float)m1;
        const float d2 = d * (float)sc2, min2 = dmin * (float)m2;
        for (int l = 0; l < 32; ++l) {
            const uint8_t q = qs[32 * j + l];
            y[64 * j + l] = d1 * (float)(q & 0x0f) - min1;
            y[64 * j + 32 + l] = d2 * (float)(q >> 4) - min2;
        }
    }
}

/* src/Dequant.jl:379-441 */
static void deq_q5_k_block(const uint8_t *b, float *y)
{
    const float d = orc_half_to_float(rd16(b));
    const float dmin = orc_half_to_float(rd16(b + 2));
    const uint8_t *s = b + 4;
    const uint8_t *qh = b + 16;
    const uint8_t *qs = b + 48;
    for (int j = 0; j < 4; ++j) {
        unsigned sc1, m1, sc2, m2;
        k_scale_min(s, 2 * j, &sc1, &m1);
        k_scale_min(s, 2 * j + 1, &sc2, &m2);
        const float d1 = d * (float)sc1, min1 = dmin * (float)m1;
        const float d2 = d * (float)sc2, min2 = dmin * (float)m2;
        const unsigned u1 = 1u << (2 * j), u2 = 1u << (2 * j + 1);
        for (int l = 0; l < 32; ++l) {
            const uint8_t q = qs[32 * j + l];
            const uint8_t h = qh[l];
            const unsigned lo = (q & 0x0fu) + ((h & u1) ? 16u : 0u);
            const unsigned hi = (unsigned)(q >> 4) + ((h & u2) ? 16u : 0u);
            y[64 * j + l] = d1 * (float)lo - min1;
            y[64 * j + 32 + l] = d2 * (float)hi - min2;
        }
    }
}

/* src/Dequant.jl:558-601 (the correct decoder; NOT the
 * QuantsCPU.dequantize_q6_k_block! variant at src/QuantsCPU.jl:648-694,
 * which picks the wrong scale for 192 of 256 elements). */
static void deq_q6_k_block(const uint8_t *b, float *y)
{
    const uint8_t *ql = b;
    const uint8_t *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    const float d = orc_half_to_float(rd16(b + 208));
    for (int n = 0; n < 2; ++n) {
        const uint8_t *L = ql + 64 * n;
        const uint8_t *H = qh + 32 * n;
        const int8_t *S = sc + 8 * n;
        for (int l = 0; l < 32; ++l) {
            const int is = l / 16;
            const unsigned h = H[l];
            const int q1 = (int)((L[l] & 0x0fu) | ((h & 3u) << 4)) - 32;
            const int q2 = (int)((L[l + 32] & 0x0fu) | (((h >> 2) & 3u) << 4)) - 32;
            const int q3 = (int)((unsigned)(L[l] >> 4) | (((h >> 4) & 3u) << 4)) - 32;
            const int q4 = (int)((unsigned)(L[l + 32] >> 4) | (((h >> 6) & 3u) << 4)) - 32;
            y[128 * n + l] = d * (float)S[is] * (float)q1;
            y[128 * n + 32 + l] = d * (float)S[is + 2] * (float)q2;
            y[128 * n + 64 + l] = d * (float)S[is + 4] * (float)q3;
            y[128 * n + 96 + l] = d * (float)S[is + 6] * (float)q4;
        }
    }
}

/* src/Dequant.jl:304-321 */
static void deq_q8_0_block(const uint8_t *b, float *y)
{
    const float d = orc_half_to_float(rd16(b));
    for (int j = 0; j < 32; ++j)
        y[j] = d * (float)(int8_t)b[2 + j];
}

/* src/Dequant.jl:683-693 (dequantize_iq4_nl_into!): y[j] = d *
 * KVALUES_IQ4NL[qs[j] & 15], y[j + 16] = d * KVALUES_IQ4NL[qs[j] >> 4]
 * (the grid is src/QuantsData.jl:384). */
static void deq_iq4_nl_block(const uint8_t *b, float *y)
{
    static const int8_t kv[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                  1,    13,   25,  38,  53,  69,  89,  113};
    const float d = orc_half_to_float(rd16(b));
    for (int j = 0; j < 16; ++j) {
        y[j] = d * (float)kv[b[2 + j] & 15];
        y[j + 16] = d * (float)kv[b[2 + j] >> 4];
    }
}

typedef void (*deq_fn)(const uint8_t *, float *);

static deq_fn deq_for(int type)
{
    switch (type) {
    case ORC_Q8_0: return deq_q8_0_block;
    case ORC_Q4_K: return deq_q4_k_block;
    case ORC_Q5_K: return deq_q5_k_block;
    case ORC_Q6_K: return deq_q6_k_block;
    case ORC_IQ4_NL: return deq_iq4_nl_block;
    default: return NULL;
    }
}

int orc_dequant(int type, const uint8_t *src, float *dst, int64_t n)
{
    const deq_fn f = deq_for(type);
    const int be = orc_block_elems(type), bb = orc_block_bytes(type);
    if (!f || n < 0 || n % be)
        return -1;
    const int64_t nb = n / be;
    for (int64_t i = 0; i < nb; ++i)
        f(src + i * bb, dst + i * be);
    return 0;
}

/* ------------------------------------------------------------------ */
/* GEMV semantics                                                       */
/* ------------------------------------------------------------------ */

static int check_dims(int type, int inner, int outer)
{
    const int be = orc_block_elems(type);
    if (!be || inner <= 0 || outer < 0 || inner % be)
        return -1;
    return 0;
}

/* out[r] = sum_c W[r,c] x[c]; W from the exact dequant, fp64 accumulate.
 * Row r's blocks are [r*nb, (r+1)*nb) (src/ModelCPU.jl:296-297). */
int orc_gemv_f64(int type, const uint8_t *w, const float *x, double *out,
                 int inner, int outer)
{
    if (check_dims(type, inner, outer))
        return -1;
    const deq_fn f = deq_for(type);
    const int be = orc_block_elems(type), bb = orc_block_bytes(type);
    const int nb = inner / be;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < outer; ++r) {
        float blk[256];
        double acc = 0.0;
        for (int b = 0; b < nb; ++b) {
            f(w + ((size_t)r * nb + b) * bb, blk);
            const float *xv = x + (size_t)b * be;
            for (int i = 0; i < be; ++i)
                acc += (double)blk[i] * (double)xv[i];
        }
        out[r] = acc;
    }
    return 0;
}

/* The per-token prefill loop, src/ModelCPU.jl:1001-1017: every token t is one
 * GEMV of the same weight, Y[t][r] = sum_c W[r][c] * X[t][c].  Each output is
 * summed in fp64 in column order, exactly as orc_gemv_f64 sums it, so row t of
 * Y equals orc_gemv_f64 on X[t] bit for bit; rows of W are dequantized once
 * per group of 8 and shared by all T tokens. */
int orc_gemm_f64(int type, const uint8_t *w, const float *X, double *Y, int T,
                 int inner, int outer)
{
    if (check_dims(type, inner, outer) || T < 0)
        return -1;
    const deq_fn f = deq_for(type);
    const int be = orc_block_elems(type), bb = orc_block_bytes(type);
    const int nb = inner / be;
    enum { RG = 8 };
    int bad = 0;
#pragma omp parallel
    {
        double *wr = (double *)malloc(sizeof(double) * (size_t)RG * (size_t)inner);
        if (!wr) {
#pragma omp atomic write
            bad = 1;
        }
#pragma omp for schedule(dynamic, 1)
        for (int r0 = 0; r0 < outer; r0 += RG) {
            if (!wr)
                continue;
            const int nr = outer - r0 < RG ? outer - r0 : RG;
            float blk[256];
            for (int i = 0; i < nr; ++i)
                for (int b = 0; b < nb; ++b) {
                    f(w + ((size_t)(r0 + i) * nb + b) * bb, blk);
                    for (int e = 0; e < be; ++e)
                        wr[(size_t)i * inner + (size_t)b * be + e] = (double)blk[e];
                }
            for (int t = 0; t < T; ++t) {
                const float *xt = X + (size_t)t * inner;
                double acc[RG] = {0};
                for (int c = 0; c < inner; ++c) {
                    const double xc = (double)xt[c];
                    for (int i = 0; i < nr; ++i)
                        acc[i] += wr[(size_t)i * inner + c] * xc;
                }
                for (int i = 0; i < nr; ++i)
                    Y[(size_t)t * outer + r0 + i] = acc[i];
            }
        }
        free(wr);
    }
    return bad ? -2 : 0;
}

int orc_row_norms(int type, const uint8_t *w, double *norms, int inner, int outer)
{
    if (check_dims(type, inner, outer))
        return -1;
    const deq_fn f = deq_for(type);
    const int be = orc_block_elems(type), bb = orc_block_bytes(type);
    const int nb = inner / be;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < outer; ++r) {
        float blk[256];
        double acc = 0.0;
        for (int b = 0; b < nb; ++b) {
            f(w + ((size_t)r * nb + b) * bb, blk);
            for (int i = 0; i < be; ++i)
                acc += (double)blk[i] * (double)blk[i];
        }
        norms[r] = sqrt(acc);
    }
    return 0;
}

/* src/ModelCPU.jl:290-306: serial fp32 `sum_val += w*x` (no FMA; the file
 * is built with -ffp-contract=off). */
int orc_gemv_f32_serial(int type, const uint8_t *w, const float *x, float *out,
                        int inner, int outer)
{
    if (check_dims(type, inner, outer))
        return -1;
    const deq_fn f = deq_for(type);
    const int be = orc_block_elems(type), bb = orc_block_bytes(type);
    const int nb = inner / be;
    float blk[256];
    for (int r = 0; r < outer; ++r) {
        float acc = 0.0f;
        for (int b = 0; b < nb; ++b) {
            f(w + ((size_t)r * nb + b) * bb, blk);
            const float *xv = x + (size_t)b * be;
            for (int i = 0; i < be; ++i) {
                const float p = blk[i] * xv[i];
                acc = acc + p;
            }
        }
        out[r] = acc;
    }
    return 0;
}

/* src/CommonOps.jl:142-163: strict `>` scan from the start, so the lowest
 * index wins among equal maxima; NaN and +Inf are errors; -Inf is skipped;
 * all -Inf gives the first index. */
int orc_argmax(const float *logits, int64_t n, int64_t *index, int *all_neg_inf)
{
    if (n <= 0)
        return -3;
    float best = -INFINITY;
    int64_t bi = 0;
    int all_ni = 1;
    for (int64_t i = 0; i < n; ++i) {
        const float v = logits[i];
        if (isnan(v))
            return -1;
        if (v == INFINITY)
            return -2;
        if (v != -INFINITY) {
            all_ni = 0;
            if (v > best) {
                best = v;
                bi = i;
            }
        }
    }
    *index = bi;
    if (all_neg_inf)
        *all_neg_inf = all_ni;
    return 0;
}

/* src/ModelCPU.jl:482-508 in fp64: g = Wg x; g <- g/(1+exp(-g));
 * u = Wu x; h = g .* u; y = Wd h. */
int orc_ffn_swiglu_f64(int gate_type, const uint8_t *wg, int up_type,
                       const uint8_t *wu, int down_type, const uint8_t *wd,
                       const float *x, int hidden, int inter,
                       double *g, double *u, double *h, double *y)
{
    if (check_dims(gate_type, hidden, inter) || check_dims(up_type, hidden, inter) ||
        check_dims(down_type, inter, hidden))
        return -1;
    double *gg = malloc(sizeof(double) * (size_t)inter);
    double *uu = malloc(sizeof(double) * (size_t)inter);
    double *hh = malloc(sizeof(double) * (size_t)inter);
    if (!gg || !uu || !hh) {
        free(gg); free(uu); free(hh);
        return -2;
    }
    orc_gemv_f64(gate_type, wg, x, gg, hidden, inter);
    orc_gemv_f64(up_type, wu, x, uu, hidden, inter);
    for (int i = 0; i < inter; ++i)
        hh[i] = gg[i] / (1.0 + exp(-gg[i])) * uu[i];
    /* down projection over the fp64 h */
    const deq_fn f = deq_for(down_type);
    const int be = orc_block_elems(down_type), bb = orc_block_bytes(down_type);
    const int nb = inter / be;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < hidden; ++r) {
        float blk[256];
        double acc = 0.0;
        for (int b = 0; b < nb; ++b) {
            f(wd + ((size_t)r * nb + b) * bb, blk);
            for (int i = 0; i < be; ++i)
                acc += (double)blk[i] * hh[(size_t)b * be + i];
        }
        y[r] = acc;
    }
    if (g) memcpy(g, gg, sizeof(double) * (size_t)inter);
    if (u) memcpy(u, uu, sizeof(double) * (size_t)inter);
    if (h) memcpy(h, hh, sizeof(double) * (size_t)inter);
    free(gg); free(uu); free(hh);
    return 0;
}

/* rmsnorm_cpu!, src/ModelCPU.jl:111-123, in fp64 over the fp32 inputs:
 * out[i] = x[i] * (1 / sqrt(sum(x^2) / n + eps)) * w[i]. */
int orc_rmsnorm_f64(const float *x, const float *w, float eps, int n, double *out)
{
    if (n <= 0)
        return -1;
    double ss = 0.0;
    for (int i = 0; i < n; ++i)
        ss += (double)x[i] * (double)x[i];
    const double scale = 1.0 / sqrt(ss / (double)n + (double)eps);
    for (int i = 0; i < n; ++i)
        out[i] = (double)x[i] * scale * (double)w[i];
    return 0;
}

/* y = W v for an fp64 input vector (dequantized rows, fp64 sums). */
static void gemv_f64_dvec(int type, const uint8_t *w, const double *v, double *y, int inner,
                          int outer)
{
    const deq_fn f = deq_for(type);
    const int be = orc_block_elems(type), bb = orc_block_bytes(type);
    const int nb = inner / be;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < outer; ++r) {
        float blk[256];
        double acc = 0.0;
        for (int b = 0; b < nb; ++b) {
            f(w + ((size_t)r * nb + b) * bb, blk);
            for (int i = 0; i < be; ++i)
                acc += (double)blk[i] * v[(size_t)b * be + i];
        }
        y[r] = acc;
    }
}

/* The MLP half of a decoder layer, src/ModelCPU.jl:913-920, in fp64:
 * n = rmsnorm(x) .* nw, h = silu(Wg n) * (Wu n), y = x + Wd h. */
int orc_ffn_block_f64(int gate_type, const uint8_t *wg, int up_type, const uint8_t *wu,
                      int down_type, const uint8_t *wd, const float *x, const float *nw,
                      float eps, int hidden, int inter, double *n, double *g, double *u,
                      double *h, double *y)
{
    if (check_dims(gate_type, hidden, inter) || check_dims(up_type, hidden, inter) ||
        check_dims(down_type, inter, hidden))
        return -1;
    if (orc_rmsnorm_f64(x, nw, eps, hidden, n))
        return -1;
    gemv_f64_dvec(gate_type, wg, n, g, hidden, inter);
    gemv_f64_dvec(up_type, wu, n, u, hidden, inter);
    for (int i = 0; i < inter; ++i)
        h[i] = g[i] / (1.0 + exp(-g[i])) * u[i];
    gemv_f64_dvec(down_type, wd, h, y, inter, hidden);
    for (int r = 0; r < hidden; ++r)
        y[r] += (double)x[r];
    return 0;
}

/* ------------------------------------------------------------------ */
/* The reference C int8-activation path                                  */
/* ------------------------------------------------------------------ */
/* Q8_K block (src/kernels/quant_kernels.c:52-56): float d at 0, int8 qs[256]
 * at 4, int16 bsums[16] at 260; 292 bytes. */
#define Q8K_BYTES 292

/* quant_kernels.c:166-194: per 256 values amax = max|x|, d = amax/127,
 * id = d ? 1/d : 0, q = (int8) roundf(x*id) (half away from zero),
 * bsums = sums of 16 consecutive q. */
int orc_quantize_row_q8k(const float *x, uint8_t *q8, int64_t k)
{
    if (k < 0 || k % 256)
        return -1;
    for (int64_t i = 0; i < k / 256; ++i) {
        const float *src = x + i * 256;
        uint8_t *blk = q8 + i * Q8K_BYTES;
        float amax = 0.0f;
        for (int j = 0; j < 256; ++j) {
            const float ax = fabsf(src[j]);
            if (ax > amax)
                amax = ax;
        }
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        memcpy(blk, &d, 4);
        int8_t *qs = (int8_t *)(blk + 4);
        for (int g = 0; g < 16; ++g) {
            int sum = 0;
            for (int l = 0; l < 16; ++l) {
                const int8_t q = (int8_t)roundf(src[16 * g + l] * id);
                qs[16 * g + l] = q;
                sum += q;
            }
            const int16_t s16 = (int16_t)sum;
            memcpy(blk + 260 + 2 * g, &s16, 2);
        }
    }
    return 0;
}

static inline float q8k_d(const uint8_t *blk) { float d; memcpy(&d, blk, 4); return d; }
static inline int16_t q8k_bsum(const uint8_t *blk, int g)
{
    int16_t s;
    memcpy(&s, blk + 260 + 2 * g, 2);
    return s;
}

/* The AVX2 horizontal sums (quant_kernels.c:91-98, 274-275). */
static inline float hsum8(const float a[8])
{
    const float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
    return (s0 + s2) + (s1 + s3);
}
static inline float hsum4(const float a[4]) { return (a[0] + a[2]) + (a[1] + a[3]); }

/* 8 sc followed by 8 m, sub-block order (the utmp unpack at :221-226). */
static void k_unpack16(const uint8_t *s, unsigned out[16])
{
    for (int i = 0; i < 8; ++i)
        k_scale_min(s, i, &out[i], &out[8 + i]);
}

/* vec_dot_q4_K_q8_K, AVX2 branch :212-277.  Integer lane t (0..7) of sumi
 * holds bytes 4t..4t+3 of every 32-byte qs chunk. */
static float dot_q4k_q8k(const uint8_t *x, const uint8_t *y, int nb)
{
    float acc[8] = {0}, accm[4] = {0};
    for (int i = 0; i < nb; ++i) {
        const uint8_t *bx = x + (size_t)i * 144, *by = y + (size_t)i * Q8K_BYTES;
        const float yd = q8k_d(by);
        const float d = yd * orc_half_to_float(rd16(bx));
        const float dmin = -yd * orc_half_to_float(rd16(bx + 2));
        unsigned sm[16];
        k_unpack16(bx + 4, sm);
        const int8_t *q8 = (const int8_t *)(by + 4);
        int q8s[8];
        for (int k = 0; k < 8; ++k)
            q8s[k] = (int16_t)(q8k_bsum(by, 2 * k) + q8k_bsum(by, 2 * k + 1));
        for (int k = 0; k < 4; ++k) {
            const int prod = (int)sm[8 + 2 * k] * q8s[2 * k] + (int)sm[8 + 2 * k + 1] * q8s[2 * k + 1];
            accm[k] = fmaf(dmin, (float)prod, accm[k]);
        }
        int sumi[8] = {0};
        const uint8_t *q4 = bx + 16;
        for (int j = 0; j < 4; ++j) {
            for (int t = 0; t < 8; ++t) {
                int pl = 0, ph = 0;
                for (int b = 4 * t; b < 4 * t + 4; ++b) {
                    pl += (q4[32 * j + b] & 0x0f) * q8[64 * j + b];
                    ph += (q4[32 * j + b] >> 4) * q8[64 * j + 32 + b];
                }
                sumi[t] += (int)sm[2 * j] * pl + (int)sm[2 * j + 1] * ph;
            }
        }
        for (int t = 0; t < 8; ++t)
            acc[t] = fmaf(d, (float)sumi[t], acc[t]);
    }
    return hsum8(acc) + hsum4(accm);
}

/* vec_dot_q5_K_q8_K, AVX2 branch :319-397.  The min term is reduced to one
 * integer and folded as `summs += dmin * isum`, which gcc contracts to an
 * FMA under its default -ffp-contract=fast with -mfma. */
static float dot_q5k_q8k(const uint8_t *x, const uint8_t *y, int nb)
{
    float acc[8] = {0};
    float summs = 0.0f;
    for (int i = 0; i < nb; ++i) {
        const uint8_t *bx = x + (size_t)i * 176, *by = y + (size_t)i * Q8K_BYTES;
        const float yd = q8k_d(by);
        const float d = yd * orc_half_to_float(rd16(bx));
        const float dmin = -yd * orc_half_to_float(rd16(bx + 2));
        unsigned sm[16];
        k_unpack16(bx + 4, sm);
        const int8_t *q8 = (const int8_t *)(by + 4);
        int isum = 0;
        for (int k = 0; k < 8; ++k) {
            const int s = (int16_t)(q8k_bsum(by, 2 * k) + q8k_bsum(by, 2 * k + 1));
            isum += (int)sm[8 + k] * s;
        }
        summs = fmaf(dmin, (float)isum, summs);
        const uint8_t *qh = bx + 16, *q5 = bx + 48;
        int sumi[8] = {0};
        for (int j = 0; j < 4; ++j) {
            for (int t = 0; t < 8; ++t) {
                int p0 = 0, p1 = 0;
                for (int b = 4 * t; b < 4 * t + 4; ++b) {
                    const int lo = (q5[32 * j + b] & 0x0f) + (((qh[b] >> (2 * j)) & 1) << 4);
                    const int hi = (q5[32 * j + b] >> 4) + (((qh[b] >> (2 * j + 1)) & 1) << 4);
                    p0 += lo * q8[64 * j + b];
                    p1 += hi * q8[64 * j + 32 + b];
                }
                sumi[t] += (int)sm[2 * j] * p0 + (int)sm[2 * j + 1] * p1;
            }
        }
        for (int t = 0; t < 8; ++t)
            acc[t] = fmaf(d, (float)sumi[t], acc[t]);
    }
    return hsum8(acc) + summs;
}

/* vec_dot_q6_K_q8_K, AVX2 branch :444-521.  Lanes 0..3 of each 32-element
 * group use scale 2g, lanes 4..7 use 2g+1. */
static float dot_q6k_q8k(const uint8_t *x, const uint8_t *y, int nb)
{
    float acc[8] = {0};
    for (int i = 0; i < nb; ++i) {
        const uint8_t *bx = x + (size_t)i * 210, *by = y + (size_t)i * Q8K_BYTES;
        const float d = q8k_d(by) * orc_half_to_float(rd16(bx + 208));
        const uint8_t *ql = bx, *qh = bx + 128;
        const int8_t *sc = (const int8_t *)(bx + 192);
        const int8_t *q8 = (const int8_t *)(by + 4);
        int sumi[8] = {0};
        for (int j = 0; j < 2; ++j) {
            for (int k = 0; k < 4; ++k) {
                for (int t = 0; t < 8; ++t) {
                    int p = 0;
                    for (int b = 4 * t; b < 4 * t + 4; ++b) {
                        const unsigned lbyte = ql[64 * j + 32 * (k & 1) + b];
                        const unsigned lo = (k < 2) ? (lbyte & 0x0fu) : (lbyte >> 4);
                        const unsigned hb = (qh[32 * j + b] >> (2 * k)) & 3u;
                        const int q = (int)(lo | (hb << 4)) - 32;
                        p += q * q8[128 * j + 32 * k + b];
                    }
                    const int s = sc[2 * (4 * j + k) + (t >= 4)];
                    sumi[t] += s * p;
                }
            }
        }
        for (int t = 0; t < 8; ++t)
            acc[t] = fmaf(d, (float)sumi[t], acc[t]);
    }
    return hsum8(acc);
}

/* q{4,5,6}_k_gemv drivers, quant_kernels.c:602-650: quantize x once, then
 * one dot per row. */
int orc_gemv_q8k(int type, const uint8_t *w, const float *x, float *out,
                 uint8_t *q8, int inner, int outer)
{
    if (type != ORC_Q4_K && type != ORC_Q5_K && type != ORC_Q6_K)
        return -1;
    if (check_dims(type, inner, outer))
        return -1;
    const int nb = inner / 256, bb = orc_block_bytes(type);
    orc_quantize_row_q8k(x, q8, inner);
#pragma omp parallel for schedule(static)
    for (int r = 0; r < outer; ++r) {
        const uint8_t *row = w + (size_t)r * nb * bb;
        float v;
        if (type == ORC_Q4_K)
            v = dot_q4k_q8k(row, q8, nb);
        else if (type == ORC_Q5_K)
            v = dot_q5k_q8k(row, q8, nb);
        else
            v = dot_q6k_q8k(row, q8, nb);
        out[r] = v;
    }
    return 0;
}

/* q8_0_gemv AVX2 branch, quant_kernels.c:664-683: per 8 elements
 * prod = float(q)*x (rounded), acc = fma(d, prod, acc), lane t = element
 * j+t; hsum at the end of the row. */
int orc_gemv_q8_0_lanes(const uint8_t *w, const float *x, float *out,
                        int inner, int outer)
{
    if (check_dims(ORC_Q8_0, inner, outer))
        return -1;
    const int nb = inner / 32;
    for (int r = 0; r < outer; ++r) {
        float acc[8] = {0};
        for (int b = 0; b < nb; ++b) {
            const uint8_t *blk = w + ((size_t)r * nb + b) * 34;
            const float d = orc_half_to_float(rd16(blk));
            for (int j = 0; j < 32; j += 8)
                for (int t = 0; t < 8; ++t) {
                    const float prod = (float)(int8_t)blk[2 + j + t] * x[32 * b + j + t];
                    acc[t] = fmaf(d, prod, acc[t]);
                }
        }
        out[r] = hsum8(acc);
    }
    return 0;
}
