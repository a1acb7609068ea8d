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
// y = W (rmsnorm(x) .* nw) in one launch (the wide kernels' folded norm, per
// workgroup or persistent by row count) for Q4_K / Q5_K rows of at most 16
// blocks; hipErrorNotSupported otherwise.
bool gemv_norm_fusable(int type, int inner, int outer);
hipError_t launch_gemv_norm(int type, const void *w, const float *x, const float *nw, float eps,
                            float *y, int inner, int outer, hipStream_t s);
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

// CUs of the current device (queried once per device)
int device_cus();

// kq_prefill.hip
// The prefill GEMM addresses its operands as 32-bit byte offsets from the
// start of Xh (T x inner fp16) and W (outer Q4_K rows), and counts its
// output tiles in ints.
inline bool prefill_fits(int T, int inner, int outer)
{
    return 2 * (int64_t)T * inner <= (int64_t)UINT32_MAX &&
           (int64_t)outer * (inner / 256) * 144 <= (int64_t)UINT32_MAX &&
           (int64_t)T * outer <= (int64_t)INT32_MAX; // tile counts stay ints
}
// Rows of at most this many columns run in the fp32 kernel (k_prefill_q4k_f32).
constexpr int kPrefillF32MaxK = 512;
// Longer rows of at most this many columns take fp16 weights rounded once
// from their exact values (k_prefill_q4k<true>).
constexpr int kPrefillExactWMaxK = 2048;
// The caller's scratch xh: the fp16 activations (T x inner), one int per
// token (its power-of-two scale) from the next 16-byte boundary, then, from
// the next 16-byte boundary, the partial sums of a split over K.  A split
// keeps nsplit x (64-token x 128-row tiles) <= kPrefillMaxTiles, so its
// nsplit - 1 partial planes of T x outer floats hold at most
// T x 128 x kPrefillMaxTiles / ceil(T / 64) floats whatever outer is.
constexpr int kPrefillMaxTiles = 256;
constexpr int kPrefillBM = 64, kPrefillBN = 128; // workgroup tile: tokens x weight rows
inline size_t prefill_scale_offset(int T, int inner)
{
    return ((size_t)2 * (size_t)T * (size_t)inner + 15) & ~(size_t)15;
}
inline size_t prefill_part_offset(int T, int inner)
{
    return (prefill_scale_offset(T, inner) + (size_t)4 * (size_t)T + 15) & ~(size_t)15;
}
inline size_t prefill_part_floats(int T)
{
    const size_t mtiles = ((size_t)T + kPrefillBM - 1) / kPrefillBM;
    return (size_t)T * kPrefillBN * (size_t)kPrefillMaxTiles / mtiles;
}
// XCD-aware order: workgroup bid's place `lin` in tile order, so that the
// consecutive workgroups of one XCD (bid mod 8) take consecutive places and
// share the operand bytes of those tiles in their L2 (tile order below).
// The grid is prefill_grid workgroups; lin >= tiles x nsplit exits.
__host__ __device__ inline int prefill_grid(int tiles, int nsplit)
{
    return (tiles * nsplit + 7) / 8 * 8;
}
__host__ __device__ inline int prefill_lin(int bid, int tiles, int nsplit)
{
    const int per_xcd = (tiles * nsplit + 7) / 8;
    return (bid % 8) * per_xcd + bid / 8;
}
// Workgroup `lin` (in tile order) of a launch of mtiles x ntiles tiles and
// nsplit splits over K: its split, its tile and the split's block columns
// kb0 .. kb0 + nk - 1 of the nblk.  Tile order within a split: groups of
// kPrefillGroupM M tiles (token bands), the group's M tiles fastest, then N.
// An XCD's 32 consecutive tiles at 512 tokens are then 4 token bands x 8
// weight bands, 2 MB of fp16 activations and 2.4 MB of weight blocks per
// 4 MB L2, where all 8 token bands of 4 weight bands (M fastest over all of
// them) need 4 MB + 1.2 MB.  Measured on MI355X (us per call, stream
// launches, two runs each, interleaved): 512 x 4096 x 4096 30.5 against
// 31.4-31.5, 512 x 14336 x 4096 102.8-103.0 against 104.7-105.0, 512 x 4096
// x 14336 84.1-84.6 against 84.4-84.9; groups of 2 M tiles were no better at
// 512 tokens and 0.7 us slower at 256 (2 x 16 bands per XCD).
constexpr int kPrefillGroupM = 4;
struct PrefillSplit {
    int sp, mt, nt, kb0, nk;
};
__host__ __device__ inline PrefillSplit prefill_split_of(int lin, int mtiles, int ntiles, int nblk,
                                                        int nsplit)
{
    PrefillSplit s;
    const int tiles = mtiles * ntiles;
    s.sp = lin / tiles;
    const int tl = lin - s.sp * tiles;
    const int g = tl / (kPrefillGroupM * ntiles);
    const int gm = mtiles - kPrefillGroupM * g < kPrefillGroupM ? mtiles - kPrefillGroupM * g : kPrefillGroupM;
    const int idx = tl - g * kPrefillGroupM * ntiles;
    s.mt = kPrefillGroupM * g + idx % gm;
    s.nt = idx / gm;
    s.kb0 = s.sp * nblk / nsplit;
    s.nk = (s.sp + 1) * nblk / nsplit - s.kb0;
    return s;
}
inline size_t prefill_scratch_bytes(int T, int inner)
{
    return prefill_part_offset(T, inner) + 4 * prefill_part_floats(T);
}
// Splits over K of one prefill launch on a device of ncu CUs (1: none).  A
// weight of few rows leaves most CUs without a tile (512 x 512 x 4096 is 32
// tiles for 256 CUs), so each tile's block columns are shared out over
// nsplit workgroups, as many as keep nsplit x tiles within the CUs (and
// within the partial planes the scratch holds) and at least two columns per
// split, and a second launch adds the partial sums.  Rows of fewer than 8
// block columns are not split: a workgroup's fixed cost (the launch, the
// first copies, the partial-sum exchange and the 32 KB of stores) is then
// most of its time, and the summing launch adds to it (measured on MI355X,
// us per call: 512 x 512 x 4096 18.9-21.4 against 27.6 unsplit, 64 x 4096 x
// 4096 18.9-19.3 against 23.9, 512 x 2048 x 4096 25.5-25.8 against 28.1;
// 512 x 1024 x 1024 split four ways 18.2-19.0 against 13.0).
inline int prefill_splits(int T, int inner, int outer, int ncu)
{
    const int mtiles = (T + kPrefillBM - 1) / kPrefillBM, ntiles = (outer + kPrefillBN - 1) / kPrefillBN;
    const int tiles = mtiles * ntiles, nblk = inner / 256;
    const int cap = ncu < kPrefillMaxTiles ? ncu : kPrefillMaxTiles;
    if (tiles * 2 > cap || nblk < 8)
        return 1;
    const int s = cap / tiles < nblk / 2 ? cap / tiles : nblk / 2;
    return s > 1 ? s : 1;
}
hipError_t launch_prefill_q4k(const void *w, const float *X, void *xh, float *Y, int T,
                              int inner, int outer, hipStream_t s);
// Its two halves for rows of more than kPrefillF32MaxK columns: X rounded into
// xh (fp16 rows and one scale exponent per token), then the product from xh
// (which also takes the partial sums of a split over K, leaving the rounded
// rows as they were), so several weights can share one rounding.
hipError_t launch_prefill_convert(const float *X, void *xh, int T, int inner, hipStream_t s);
hipError_t launch_prefill_gemm(const void *w, void *xh, float *Y, int T, int inner, int outer,
                               hipStream_t s);
// The same product on fp32 operands (k_prefill_q4k_f32), any inner; needs
// T * outer <= INT32_MAX.
hipError_t launch_prefill_q4k_f32(const void *w, const float *X, float *Y, int T, int inner,
                                  int outer, hipStream_t s);

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
