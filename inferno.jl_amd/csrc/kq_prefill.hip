// kq_prefill.hip -- batched prefill GEMM on gfx950 matrix cores:
//   Y[t, n] = sum_k W[n, k] * X[t, k],  W: N x K Q4_K,  X: T x K fp32.
//
// The reference has no GEMM here: src/ModelCPU.jl:1001-1017 (Inferno.jl)
// runs T independent GEMVs, so the semantics are the Q4_K GEMV applied row
// by row.  On MI355X the T tokens share every weight byte, which makes this
// a dense contraction: X is rounded once to fp16 (the matrix-core operand
// type; fp16 keeps the 1e-4*||w||*||x|| bound where bf16 does not), each
// token row on its own power-of-two scale (k_x_to_f16), and
// v_mfma_f32_32x32x16_f16 accumulates in fp32.  A dot product over fp16
// operands errs by about 2.8e-4 ||w|| ||x|| / sqrt(K) on random data, so short
// rows need more care: rows of at most 512 columns, and the fp32-operand
// entry point, run k_prefill_q4k_f32 (below); rows of at most 2048 columns
// round each weight once from its exact value (k_prefill_q4k<true>) instead
// of through fp16 sub-block scales.
//
// Tile: 64 tokens x 128 weight rows per workgroup of 8 waves (256
// workgroups at 512 x 4096 x 4096).  Both operands of one Q4_K block column
// (256 k: 32 KB of fp16 activations, 18 KB of weight blocks) stream through
// a three-slot LDS ring filled by direct-to-LDS 128-bit copies: while a wave
// reduces column kb from registers it reads column kb + 1 out of the ring,
// and the copies of columns kb + 2 and kb + 3 are in flight.  Wave (rh, j)
// reduces weight rows 64 rh .. 64 rh + 63 of the tile over sub-block pair j
// of every column, dequantizing its matrix-core operand straight from the
// block bytes into registers (every weight is dequantized once per
// workgroup; the two lane halves decode one row's scales each).  The weights are the A operand, so each
// lane ends with 4 consecutive output rows of one token: the four K-quarter
// partial sums meet in LDS and leave as 16-byte stores.
#include "kq_common.h"
#include "kq_launch.h"

namespace ihip {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int PF_BM = kPrefillBM, PF_BN = kPrefillBN; // workgroup tile: tokens x weight rows

// One token row of X to fp16 (one workgroup per row, 8 values per thread and
// step: two 16-byte loads, one 16-byte store).  The reference multiplies fp32
// activations of any finite size (src/ModelCPU.jl:285-307), while fp16 holds
// magnitudes up to 65504 only and rounds those below 2^-14 to its subnormal
// steps.  So every row is scaled by a power of two 2^s, chosen so that its
// largest magnitude lands in [2^14, 2^15), before the rounding, and s goes to
// xs[t]; the GEMM's epilogue multiplies the row's outputs by 2^-s, which is
// exact.  Every value keeps fp16's 11 significant bits down to 2^-29 of the
// row's maximum.  A row holding NaN or an infinity is converted unscaled
// (s = 0), so the non-finite value reaches its outputs.  Rows of at most
// 8192 values stay in registers between the maximum and the conversion;
// longer rows are read twice.
constexpr int PF_CVT_REG = 4; // 8-value steps a thread holds: 256 x 8 x 4 = 8192 values
__global__ __launch_bounds__(256) void k_x_to_f16(const float *__restrict__ X,
                                                  _Float16 *__restrict__ Xh, int *__restrict__ xs,
                                                  int K)
{
    __shared__ uint32_t wmax[4];
    const int t = blockIdx.x, tid = threadIdx.x;
    const float *row = X + (size_t)t * K;
    _Float16 *hrow = Xh + (size_t)t * K;
    // |x| bits of eight values: NaN > +Inf > every finite value
    auto absmax8 = [](float4 a, float4 b) {
        const uint32_t m0 = max(__float_as_uint(a.x) & 0x7fffffffu, __float_as_uint(a.y) & 0x7fffffffu);
        const uint32_t m1 = max(__float_as_uint(a.z) & 0x7fffffffu, __float_as_uint(a.w) & 0x7fffffffu);
        const uint32_t m2 = max(__float_as_uint(b.x) & 0x7fffffffu, __float_as_uint(b.y) & 0x7fffffffu);
        const uint32_t m3 = max(__float_as_uint(b.z) & 0x7fffffffu, __float_as_uint(b.w) & 0x7fffffffu);
        return max(max(m0, m1), max(m2, m3));
    };
    const bool in_regs = K <= 256 * 8 * PF_CVT_REG; // workgroup-uniform
    float4 v[PF_CVT_REG][2];
    uint32_t m = 0;
    if (in_regs) {
#pragma unroll
        for (int k = 0; k < PF_CVT_REG; ++k) {
            const int i = 8 * (tid + 256 * k);
            v[k][0] = v[k][1] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (i < K) { // K is a multiple of 256: whole 8-value steps
                v[k][0] = *reinterpret_cast<const float4 *>(row + i);
                v[k][1] = *reinterpret_cast<const float4 *>(row + i + 4);
            }
            m = max(m, absmax8(v[k][0], v[k][1]));
        }
    } else {
        for (int i = 8 * tid; i < K; i += 8 * 256)
            m = max(m, absmax8(*reinterpret_cast<const float4 *>(row + i),
                               *reinterpret_cast<const float4 *>(row + i + 4)));
    }
    // the row's maximum: DPP steps within each row of 16 lanes, then the
    // four rows' and the four waves' values through LDS
    m = dpp_max_u32<0xb1, 0xf>(m);
    m = dpp_max_u32<0x4e, 0xf>(m);
    m = dpp_max_u32<0x141, 0xf>(m);
    m = dpp_max_u32<0x140, 0xf>(m);
    {
        const int lane = tid & 63, w = tid >> 6;
        const uint32_t r0 = __builtin_amdgcn_readlane(m, 0), r1 = __builtin_amdgcn_readlane(m, 16);
        const uint32_t r2 = __builtin_amdgcn_readlane(m, 32), r3 = __builtin_amdgcn_readlane(m, 48);
        if (lane == 0)
            wmax[w] = max(max(r0, r1), max(r2, r3));
    }
    __syncthreads();
    m = max(max(wmax[0], wmax[1]), max(wmax[2], wmax[3]));
    const bool finite = m < 0x7f800000u;
    // m = 0 (an all-zero row): frexp's exponent is 0, any scale keeps the zeros
    const int s = finite ? 15 - __builtin_amdgcn_frexp_expf(__uint_as_float(m)) : 0;
    auto cvt8 = [s](float4 a, float4 b) {
        half8 h;
        h[0] = (_Float16)__builtin_ldexpf(a.x, s); h[1] = (_Float16)__builtin_ldexpf(a.y, s);
        h[2] = (_Float16)__builtin_ldexpf(a.z, s); h[3] = (_Float16)__builtin_ldexpf(a.w, s);
        h[4] = (_Float16)__builtin_ldexpf(b.x, s); h[5] = (_Float16)__builtin_ldexpf(b.y, s);
        h[6] = (_Float16)__builtin_ldexpf(b.z, s); h[7] = (_Float16)__builtin_ldexpf(b.w, s);
        return h;
    };
    if (in_regs) {
#pragma unroll
        for (int k = 0; k < PF_CVT_REG; ++k) {
            const int i = 8 * (tid + 256 * k);
            if (i < K)
                *reinterpret_cast<half8 *>(hrow + i) = cvt8(v[k][0], v[k][1]);
        }
    } else {
        for (int i = 8 * tid; i < K; i += 8 * 256)
            *reinterpret_cast<half8 *>(hrow + i) = cvt8(*reinterpret_cast<const float4 *>(row + i),
                                                        *reinterpret_cast<const float4 *>(row + i + 4));
    }
    if (tid == 0)
        xs[t] = s;
}

// One ring slot holds block column kb of both operands:
//  * activations, 64 token rows x 512 bytes: row m holds 32 chunks of 16
//    bytes, chunk c at slot c ^ (m & 15), so that the 16 lanes of a 128-bit
//    read (same chunk, consecutive rows) hit distinct banks;
//  * weights, 128 rows x 144 bytes: the rows' Q4_K blocks of column kb.
constexpr int PF_ROW_BYTES = 512;
constexpr int PF_A_STAGE = PF_BM * PF_ROW_BYTES; // 32 KB
constexpr int PF_B_STAGE = PF_BN * 144;          // 18 KB
constexpr int PF_SLOT = PF_A_STAGE + PF_B_STAGE; // 50 KB
constexpr int PF_NSLOT = 3;
constexpr int PF_THREADS = 512;                  // 8 waves
constexpr int PF_B_COPIES = PF_B_STAGE / 1024;   // 18 wave copies of 1 KB

static_assert(PF_B_STAGE % 1024 == 0, "weight stage is whole wave copies");
static_assert(PF_NSLOT * PF_SLOT <= 160 * 1024, "ring fits the 160 KB of LDS");

// One direct-to-LDS copy: lane l's 16 bytes at base + off land at LDS byte
// lds + 16 l.  The base is wave-uniform (scalar registers) and the lane's
// offset a 32-bit register, so a column's copies cost no vector address
// arithmetic.  Written as inline assembly so that the compiler, which would
// otherwise make every later LDS read wait for all copies in flight
// (including those issued ahead for later block columns), leaves the waits to
// the explicit per-wave s_waitcnt of the main loop.
__device__ __forceinline__ void pf_copy16(const void *base, uint32_t off, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(off), "s"(base), "s"(lds)
                 : "memory", "m0");
}

// Per-lane byte offsets of the copies of block column 0 (from Xh and from W);
// column kb adds 512 kb bytes (activations) or 144 kb bytes (weights) to the
// wave-uniform base.  Wave w issues activation
// copies w, w + 8, w + 16, w + 24 (64 chunks each: chunk q = stage row q / 32,
// activation chunk (q % 32) ^ (row & 15)) and weight copies w, w + 8 and, for
// w < 2, w + 16 (chunk q = tile row q / 9, 16-byte piece q % 9): 7 copies for
// waves 0-1, 6 for the others.  Rows past T (tokens) or N (weights) re-read
// the last row.
struct PfSrc {
    uint32_t a0, a1, a2, a3, b0, b1, b2; // plain members: kept in registers
};

__device__ __forceinline__ uint32_t pf_src_a(int m0, int T, int K, int w, int lane, int k)
{
    const int q = (8 * k + w) * 64 + lane;
    const int rp = q >> 5, c = (q & 31) ^ (rp & 15);
    return 2u * ((uint32_t)min(m0 + rp, T - 1) * (uint32_t)K + 8u * (uint32_t)c);
}

__device__ __forceinline__ uint32_t pf_src_b(int n0, int N, uint32_t row_bytes, int lane, int i)
{
    const int q = 64 * min(i, PF_B_COPIES - 1) + lane;
    const int row = q / 9, piece = q - 9 * row;
    return (uint32_t)min(n0 + row, N - 1) * row_bytes + 16u * (uint32_t)piece;
}

// Issue this wave's copies of block column kb into the ring slot at LDS
// address `slot`.
__device__ __forceinline__ void pf_issue(const PfSrc &S, const uint8_t *Xb, const uint8_t *W, int kb,
                                         int w, uint32_t slot)
{
    const uint8_t *xa = Xb + (size_t)kb * 512, *wb = W + (size_t)kb * 144;
    pf_copy16(xa, S.a0, slot + 1024 * w);
    pf_copy16(xa, S.a1, slot + 1024 * (w + 8));
    pf_copy16(xa, S.a2, slot + 1024 * (w + 16));
    pf_copy16(xa, S.a3, slot + 1024 * (w + 24));
    pf_copy16(wb, S.b0, slot + PF_A_STAGE + 1024 * w);
    pf_copy16(wb, S.b1, slot + PF_A_STAGE + 1024 * (w + 8));
    if (w + 16 < PF_B_COPIES) // wave-uniform
        pf_copy16(wb, S.b2, slot + PF_A_STAGE + 1024 * (w + 16));
}

// 8 nibbles (the low or high nibble of 8 bytes) -> 8 fp16 weights
// q * dsc - dmm.  A byte 0000qqqq is the OCP e4m3 encoding of q * 2^-9; the
// scaled convert multiplies by 2^9, giving q exactly in fp16, and one packed
// fp16 FMA per pair applies the sub-block scale and min.
__device__ __forceinline__ half8 pf_dequant8(uint2 bytes, bool high, half2v dsc, half2v dmm)
{
    uint32_t w0 = bytes.x, w1 = bytes.y;
    if (high) {
        w0 >>= 4;
        w1 >>= 4;
    }
    w0 &= 0x0f0f0f0fu;
    w1 &= 0x0f0f0f0fu;
    const half2v q01 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 512.0f, false);
    const half2v q23 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 512.0f, true);
    const half2v q45 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 512.0f, false);
    const half2v q67 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 512.0f, true);
    const half2v r01 = __builtin_elementwise_fma(q01, dsc, dmm);
    const half2v r23 = __builtin_elementwise_fma(q23, dsc, dmm);
    const half2v r45 = __builtin_elementwise_fma(q45, dsc, dmm);
    const half2v r67 = __builtin_elementwise_fma(q67, dsc, dmm);
    half8 r;
    r[0] = r01[0]; r[1] = r01[1]; r[2] = r23[0]; r[3] = r23[1];
    r[4] = r45[0]; r[5] = r45[1]; r[6] = r67[0]; r[7] = r67[1];
    return r;
}

// The same 8 weights rounded once from their exact fp32 values,
// rn16((d sc) q - dmin m): q exact in fp32 from the scaled convert, one fp32
// FMA (d sc q is exact, so the FMA rounds only the difference), then
// v_cvt_pk_f16_f32.  Rounding d sc and dmin m to fp16 first, as
// pf_dequant8 does, puts one shared relative error on all 32 weights of a
// sub-block; this form leaves each weight its own.
__device__ __forceinline__ half8 pf_dequant8_exact(uint2 bytes, bool high, float dsc, float dmm)
{
    typedef float f2v __attribute__((ext_vector_type(2)));
    uint32_t w0 = bytes.x, w1 = bytes.y;
    if (high) {
        w0 >>= 4;
        w1 >>= 4;
    }
    w0 &= 0x0f0f0f0fu;
    w1 &= 0x0f0f0f0fu;
    const f2v q01 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w0, 512.0f, false);
    const f2v q23 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w0, 512.0f, true);
    const f2v q45 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w1, 512.0f, false);
    const f2v q67 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w1, 512.0f, true);
    const f2v r01 = {fmaf(q01[0], dsc, dmm), fmaf(q01[1], dsc, dmm)};
    const f2v r23 = {fmaf(q23[0], dsc, dmm), fmaf(q23[1], dsc, dmm)};
    const f2v r45 = {fmaf(q45[0], dsc, dmm), fmaf(q45[1], dsc, dmm)};
    const f2v r67 = {fmaf(q67[0], dsc, dmm), fmaf(q67[1], dsc, dmm)};
    const half2v h01 = __builtin_convertvector(r01, half2v), h23 = __builtin_convertvector(r23, half2v);
    const half2v h45 = __builtin_convertvector(r45, half2v), h67 = __builtin_convertvector(r67, half2v);
    half8 r;
    r[0] = h01[0]; r[1] = h01[1]; r[2] = h23[0]; r[3] = h23[1];
    r[4] = h45[0]; r[5] = h45[1]; r[6] = h67[0]; r[7] = h67[1];
    return r;
}

// One column's operands of this lane, read from a ring slot: 2 x 8 quant
// bytes of weight rows `blk0` / `blk1` (rows li and li + 32 of the wave's 64)
// for sub-block pair j, the block header of row li + 32 h only (the two lane
// halves decode one row's scales each and exchange them), and the 16-byte
// fp16 activation chunks of tokens li and li + 32 for the four 16-wide K
// steps (k = 64j + 16s + 8h + (0..7), chunk 8j + 2s + h).
struct PfOps {
    uint4 hd;
    uint2 q0[2], q1[2];
    half8 x[4][2];
};

__device__ __forceinline__ void pf_read(const uint8_t *sa, const uint8_t *blk0, const uint8_t *blk1,
                                        int j, int h, int li, PfOps &o)
{
    o.hd = *reinterpret_cast<const uint4 *>(h ? blk1 : blk0);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const uint8_t *blk = u ? blk1 : blk0;
        o.q0[u] = *reinterpret_cast<const uint2 *>(blk + 16 + 32 * j + 8 * h);
        o.q1[u] = *reinterpret_cast<const uint2 *>(blk + 16 + 32 * j + 16 + 8 * h);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int m = 32 * t + li, c = 8 * j + 2 * s + h;
            o.x[s][t] = *reinterpret_cast<const half8 *>(sa + m * PF_ROW_BYTES + 16 * (c ^ (m & 15)));
        }
}

// Dequantize the column's weights into matrix-core operands and accumulate.
// acc[u][t] is the 32 x 32 tile (weight rows 32u.., tokens 32t..): lane l,
// register r hold token 32t + l % 32, weight row 32u + 8 (r / 4) + 4 (l / 32) + r % 4.
// EXACTW: each weight rounded once from its exact value (pf_dequant8_exact),
// for rows of at most kPrefillExactWMaxK columns, where the shared rounding
// of a sub-block's scale averages over too few sub-blocks.
template <bool EXACTW>
__device__ __forceinline__ void pf_mma(const PfOps &o, int j, float16v (&acc)[2][2])
{
    // Scale d*sc and min -dmin*m of sub-blocks 2j (A) and 2j + 1 (B) for
    // this lane half's row (rounded once to fp16 and packed (A, B), or kept
    // in fp32 when EXACTW) ...
    const float d = h2f(o.hd.x & 0xffffu), dmin = h2f(o.hd.x >> 16);
    float scA, mA, scB, mB;
    k_scale_min_pair(o.hd.y, o.hd.z, o.hd.w, j, scA, mA, scB, mB);
    // ... then exchanged between the lane halves: v_permlane32_swap of a
    // register with itself leaves lanes 0-31's value (row li) in the first
    // result and lanes 32-63's (row li + 32) in the second, in every lane.
    if constexpr (EXACTW) {
        const float dsa = d * scA, dsb = d * scB, dma = -(dmin * mA), dmb = -(dmin * mB);
        const auto xa = __builtin_amdgcn_permlane32_swap(__float_as_uint(dsa), __float_as_uint(dsa), false, false);
        const auto xb = __builtin_amdgcn_permlane32_swap(__float_as_uint(dsb), __float_as_uint(dsb), false, false);
        const auto ya = __builtin_amdgcn_permlane32_swap(__float_as_uint(dma), __float_as_uint(dma), false, false);
        const auto yb = __builtin_amdgcn_permlane32_swap(__float_as_uint(dmb), __float_as_uint(dmb), false, false);
        float dsA[2], dmA[2], dsB[2], dmB[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            dsA[u] = __uint_as_float((uint32_t)xa[u]);
            dsB[u] = __uint_as_float((uint32_t)xb[u]);
            dmA[u] = __uint_as_float((uint32_t)ya[u]);
            dmB[u] = __uint_as_float((uint32_t)yb[u]);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const half8 wq = pf_dequant8_exact((s & 1) ? o.q1[u] : o.q0[u], s >= 2,
                                                   s >= 2 ? dsB[u] : dsA[u], s >= 2 ? dmB[u] : dmA[u]);
#pragma unroll
                for (int t = 0; t < 2; ++t)
                    acc[u][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wq, o.x[s][t], acc[u][t], 0, 0, 0);
            }
    } else {
        const half2v ds = {(_Float16)(d * scA), (_Float16)(d * scB)};
        const half2v dm = {(_Float16)(-(dmin * mA)), (_Float16)(-(dmin * mB))};
        const uint32_t dsu = __builtin_bit_cast(uint32_t, ds), dmu = __builtin_bit_cast(uint32_t, dm);
        const auto xs = __builtin_amdgcn_permlane32_swap(dsu, dsu, false, false);
        const auto xm = __builtin_amdgcn_permlane32_swap(dmu, dmu, false, false);
        half2v dsA[2], dmA[2], dsB[2], dmB[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const half2v s2 = __builtin_bit_cast(half2v, (uint32_t)xs[u]);
            const half2v m2 = __builtin_bit_cast(half2v, (uint32_t)xm[u]);
            dsA[u] = half2v{s2[0], s2[0]};
            dmA[u] = half2v{m2[0], m2[0]};
            dsB[u] = half2v{s2[1], s2[1]};
            dmB[u] = half2v{m2[1], m2[1]};
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const half8 wq = pf_dequant8((s & 1) ? o.q1[u] : o.q0[u], s >= 2, s >= 2 ? dsB[u] : dsA[u],
                                             s >= 2 ? dmB[u] : dmA[u]);
#pragma unroll
                for (int t = 0; t < 2; ++t)
                    acc[u][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wq, o.x[s][t], acc[u][t], 0, 0, 0);
            }
    }
}

// Wait for this wave's copies, leaving the last n in flight (n is 0 or one
// or two columns' copy counts, 6 or 7 each), and for its LDS reads: after the
// next barrier no wave still reads a slot that a copy is about to refill.
static_assert(PF_B_COPIES == 18, "copy counts 7 (waves 0-1) and 6");
__device__ __forceinline__ void pf_wait_copies(int n)
{
    switch (n) {
    case 14: __builtin_amdgcn_s_waitcnt(14 | 0x0070); break; // vmcnt(14) lgkmcnt(0)
    case 12: __builtin_amdgcn_s_waitcnt(12 | 0x0070); break;
    case 7: __builtin_amdgcn_s_waitcnt(7 | 0x0070); break;
    case 6: __builtin_amdgcn_s_waitcnt(6 | 0x0070); break;
    default: __builtin_amdgcn_s_waitcnt(0 | 0x0070); break; // vmcnt(0) lgkmcnt(0)
    }
}

// Y[t, n] = sum_k W[n, k] Xh[t, k] for one 64-token x 128-row tile, over
// the block columns of one split of K: split sp of nsplit takes columns
// sp * nblk / nsplit .. (sp + 1) * nblk / nsplit - 1 and writes its sums to
// Y (split 0) or to partial plane sp - 1 of `part` (T x N floats each), which
// k_prefill_splits_sum then adds into Y.  Wave (rh, j) = (wave & 1, wave >> 1)
// accumulates weight rows 64 rh .. +63 over sub-block pair j of every block
// column; at the end wave (rh, j) finishes tile combination c = j (weight
// half u = c >> 1, token half t = c & 1) of its row half from the four
// waves' partial sums.
template <bool EXACTW>
__global__ __launch_bounds__(PF_THREADS) void k_prefill_q4k(const uint8_t *__restrict__ W,
                                                            const _Float16 *__restrict__ Xh,
                                                            const int *__restrict__ xs,
                                                            float *__restrict__ Y,
                                                            float *__restrict__ part, int T, int K,
                                                            int N, int mtiles, int ntiles, int nsplit)
{
    __shared__ __attribute__((aligned(16))) uint8_t ring[PF_NSLOT * PF_SLOT];

    const int tiles = mtiles * ntiles;
    const int lin = prefill_lin((int)blockIdx.x, tiles, nsplit);
    if (lin >= tiles * nsplit)
        return; // whole workgroup

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rh = wave & 1, j = wave >> 1;
    const int h = lane >> 5, li = lane & 31;
    const int nblk = K / 256;
    const size_t row_bytes = (size_t)nblk * 144;
    const PrefillSplit ps = prefill_split_of(lin, mtiles, ntiles, nblk, nsplit);
    const int m0 = ps.mt * PF_BM, n0 = ps.nt * PF_BN;
    const int kb0 = ps.kb0, nk = ps.nk; // this split's block columns (nk >= 1)
    float *const out = ps.sp == 0 ? Y : part + (size_t)(ps.sp - 1) * (size_t)T * (size_t)N;
    const int brow = 64 * rh + li;                        // this lane's first weight row
    const int copies = 4 + (PF_B_COPIES - wave + 7) / 8; // copies this wave issues per column

    float16v acc[2][2];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[u][t][r] = 0.0f;

    // byte offsets below 2^32: the launcher checks T * K * 2 and N * row_bytes
    PfSrc S;
    S.a0 = pf_src_a(m0, T, K, wave, lane, 0);
    S.a1 = pf_src_a(m0, T, K, wave, lane, 1);
    S.a2 = pf_src_a(m0, T, K, wave, lane, 2);
    S.a3 = pf_src_a(m0, T, K, wave, lane, 3);
    S.b0 = pf_src_b(n0, N, (uint32_t)row_bytes, lane, wave);
    S.b1 = pf_src_b(n0, N, (uint32_t)row_bytes, lane, wave + 8);
    S.b2 = pf_src_b(n0, N, (uint32_t)row_bytes, lane, wave + 16);
    // the split's first block column: activations 512 bytes and weight rows
    // 144 bytes per column further on
    const uint8_t *Xb = reinterpret_cast<const uint8_t *>(Xh) + (size_t)kb0 * 512;
    W += (size_t)kb0 * 144;
    const uint32_t ring_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)ring;

    // Column kb lives in slot kb % 3.  A wave reads column kb + 1 into
    // registers while it dequantizes and multiplies column kb, so the LDS
    // reads of the next column overlap this column's matrix-core work; the
    // copies of column kb + 3 go into column kb's slot, which every wave has
    // read (into registers) before the barrier of iteration kb.
    const int nfill = min(nk, PF_NSLOT);
    for (int c = 0; c < nfill; ++c)
        pf_issue(S, Xb, W, c, wave, ring_lds + c * PF_SLOT);
    pf_wait_copies((nfill - 1) * copies);
    lds_barrier();
    const uint8_t *ba = ring + PF_A_STAGE + brow * 144; // this lane's weight rows in slot 0
    PfOps o0, o1;
    pf_read(ring, ba, ba + 32 * 144, j, h, li, o0);

    // Block column kb, which has a successor: wait for the successor's
    // copies, publish it, refill column kb's slot (`slot` = kb % 3), read the
    // successor into `nxt`, then reduce `cur`.  The last column is reduced
    // after the loop, so that no branch inside the loop decides whether a
    // read was issued (the compiler would then wait for every LDS read in
    // flight, the successor's included, before the first matrix product).
    auto step = [&](int kb, int slot, PfOps &cur, PfOps &nxt) {
        pf_wait_copies(kb + 2 < nk ? copies : 0);
        lds_barrier();
        if (kb + 3 < nk)
            pf_issue(S, Xb, W, kb + 3, wave, ring_lds + slot * PF_SLOT);
        const int ns = slot == 2 ? 0 : slot + 1;
        pf_read(ring + ns * PF_SLOT, ba + ns * PF_SLOT, ba + ns * PF_SLOT + 32 * 144, j, h, li, nxt);
        __builtin_amdgcn_sched_barrier(0);
        pf_mma<EXACTW>(cur, j, acc);
    };
    int kb = 0, slot = 0;
    for (; kb + 2 < nk; kb += 2) {
        step(kb, slot, o0, o1);
        slot = slot == 2 ? 0 : slot + 1;
        step(kb + 1, slot, o1, o0);
        slot = slot == 2 ? 0 : slot + 1;
    }
    if (kb + 1 < nk) {
        step(kb, slot, o0, o1);
        pf_mma<EXACTW>(o1, j, acc);
    } else {
        pf_mma<EXACTW>(o0, j, acc);
    }
    __syncthreads(); // every wave is done with the ring

    // partial sums in LDS: float4 P[rh][c][src][q][lane] (128 KB), where
    // q = r / 4 picks 4 consecutive weight rows of one token
    float4 *P = reinterpret_cast<float4 *>(ring);
    auto pidx = [&](int c, int src, int q) { return (((rh * 4 + c) * 4 + src) * 4 + q) * 64 + lane; };
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        if (c == j)
            continue; // wave-uniform
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float16v &a = acc[c >> 1][c & 1];
            P[pidx(c, j, q)] = make_float4(a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]);
        }
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        if (c != j)
            continue; // wave-uniform: this wave finishes combination c
        const int u = c >> 1, t = c & 1;
        float4 v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
            v[q] = make_float4(acc[u][t][4 * q], acc[u][t][4 * q + 1], acc[u][t][4 * q + 2],
                               acc[u][t][4 * q + 3]);
#pragma unroll
        for (int src = 0; src < 4; ++src) {
            if (src == j)
                continue;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 p = P[pidx(c, src, q)];
                v[q].x += p.x;
                v[q].y += p.y;
                v[q].z += p.z;
                v[q].w += p.w;
            }
        }
        const int m = m0 + 32 * t + li;
        if (m >= T)
            break;
        const int sm = -xs[m]; // undo the row's power-of-two scale (exact)
#pragma unroll
        for (int q = 0; q < 4; ++q)
            v[q] = make_float4(__builtin_ldexpf(v[q].x, sm), __builtin_ldexpf(v[q].y, sm),
                               __builtin_ldexpf(v[q].z, sm), __builtin_ldexpf(v[q].w, sm));
        const int nb = n0 + 64 * rh + 32 * u + 4 * h; // + 8 q: 4 consecutive rows
        float *yrow = out + (size_t)m * N;
        if ((N & 3) == 0) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (nb + 8 * q < N)
                    *reinterpret_cast<float4 *>(yrow + nb + 8 * q) = v[q];
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = nb + 8 * q;
                if (n < N) yrow[n] = v[q].x;
                if (n + 1 < N) yrow[n + 1] = v[q].y;
                if (n + 2 < N) yrow[n + 2] = v[q].z;
                if (n + 3 < N) yrow[n + 3] = v[q].w;
            }
        }
    }
}

// Y += P[0] + P[1] + ... + P[nparts - 1] (n floats each), in that order, so
// the result does not depend on which split finished first.
template <bool VEC>
__global__ __launch_bounds__(256) void k_prefill_splits_sum(float *__restrict__ Y,
                                                            const float *__restrict__ P, int64_t n,
                                                            int nparts)
{
    const int64_t stride = (int64_t)gridDim.x * 256;
    if constexpr (VEC) { // n % 4 == 0: every plane starts 16-byte aligned
        float4 *Y4 = reinterpret_cast<float4 *>(Y);
        const float4 *P4 = reinterpret_cast<const float4 *>(P);
        const int64_t n4 = n >> 2;
        for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) {
            float4 v = Y4[i];
            for (int q = 0; q < nparts; ++q) {
                const float4 p = P4[q * n4 + i];
                v.x += p.x;
                v.y += p.y;
                v.z += p.z;
                v.w += p.w;
            }
            Y4[i] = v;
        }
    } else {
        for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
            float v = Y[i];
            for (int q = 0; q < nparts; ++q)
                v += P[q * n + i];
            Y[i] = v;
        }
    }
}

// Rows of at most kPrefillF32MaxK columns: an fp32 GEMM on the fp32 matrix
// cores (v_mfma_f32_32x32x2_f32), with the weights dequantized to fp32 exactly
// (src/Dequant.jl:364-371) and X read as it is.  With fp16 operands a dot
// product's rounding error, relative to ||w_row|| ||x||, shrinks only as
// 1/sqrt(K): over 512 x 2048 outputs of seeded random data the largest
// error reached 1.7x the row bound 1e-4 ||w_row|| ||x|| at K = 256 and
// 0.97-1.05x at K = 512 (0.73 at 768, 0.70 at 1024, 0.30 at 4096), so short
// rows take this path, whose error is fp32 rounding.
//
// Tile: 64 tokens x 64 weight rows per workgroup of 4 waves; wave (rw, tw)
// owns weight rows 32 rw.. and tokens 32 tw.. .  K goes through LDS 64
// columns at a time (48 KB, so that two or three workgroups share a CU and
// one fills its chunk while another multiplies), both operands stored
// k-major (W[k][row], X[k][token]) with rows of 96 floats, so a matrix-core
// operand read (32 consecutive rows or tokens at k and at k + 1) hits 64
// distinct banks.
constexpr int PF32_KC = 64;   // columns per LDS chunk (two Q4_K sub-blocks): 48 KB of LDS
constexpr int PF32_LD = 96;   // floats per LDS row
__global__ __launch_bounds__(256) void k_prefill_q4k_f32(const uint8_t *__restrict__ W,
                                                         const float *__restrict__ X,
                                                         float *__restrict__ Y, int T, int K, int N,
                                                         int mtiles)
{
    __shared__ __attribute__((aligned(16))) float Wl[PF32_KC * PF32_LD];
    __shared__ __attribute__((aligned(16))) float Xl[PF32_KC * PF32_LD];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rw = wave & 1, tw = wave >> 1;
    const int mt = (int)blockIdx.x % mtiles, nt = (int)blockIdx.x / mtiles;
    const int m0 = mt * 64, n0 = nt * 64;
    const int nblk = K / 256;
    // fill roles: thread t stages row (or token) t / 4, 32 columns 32 (t % 4) ..
    const int fr = tid >> 2, fp = tid & 3;
    const uint8_t *wrow = W + (size_t)min(n0 + fr, N - 1) * (size_t)nblk * 144;
    const float *xrow = X + (size_t)min(m0 + fr, T - 1) * (size_t)K;

    float16v acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    for (int c = 0; c < 4 * nblk; ++c) {
        // weights: columns 16 fp .. of chunk c are elements l0 .. l0 + 15 of
        // sub-block sb = 2 (c % 4) + fp / 2 of block c / 4, element
        // 64 j + 32 h + l = (d sc) q_l - dmin m with q_l the low (h = 0) or
        // high nibble of qs[32 j + l] (src/Dequant.jl:364-371)
        {
            const uint8_t *blk = wrow + (size_t)(c >> 2) * 144;
            const int sb = 2 * (c & 3) + (fp >> 1), j = sb >> 1, h = sb & 1, l0 = 16 * (fp & 1);
            const uint4 hd = *reinterpret_cast<const uint4 *>(blk);
            const float d = h2f(hd.x & 0xffffu), dmin = h2f(hd.x >> 16);
            uint32_t sc, m;
            k_scale_min(hd.y, hd.z, hd.w, sb, sc, m);
            const float d1 = d * (float)sc, m1 = dmin * (float)m;
            const uint4 qa = *reinterpret_cast<const uint4 *>(blk + 16 + 32 * j + l0);
            const uint32_t qw[4] = {qa.x, qa.y, qa.z, qa.w};
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t q = ((qw[i >> 2] >> (8 * (i & 3))) >> (4 * h)) & 0xfu;
                Wl[(16 * fp + i) * PF32_LD + fr] = d1 * (float)q - m1;
            }
        }
        // activations: token fr, columns 64 c + 16 fp ..
        {
            const float4 *xs = reinterpret_cast<const float4 *>(xrow + (size_t)c * PF32_KC + 16 * fp);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 v = xs[i];
                Xl[(16 * fp + 4 * i + 0) * PF32_LD + fr] = v.x;
                Xl[(16 * fp + 4 * i + 1) * PF32_LD + fr] = v.y;
                Xl[(16 * fp + 4 * i + 2) * PF32_LD + fr] = v.z;
                Xl[(16 * fp + 4 * i + 3) * PF32_LD + fr] = v.w;
            }
        }
        __syncthreads();
        // A = weights (lane l: row l % 32 at k + l / 32), B = activations
        // (token l % 32 at k + l / 32)
        const float *wa = Wl + (lane >> 5) * PF32_LD + 32 * rw + (lane & 31);
        const float *xb = Xl + (lane >> 5) * PF32_LD + 32 * tw + (lane & 31);
#pragma unroll 8
        for (int k = 0; k < PF32_KC; k += 2)
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(wa[k * PF32_LD], xb[k * PF32_LD], acc, 0, 0, 0);
        __syncthreads();
    }
    // lane l, register r: weight row 32 rw + 8 (r / 4) + 4 (l / 32) + r % 4,
    // token 32 tw + l % 32
    const int m = m0 + 32 * tw + (lane & 31);
    if (m >= T)
        return;
    float *yrow = Y + (size_t)m * (size_t)N;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int n = n0 + 32 * rw + 8 * q + 4 * (lane >> 5);
        const float4 v = make_float4(acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]);
        if ((N & 3) == 0 && n + 3 < N) {
            *reinterpret_cast<float4 *>(yrow + n) = v;
        } else {
            if (n < N) yrow[n] = v.x;
            if (n + 1 < N) yrow[n + 1] = v.y;
            if (n + 2 < N) yrow[n + 2] = v.z;
            if (n + 3 < N) yrow[n + 3] = v.w;
        }
    }
}

hipError_t launch_prefill_q4k_f32(const void *w, const float *X, float *Y, int T, int inner,
                                  int outer, hipStream_t s)
{
    if (T <= 0 || outer <= 0 || inner <= 0 || inner % 256 || (int64_t)T * outer > (int64_t)INT32_MAX)
        return hipErrorInvalidValue;
    const int mtiles = (T + 63) / 64, ntiles = (outer + 63) / 64;
    hipLaunchKernelGGL(k_prefill_q4k_f32, dim3((unsigned)(mtiles * ntiles)), dim3(256), 0, s,
                       (const uint8_t *)w, X, Y, T, inner, outer, mtiles);
    return hipGetLastError();
}

hipError_t launch_prefill_convert(const float *X, void *xh, int T, int inner, hipStream_t s)
{
    if (T <= 0 || inner <= 0 || inner % 256)
        return hipErrorInvalidValue;
    int *xs = reinterpret_cast<int *>(static_cast<uint8_t *>(xh) + prefill_scale_offset(T, inner));
    hipLaunchKernelGGL(k_x_to_f16, dim3((unsigned)T), dim3(256), 0, s, X, (_Float16 *)xh, xs, inner);
    return hipGetLastError();
}

hipError_t launch_prefill_q4k(const void *w, const float *X, void *xh, float *Y, int T,
                              int inner, int outer, hipStream_t s)
{
    if (T <= 0 || inner % 256 || !prefill_fits(T, inner, outer))
        return hipErrorInvalidValue;
    if (inner <= kPrefillF32MaxK)
        return launch_prefill_q4k_f32(w, X, Y, T, inner, outer, s);
    const hipError_t e = launch_prefill_convert(X, xh, T, inner, s);
    if (e != hipSuccess)
        return e;
    return launch_prefill_gemm(w, xh, Y, T, inner, outer, s);
}

hipError_t launch_prefill_gemm(const void *w, void *xh, float *Y, int T, int inner, int outer,
                               hipStream_t s)
{
    if (T <= 0 || inner <= kPrefillF32MaxK || inner % 256 || !prefill_fits(T, inner, outer))
        return hipErrorInvalidValue;
    int *xs = reinterpret_cast<int *>(static_cast<uint8_t *>(xh) + prefill_scale_offset(T, inner));
    float *P = reinterpret_cast<float *>(static_cast<uint8_t *>(xh) + prefill_part_offset(T, inner));
    const int mtiles = (T + PF_BM - 1) / PF_BM, ntiles = (outer + PF_BN - 1) / PF_BN;
    const int nsplit = prefill_splits(T, inner, outer, device_cus());
    const dim3 grid(prefill_grid(mtiles * ntiles, nsplit));
    if (inner <= kPrefillExactWMaxK)
        hipLaunchKernelGGL(k_prefill_q4k<true>, grid, dim3(PF_THREADS), 0, s, (const uint8_t *)w,
                           (const _Float16 *)xh, (const int *)xs, Y, P, T, inner, outer, mtiles, ntiles, nsplit);
    else
        hipLaunchKernelGGL(k_prefill_q4k<false>, grid, dim3(PF_THREADS), 0, s, (const uint8_t *)w,
                           (const _Float16 *)xh, (const int *)xs, Y, P, T, inner, outer, mtiles, ntiles, nsplit);
    if (nsplit > 1) {
        const int64_t n = (int64_t)T * outer;
        const int64_t units = (n & 3) == 0 ? n >> 2 : n;
        const unsigned grid = (unsigned)std::min<int64_t>((units + 255) / 256, 2048);
        if ((n & 3) == 0)
            hipLaunchKernelGGL(k_prefill_splits_sum<true>, dim3(grid), dim3(256), 0, s, Y,
                               (const float *)P, n, nsplit - 1);
        else
            hipLaunchKernelGGL(k_prefill_splits_sum<false>, dim3(grid), dim3(256), 0, s, Y,
                               (const float *)P, n, nsplit - 1);
    }
    return hipGetLastError();
}

} // namespace ihip
