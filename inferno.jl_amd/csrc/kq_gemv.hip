// kq_gemv.hip -- gfx950 dequant-fused GEMV kernels for GGML K-quant, Q8_0
// and IQ4_NL weights and fp32 activations: y[r] = sum_c W[r,c] x[c].
//
// Semantics: the fp32-activation path of Inferno.jl's mul_quant_mat_vec
// (src/ModelCPU.jl:285-379) with the weights of src/Dequant.jl:304-601, to
// the 1e-4 * ||w_row|| * ||x|| row bound.  (The reference C path's int8
// re-quantization of x, src/kernels/quant_kernels.c:166-194, is the separate
// bit-exact variant in kq_q8k.hip.)
//
// A decode GEMV is a single pass over the weight bytes, so every kernel here
// puts all of a wave's weight loads in flight before it waits on any of them
// and reuses each lane's activations over many rows.  x enters as 22-bit
// fixed-point integers per 32 values, split into three byte digits, so the
// weight products run on the integer dot units (v_dot4, exact sums; the
// representation and its error bound are described at XDig below), and the
// `dmin*m` term of Q4_K/Q5_K and the weight offsets of Q6_K / Q8_0 / IQ4_NL
// are taken off through per-sub-block sums of x that all rows share.
//
//   * Q4_K / Q5_K ("wide" kernels, k_gemv_kwide / k_gemv_kpers): blocks are
//     16-byte multiples, so lanes load straight from HBM with 128-bit loads.
//     A wave covers 16 blocks (4096 columns) of R rows per pass: lane =
//     (block, sub-block pair), 64 weights per lane per row.
//   * Q6_K (210 B), Q8_0 (34 B) and IQ4_NL (18 B) blocks are not 16-byte
//     aligned, but 8 of them are.  k_gemv_sdig streams each wave's rows
//     through a private LDS ring filled by gfx950's direct-to-LDS 128-bit
//     copies (no registers, no workgroup barrier), then re-slices blocks
//     from LDS.
//   * Greedy argmax (lm_head) is fused into the streamed kernel's epilogue:
//     each workgroup writes one (value, index) partial to its own slot and a
//     one-workgroup kernel reduces the partials, so no two workgroups touch
//     the same address.
#include <atomic>
#include "inferno_hip.h"

#include <algorithm>
#include "kq_common.h"
#include "kq_launch.h"
#include "kq_sdig_plan.h"

namespace ihip {

// ------------------------------------------------------------------------
// Q4_K / Q5_K wide kernels
// ------------------------------------------------------------------------

// Lane geometry inside a 16-block (4096-column) pass: block b = lane >> 2,
// sub-block pair j = lane & 3.  The lane's weights are qs[32j, 32j+32) of
// block b: low nibbles are elements 64j + l (sub-block 2j), high nibbles
// 64j + 32 + l (sub-block 2j+1), l = 0..31 (src/Dequant.jl:364-371).
//
// The weight bytes go straight to registers (three 128-bit loads per row and
// lane).  x is read once per workgroup with contiguous loads and staged in LDS
// as integer digits (below), with the sum of every 32-element sub-block of x.
// Loads are issued x first, then every row's weights, so x can be staged while
// the weights are still in flight, and each row is reduced as soon as its own
// bytes land.

// float4s of a 4096-element pass per thread of an NT-thread workgroup (768
// threads: two, the second only for threads below 256)
__host__ __device__ constexpr int xnv(int nt) { return (1024 + nt - 1) / nt; }
template <int NT>
__device__ __forceinline__ void x_load_pass(const float *__restrict__ x, int col0, int inner,
                                            float4 (&xv)[xnv(NT)])
{
#pragma unroll
    for (int k = 0; k < xnv(NT); ++k) {
        const int f = threadIdx.x + NT * k; // float4 of the pass
        const int col = col0 + 4 * f;
        xv[k] = (f < 1024 && col < inner) ? *reinterpret_cast<const float4 *>(x + col)
                                          : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}


// ---- integer-digit activations -------------------------------------------
// The dot of a lane's nibbles with x can run on the integer dot units
// (v_dot4_{u32_u8,i32_i8}: four byte products and the accumulate in one
// instruction) when x is written as an integer.  Each 32-element sub-block of
// x is scaled by 2^(22-e), e the binary exponent of the sub-block's largest
// |x| (|x| < 2^e), and truncated to an integer X with |X| < 2^22: the error of
// x ~ X * 2^(e-22) is below 2^(e-22) <= |x|max * 2^-21.  The sub-block's
// |x|max is at most its own 2-norm, so the error vector of 32 values has a
// norm below sqrt(32) * 2^-21 times theirs, and over any number of sub-blocks
// ||x - X 2^(e-22)||_2 < sqrt(32) * 2^-21 * ||x||_2: a dot product is off by
// less than 2.7e-6 * ||w||_2 ||x||_2 whatever its length and data (the row
// bound is 1e-4; about 1e-7 for random data).  X is split into three byte digits,
// X = 65536 * b2 + 256 * b1 + b0 (b0, b1 unsigned, b2 signed); the products
// q * b are exact integers, so the per-sub-block sums are exact and
// independent of summation order.  A sub-block holding a non-finite value has
// its fp32 sum (which every row's dmin term multiplies) set to NaN, so the
// outputs it reaches are NaN.
struct XDig {
    uint32_t p[3][16]; // digit planes; dwords 0..7 the lane's low-nibble elements, 8..15 high
    float sa, sb;      // fp32 sums of the two sub-blocks of x (the dmin term)
    int ea, eb;        // their exponents
};

// Plane layout in LDS: dword g holds digit p of elements 4g..4g+3, with 4
// dwords of padding after every 16 so a lane's 16-dword reads (lanes 16
// dwords apart) fall on distinct banks.
constexpr int kDigPlaneDw = 1024 + 1024 / 16 * 4;
__device__ __forceinline__ int dpad(int g) { return g + ((g >> 4) << 2); }

// Byte digits of X0..X3 -> one dword per plane (digit p of element i in byte i).
__device__ __forceinline__ void dig_pack(int X0, int X1, int X2, int X3, uint32_t &d0,
                                         uint32_t &d1, uint32_t &d2)
{
    const uint32_t p01 = __builtin_amdgcn_perm(X1, X0, 0x05010400u); // X0.b0 X1.b0 X0.b1 X1.b1
    const uint32_t p23 = __builtin_amdgcn_perm(X3, X2, 0x05010400u);
    const uint32_t q01 = __builtin_amdgcn_perm(X1, X0, 0x0c0c0602u); // X0.b2 X1.b2 0 0
    const uint32_t q23 = __builtin_amdgcn_perm(X3, X2, 0x0c0c0602u);
    d0 = __builtin_amdgcn_perm(p23, p01, 0x05040100u);
    d1 = __builtin_amdgcn_perm(p23, p01, 0x07060302u);
    d2 = __builtin_amdgcn_perm(q23, q01, 0x05040100u);
}

// Digits of four elements that share exponent e (finite == false: zeros).
__device__ __forceinline__ void dig_four(float4 v, int e, bool finite, uint32_t &d0, uint32_t &d1,
                                         uint32_t &d2)
{
    const int sh = 22 - e;
    const int X0 = finite ? (int)__builtin_ldexpf(v.x, sh) : 0;
    const int X1 = finite ? (int)__builtin_ldexpf(v.y, sh) : 0;
    const int X2 = finite ? (int)__builtin_ldexpf(v.z, sh) : 0;
    const int X3 = finite ? (int)__builtin_ldexpf(v.w, sh) : 0;
    dig_pack(X0, X1, X2, X3, d0, d1, d2);
}

// |x| bits of four elements, maxed: NaN > +Inf > every finite value.
__device__ __forceinline__ uint32_t abs_bits_max(float4 v)
{
    const uint32_t m01 = max(__float_as_uint(v.x) & 0x7fffffffu, __float_as_uint(v.y) & 0x7fffffffu);
    const uint32_t m23 = max(__float_as_uint(v.z) & 0x7fffffffu, __float_as_uint(v.w) & 0x7fffffffu);
    return max(m01, m23);
}

// Stage the digits of x[col0, col0 + 4096), its 128 sub-block sums and their
// exponents.  Thread t (of NT) holds float4 k of elements 4(t + NT k): 8
// consecutive threads hold one 32-element sub-block, reduced with three DPP
// steps.
template <int NT>
__device__ __forceinline__ void x_stage_dig(uint32_t *pl, float *xsum, int *xexp,
                                            const float4 (&xv)[xnv(NT)])
{
    static_assert(NT % 64 == 0, "whole waves");
    const int tid = threadIdx.x;
#pragma unroll
    for (int k = 0; k < xnv(NT); ++k) {
        if (tid + NT * k >= 1024)
            continue; // past the pass; wave-uniform (NT and 1024 are multiples of 64)
        const float4 v = xv[k];
        float t = (v.x + v.y) + (v.z + v.w);
        uint32_t m = abs_bits_max(v);
        t = dpp_add<0xb1, 0xf>(t);
        m = dpp_max_u32<0xb1, 0xf>(m);
        t = dpp_add<0x4e, 0xf>(t);
        m = dpp_max_u32<0x4e, 0xf>(m);
        t = dpp_add<0x141, 0xf>(t);
        m = dpp_max_u32<0x141, 0xf>(m);
        const bool finite = m < 0x7f800000u;
        const int e = finite ? __builtin_amdgcn_frexp_expf(__uint_as_float(m)) : 0;
        uint32_t d0, d1, d2;
        dig_four(v, e, finite, d0, d1, d2);
        const int g = dpad(tid + NT * k);
        pl[g] = d0;
        pl[kDigPlaneDw + g] = d1;
        pl[2 * kDigPlaneDw + g] = d2;
        if ((tid & 7) == 0) {
            const int sb = (tid + NT * k) >> 3;
            xsum[sb] = finite ? t : __builtin_nanf("");
            xexp[sb] = e;
        }
    }
}

__device__ __forceinline__ void x_from_lds_dig(const uint32_t *pl, const float *xsum,
                                               const int *xexp, int b, int j, XDig &X)
{
    const int g0 = dpad(64 * b + 16 * j); // 16 contiguous dwords
#pragma unroll
    for (int p = 0; p < 3; ++p)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint4 v = *reinterpret_cast<const uint4 *>(pl + p * kDigPlaneDw + g0 + 4 * t);
            X.p[p][4 * t + 0] = v.x; X.p[p][4 * t + 1] = v.y;
            X.p[p][4 * t + 2] = v.z; X.p[p][4 * t + 3] = v.w;
        }
    const float2 s2 = *reinterpret_cast<const float2 *>(xsum + 8 * b + 2 * j);
    const int2 e2 = *reinterpret_cast<const int2 *>(xexp + 8 * b + 2 * j);
    X.sa = s2.x;
    X.sb = s2.y;
    X.ea = e2.x;
    X.eb = e2.y;
}

// Exact digit sums S0, S1 (unsigned planes) and S2 (signed) of one sub-block
// of the 4- or 5-bit weights of Q4_K / Q5_K -> 65536 * S2 + 256 * S1 + S0 in
// fp32.  |S2| <= 32 * 31 * 64 and S0, S1 <= 32 * 31 * 255, so 256 * S2 + S1
// (< 2^24) is an exact fp32 integer and the combine rounds once.  (Not for
// 6-bit weights: there 256 * S2 can reach 2^25.  The Q6_K dot applies its
// scales to each plane's integer sums and folds the planes in fp32 instead.)
__device__ __forceinline__ float dig_combine(uint32_t s0, uint32_t s1, int s2)
{
    return fmaf((float)(int)(((uint32_t)s2 << 8) + s1), 256.0f, (float)s0);
}

// IQ4_NL weights (src/Dequant.jl:683-693: element j = low nibble of qs[j],
// element j + 16 = high nibble; weight = d * grid[nibble], grid
// src/QuantsData.jl:384).  The grid, biased by +128 to unsigned bytes, is
// looked up four nibbles at a time with byte permutes (grid[0..7] and
// grid[8..15], then a choice by the nibble's bit 3); the bias comes back off
// exactly in the integer sums (iq4nl_dot_dig).
constexpr uint32_t kIQ4G0 = 0x3F2D1801u; // grid + 128: 1, 24, 45, 63
constexpr uint32_t kIQ4G1 = 0x766A5D4Fu; // 79, 93, 106, 118
constexpr uint32_t kIQ4G2 = 0xA6998D81u; // 129, 141, 153, 166
constexpr uint32_t kIQ4G3 = 0xF1D9C5B5u; // 181, 197, 217, 241

// Both nibbles of four packed index bytes q: lo gets grid + 128 of the low
// nibbles, hi of the high nibbles.  The byte choice between the grid's two
// halves comes straight from bit 3 (low) or bit 7 (high) of each byte.
__device__ __forceinline__ void iq4nl_lookup2(uint32_t q, uint32_t &lo, uint32_t &hi)
{
    const uint32_t nl = q & 0x07070707u, nh = (q >> 4) & 0x07070707u;
    const uint32_t pl = ((q >> 1) & 0x04040404u) | 0x03020100u; // byte i of the low or high half
    const uint32_t ph = ((q >> 5) & 0x04040404u) | 0x03020100u;
    lo = __builtin_amdgcn_perm(__builtin_amdgcn_perm(kIQ4G3, kIQ4G2, nl), // grid[8..15]
                               __builtin_amdgcn_perm(kIQ4G1, kIQ4G0, nl), pl); // grid[0..7]
    hi = __builtin_amdgcn_perm(__builtin_amdgcn_perm(kIQ4G3, kIQ4G2, nh),
                               __builtin_amdgcn_perm(kIQ4G1, kIQ4G0, nh), ph);
}

__device__ __forceinline__ uint32_t sel_u32(int c, uint32_t a, uint32_t b) { return c ? a : b; }

// One lane's contribution to one row: its two sub-blocks (2j, 2j + 1) of
// block b, d * (sc_A * sum_A + sc_B * sum_B) - dmin * (m_A * xsum_A + m_B *
// xsum_B) (src/Dequant.jl:364-371), the weight sums formed exactly on the
// integer dot units.
//
// IQ4_NL: blocks 2j and 2j + 1 of the 8 in the 144-byte unit, d * sum over
// grid[q] x per block (no mins).  The looked-up bytes carry the grid's +128
// bias; 128 * (the block's digit sums) takes it off again exactly.  A block
// of x holding a non-finite value (its fp32 sum NaN) makes the lane's sum NaN.
template <int FMT>
__device__ __forceinline__ float kdig_dot(const KBytes &B, int j, const XDig &X)
{
    if constexpr (FMT == kIQ4_NL) {
        const uint32_t w[12] = {B.h.x,  B.h.y,  B.h.z,  B.h.w,  B.q0.x, B.q0.y,
                                B.q0.z, B.q0.w, B.q1.x, B.q1.y, B.q1.z, B.q1.w};
        // the lane's 9 dwords start j dwords in: rotate by j, one select per
        // dword and bit of j (selects of values: a conditional of two array
        // elements is an lvalue, a select of addresses that keeps the arrays
        // out of registers)
        uint32_t t1[11], D[9];
#pragma unroll
        for (int k = 0; k < 11; ++k) t1[k] = sel_u32(j & 1, w[k + 1], w[k]);
#pragma unroll
        for (int k = 0; k < 9; ++k) D[k] = sel_u32(j & 2, t1[k + 2], t1[k]);
        // block A: d in bytes 0-1, qs in bytes 2-17; block B: d in 18-19, qs in 20-35
        uint32_t a0 = 0, a1 = 0, c0 = 0, c1 = 0, z0a = 0, z1a = 0, z0c = 0, z1c = 0;
        int a2 = 0, c2 = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t qa = __builtin_amdgcn_alignbyte(D[t + 1], D[t], 2);
            const uint32_t qc = D[5 + t];
            uint32_t la, ha, lc, hc; // elements 4t + b and 16 + 4t + b of A, of C
            iq4nl_lookup2(qa, la, ha);
            iq4nl_lookup2(qc, lc, hc);
            a0 = __builtin_amdgcn_udot4(la, X.p[0][t], a0, false);
            a0 = __builtin_amdgcn_udot4(ha, X.p[0][4 + t], a0, false);
            a1 = __builtin_amdgcn_udot4(la, X.p[1][t], a1, false);
            a1 = __builtin_amdgcn_udot4(ha, X.p[1][4 + t], a1, false);
            a2 = __builtin_amdgcn_sdot4((int)(la ^ 0x80808080u), (int)X.p[2][t], a2, false);
            a2 = __builtin_amdgcn_sdot4((int)(ha ^ 0x80808080u), (int)X.p[2][4 + t], a2, false);
            c0 = __builtin_amdgcn_udot4(lc, X.p[0][8 + t], c0, false);
            c0 = __builtin_amdgcn_udot4(hc, X.p[0][12 + t], c0, false);
            c1 = __builtin_amdgcn_udot4(lc, X.p[1][8 + t], c1, false);
            c1 = __builtin_amdgcn_udot4(hc, X.p[1][12 + t], c1, false);
            c2 = __builtin_amdgcn_sdot4((int)(lc ^ 0x80808080u), (int)X.p[2][8 + t], c2, false);
            c2 = __builtin_amdgcn_sdot4((int)(hc ^ 0x80808080u), (int)X.p[2][12 + t], c2, false);
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            z0a = __builtin_amdgcn_udot4(0x80808080u, X.p[0][t], z0a, false);
            z1a = __builtin_amdgcn_udot4(0x80808080u, X.p[1][t], z1a, false);
            z0c = __builtin_amdgcn_udot4(0x80808080u, X.p[0][8 + t], z0c, false);
            z1c = __builtin_amdgcn_udot4(0x80808080u, X.p[1][8 + t], z1c, false);
        }
        const float vA = fmaf(fmaf((float)a2, 256.0f, (float)(int)(a1 - z1a)), 256.0f, (float)(int)(a0 - z0a));
        const float vC = fmaf(fmaf((float)c2, 256.0f, (float)(int)(c1 - z1c)), 256.0f, (float)(int)(c0 - z0c));
        const float dA = h2f(D[0] & 0xffffu), dC = h2f(D[4] >> 16);
        return fmaf(dA, __builtin_ldexpf(vA, X.ea - 22) + X.sa * 0.0f,
                    dC * (__builtin_ldexpf(vC, X.eb - 22) + X.sb * 0.0f));
    }
    if constexpr (FMT == kQ8_0) {
        // the lane's 17 dwords, loaded from its own first byte (kbytes_load)
        const uint32_t D[17] = {B.h.x,  B.h.y,  B.h.z,  B.h.w,  B.q0.x, B.q0.y, B.q0.z, B.q0.w, B.q1.x,
                                B.q1.y, B.q1.z, B.q1.w, B.e0.x, B.e0.y, B.e0.z, B.e0.w, B.e1.x};
        // block A: d in bytes 0-1, qs in 2-33; block B: d in 34-35, qs in 36-67.
        // Signed weights: q + 128 (q ^ 0x80) on the unsigned planes, the
        // bias taken off as 128 * (digit sums); q itself on the signed plane.
        uint32_t a0 = 0, a1 = 0, c0 = 0, c1 = 0, z0a = 0, z1a = 0, z0c = 0, z1c = 0;
        int a2 = 0, c2 = 0;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t qa = __builtin_amdgcn_alignbyte(D[t + 1], D[t], 2);
            const uint32_t qc = D[9 + t];
            a0 = __builtin_amdgcn_udot4(qa ^ 0x80808080u, X.p[0][t], a0, false);
            a1 = __builtin_amdgcn_udot4(qa ^ 0x80808080u, X.p[1][t], a1, false);
            a2 = __builtin_amdgcn_sdot4((int)qa, (int)X.p[2][t], a2, false);
            c0 = __builtin_amdgcn_udot4(qc ^ 0x80808080u, X.p[0][8 + t], c0, false);
            c1 = __builtin_amdgcn_udot4(qc ^ 0x80808080u, X.p[1][8 + t], c1, false);
            c2 = __builtin_amdgcn_sdot4((int)qc, (int)X.p[2][8 + t], c2, false);
            z0a = __builtin_amdgcn_udot4(0x80808080u, X.p[0][t], z0a, false);
            z1a = __builtin_amdgcn_udot4(0x80808080u, X.p[1][t], z1a, false);
            z0c = __builtin_amdgcn_udot4(0x80808080u, X.p[0][8 + t], z0c, false);
            z1c = __builtin_amdgcn_udot4(0x80808080u, X.p[1][8 + t], z1c, false);
        }
        const float vA = fmaf(fmaf((float)a2, 256.0f, (float)(int)(a1 - z1a)), 256.0f, (float)(int)(a0 - z0a));
        const float vC = fmaf(fmaf((float)c2, 256.0f, (float)(int)(c1 - z1c)), 256.0f, (float)(int)(c0 - z0c));
        const float dA = h2f(D[0] & 0xffffu), dC = h2f(D[8] >> 16);
        return fmaf(dA, __builtin_ldexpf(vA, X.ea - 22) + X.sa * 0.0f,
                    dC * (__builtin_ldexpf(vC, X.eb - 22) + X.sb * 0.0f));
    }
    const uint32_t qw[8] = {B.q0.x, B.q0.y, B.q0.z, B.q0.w, B.q1.x, B.q1.y, B.q1.z, B.q1.w};
    uint32_t a0 = 0, a1 = 0, c0 = 0, c1 = 0;
    int a2 = 0, c2 = 0;
    uint32_t ew[8];
    if constexpr (FMT == kQ5_K) {
        const uint32_t sh = 2 * j;
        const uint32_t e[8] = {B.e0.x, B.e0.y, B.e0.z, B.e0.w, B.e1.x, B.e1.y, B.e1.z, B.e1.w};
#pragma unroll
        for (int t = 0; t < 8; ++t) ew[t] = e[t] >> sh;
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        uint32_t lo = qw[t] & 0x0f0f0f0fu;
        uint32_t hi = (qw[t] >> 4) & 0x0f0f0f0fu;
        if constexpr (FMT == kQ5_K) {
            lo |= (ew[t] & 0x01010101u) << 4;
            hi |= (ew[t] & 0x02020202u) << 3;
        }
        a0 = __builtin_amdgcn_udot4(lo, X.p[0][t], a0, false);
        a1 = __builtin_amdgcn_udot4(lo, X.p[1][t], a1, false);
        a2 = __builtin_amdgcn_sdot4((int)lo, (int)X.p[2][t], a2, false);
        c0 = __builtin_amdgcn_udot4(hi, X.p[0][8 + t], c0, false);
        c1 = __builtin_amdgcn_udot4(hi, X.p[1][8 + t], c1, false);
        c2 = __builtin_amdgcn_sdot4((int)hi, (int)X.p[2][8 + t], c2, false);
    }
    const float vA = dig_combine(a0, a1, a2), vB = dig_combine(c0, c1, c2);
    const float d = h2f(B.h.x & 0xffffu), dmin = h2f(B.h.x >> 16);
    float scA, mA, scB, mB;
    k_scale_min_pair(B.h.y, B.h.z, B.h.w, j, scA, mA, scB, mB);
    // ldexp after the product: exact scaling, gradual underflow for tiny x
    const float pos = __builtin_ldexpf(scA * vA, X.ea - 22) + __builtin_ldexpf(scB * vB, X.eb - 22);
    const float neg = fmaf(mA, X.sa, mB * X.sb);
    return fmaf(d, pos, -(dmin * neg));
}

// Plain GEMV (GATEUP == false) or fused gate/up + SwiGLU (GATEUP == true:
// W2 is the up weight, y[r] = silu(g[r]) * u[r]).  Wave w of workgroup g
// (NWV waves) owns rows [(NWV g + w) R, (NWV g + w + 1) R); rows past `outer`
// re-read the last row and are not stored.
//
// EXT selects an optional neighbour at compile time (a runtime test would
// cost a branch at the head of every wave):
//   GATEUP: the input is rmsnorm(x) .* nw (rmsnorm_cpu!, src/ModelCPU.jl:111-123).
//     x .* nw is staged instead of x and the row sums are multiplied by
//     1/sqrt(mean(x^2) + eps) at the end, so the norm costs no extra pass.
//   plain: y[r] = resid[r] + (W x)[r], the residual add of
//     src/ModelCPU.jl:913-920 (resid may be y itself).
//
// The body is shared with k_gemv_kwide_norm (a plain GEMV whose input is the
// normed x) through kwide_body, which takes NORM and RESID directly.
template <int FMT, int R, bool GATEUP, bool NORM, bool RESID, int NWV>
__device__ __forceinline__ void kwide_body(const uint8_t *__restrict__ W, const uint8_t *__restrict__ W2,
                                           const float *__restrict__ x, float *y, int outer, int nblk,
                                           const float *__restrict__ nw, float eps, const float *resid,
                                           int epi)
{
    using F = KFmt<FMT>;
    constexpr int NW = GATEUP ? 2 : 1;
    constexpr int NT = NWV * 64, NXV = xnv(NT);
    // x's three digit planes, its sub-block sums and exponents
    __shared__ __attribute__((aligned(16))) uint32_t xbuf[3 * kDigPlaneDw];
    __shared__ __attribute__((aligned(16))) float xsum[128];
    __shared__ __attribute__((aligned(8))) int xexp[128];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6); // wave-uniform (scalar)
    const int row0 = (blockIdx.x * NWV + wave) * R;
    const int b = lane >> 2, j = lane & 3;
    const int inner = nblk * 256;
    const size_t row_bytes = (size_t)nblk * F::BYTES;

    float acc[NW][R];
#pragma unroll
    for (int m = 0; m < NW; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;

    float ssq = 0.0f; // this thread's share of sum(x^2) (NORM)
    float rv[R];      // residuals of this wave's rows, loaded ahead of the weights
#pragma unroll
    for (int r = 0; r < R; ++r)
        rv[r] = RESID ? resid[min(row0 + r, outer - 1)] : 0.0f;
    const int npass = (nblk + 15) >> 4;
    for (int pass = 0; pass < npass; ++pass) {
        const int nb = min(16, nblk - pass * 16);
        const bool active = b < nb;
        const int blk = pass * 16 + (active ? b : 0);
        // x first, then every row's weights (measured on MI355X at 4096 x 4096:
        // 4.29 us per launch; weights first 5.10 us, the first row's weights
        // then x then the second row's 4.88 us): x is staged while the weights
        // are in flight, and a wait for x waits only for x
        float4 xv[NXV];
        x_load_pass<NT>(x, pass * 4096, inner, xv);
        if constexpr (NORM) {
            float4 wv[NXV];
            x_load_pass<NT>(nw, pass * 4096, inner, wv);
#pragma unroll
            for (int k = 0; k < NXV; ++k) {
                ssq = fmaf(xv[k].x, xv[k].x, ssq);
                ssq = fmaf(xv[k].y, xv[k].y, ssq);
                ssq = fmaf(xv[k].z, xv[k].z, ssq);
                ssq = fmaf(xv[k].w, xv[k].w, ssq);
                xv[k] = make_float4(xv[k].x * wv[k].x, xv[k].y * wv[k].y, xv[k].z * wv[k].z,
                                    xv[k].w * wv[k].w);
            }
        }
        KBytes B[NW][R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = min(row0 + r, outer - 1);
#pragma unroll
            for (int m = 0; m < NW; ++m) {
                const uint8_t *Wm = m == 0 ? W : W2;
                kbytes_load<FMT>(Wm + (size_t)row * row_bytes + (size_t)blk * F::BYTES, j, B[m][r]);
            }
        }
        // keep every load above in flight before the first use
        __builtin_amdgcn_sched_barrier(0);
        if (pass > 0)
            __syncthreads(); // the previous pass is done with xs / xsum
        x_stage_dig<NT>(xbuf, xsum, xexp, xv);
        __syncthreads();
        XDig X;
        x_from_lds_dig(xbuf, xsum, xexp, b, j, X);
        // rows one after the other, in load order: row r is reduced as soon as
        // its own bytes have landed instead of after every row's
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < NW; ++m) {
                const float c = kdig_dot<FMT>(B[m][r], j, X);
                acc[m][r] += active ? c : 0.0f;
                __builtin_amdgcn_sched_barrier(0);
            }
    }
    float scale = 1.0f;
    if constexpr (NORM) { // every wave takes part in the barrier
        __shared__ float ssw[NWV];
        const float t = wave_sum(ssq);
        if (lane == 0)
            ssw[wave] = t;
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int i = 0; i < NWV; ++i)
            tot += ssw[i];
        scale = 1.0f / sqrtf(tot / (float)inner + eps);
    }
    if (row0 >= outer)
        return; // wave-uniform, after the last barrier
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float g = wave_sum(acc[0][r]) * scale;
        float v = g;
        if constexpr (GATEUP) {
            const float u = wave_sum(acc[NW - 1][r]) * scale;
            // src/ModelCPU.jl:492-503: g / (1 + exp(-g)), then * u
            v = (g / (1.0f + expf(-g))) * u;
        }
        const int row = row0 + r;
        if (lane == 0 && row < outer)
            y[row] = RESID ? epi_apply(rv[r], v, epi) : v;
    }
}

template <int FMT, int R, bool GATEUP, bool EXT, int NWV>
__global__ __launch_bounds__(NWV * 64) void k_gemv_kwide(const uint8_t *__restrict__ W,
                                                    const uint8_t *__restrict__ W2,
                                                    const float *__restrict__ x,
                                                    float *y, int outer, int nblk,
                                                    const float *__restrict__ nw, float eps,
                                                    const float *resid, int epi)
{
    kwide_body<FMT, R, GATEUP, GATEUP && EXT, !GATEUP && EXT, NWV>(W, W2, x, y, outer, nblk, nw, eps,
                                                                   resid, epi);
}

// y = W (rmsnorm(x) .* nw) for one weight: the gate/up pass's folded norm
// (x .* nw staged, the row sums scaled by 1/sqrt(mean(x^2) + eps)) in front of
// a plain GEMV, e.g. the grouped wq/wk/wv behind a layer's input norm
// (src/ModelCPU.jl:903, 789-791).
template <int FMT, int R, int NWV>
__global__ __launch_bounds__(NWV * 64) void k_gemv_kwide_norm(const uint8_t *__restrict__ W,
                                                         const float *__restrict__ x, float *y,
                                                         int outer, int nblk,
                                                         const float *__restrict__ nw, float eps)
{
    kwide_body<FMT, R, false, true, false, NWV>(W, nullptr, x, y, outer, nblk, nw, eps, nullptr, 0);
}

// Persistent form of the digit kernel for matrices of many rows and at most
// 4096 columns (one pass): a workgroup per CU stages x's digits once, each
// lane keeps its 48 digit dwords in registers, and every wave walks row
// groups grid-stride with NB register buffers, so the loads of the next
// NB - 1 groups are in flight while a group is reduced (HBM latency under
// load is a microsecond or more, several group reductions).  A group is R
// rows (GATEUP: R gate rows and the same R up rows).  Same outputs as
// k_gemv_kwide<FMT, R, GATEUP, EXT, NWV>.
// The walk itself over LDS the caller declares (xbuf: 3 * kDigPlaneDw
// dwords, xsum / xexp: 128 each, ssw: NWV floats).
template <int FMT, int R, bool GATEUP, bool NORM, bool RESID, int NWV, int NB>
__device__ __forceinline__ void kpers_run(const uint8_t *__restrict__ W, const uint8_t *__restrict__ W2,
                                          const float *__restrict__ x, float *y, int outer, int nblk,
                                          const float *__restrict__ nw, float eps, const float *resid,
                                          int epi, uint32_t *xbuf, float *xsum, int *xexp, float *ssw)
{
    using F = KFmt<FMT>;
    constexpr int NM = GATEUP ? 2 : 1;
    constexpr int NT = NWV * 64, NXV = xnv(NT);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int b = lane >> 2, j = lane & 3;
    const bool active = b < nblk;
    const int blk = active ? b : 0;
    const int inner = nblk * 256;
    const size_t row_bytes = (size_t)nblk * F::BYTES;
    const int ngroups = (outer + R - 1) / R;
    const int stride = gridDim.x * NWV;
    const int g0 = blockIdx.x * NWV + wave;

    // weights (and the residuals) of group gi into one register buffer
    auto load = [&](KBytes (&B)[NM][R], float (&RV)[R], int gi) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = min(gi * R + r, outer - 1);
            if constexpr (RESID)
                RV[r] = resid[row]; // wave-uniform: a scalar load
#pragma unroll
            for (int m = 0; m < NM; ++m)
                kbytes_load<FMT>((m == 0 ? W : W2) + (size_t)row * row_bytes + (size_t)blk * F::BYTES,
                                 j, B[m][r]);
        }
    };

    float4 xv[NXV];
    x_load_pass<NT>(x, 0, inner, xv);
    float ssq = 0.0f;
    if constexpr (NORM) {
        float4 wv[NXV];
        x_load_pass<NT>(nw, 0, inner, wv);
#pragma unroll
        for (int k = 0; k < NXV; ++k) {
            ssq = fmaf(xv[k].x, xv[k].x, ssq);
            ssq = fmaf(xv[k].y, xv[k].y, ssq);
            ssq = fmaf(xv[k].z, xv[k].z, ssq);
            ssq = fmaf(xv[k].w, xv[k].w, ssq);
            xv[k] = make_float4(xv[k].x * wv[k].x, xv[k].y * wv[k].y, xv[k].z * wv[k].z,
                                xv[k].w * wv[k].w);
        }
    }
    KBytes B[NB][NM][R];
    float RV[NB][R];
#pragma unroll
    for (int q = 0; q < NB; ++q)
        load(B[q], RV[q], min(g0 + q * stride, ngroups - 1));
    __builtin_amdgcn_sched_barrier(0);
    x_stage_dig<NT>(xbuf, xsum, xexp, xv);
    float scale = 1.0f;
    if constexpr (NORM) {
        const float t = wave_sum(ssq);
        if (lane == 0)
            ssw[wave] = t;
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int i = 0; i < NWV; ++i)
            tot += ssw[i];
        scale = 1.0f / sqrtf(tot / (float)inner + eps);
    } else {
        __syncthreads();
    }
    XDig X;
    x_from_lds_dig(xbuf, xsum, xexp, b, j, X);

    auto reduce = [&](const KBytes (&Bq)[NM][R], const float (&RVq)[R], int gi) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = gi * R + r;
            float v[NM];
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                const float c = kdig_dot<FMT>(Bq[m][r], j, X);
                v[m] = wave_sum(active ? c : 0.0f) * scale;
            }
            float o = v[0];
            if constexpr (GATEUP)
                o = (v[0] / (1.0f + expf(-v[0]))) * v[1]; // src/ModelCPU.jl:492-503
            // every lane holds the row's value: an unpredicated store (a row
            // past `outer` re-reads and rewrites row outer - 1 with its own value)
            y[min(row, outer - 1)] = RESID ? epi_apply(RVq[r], o, epi) : o;
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Steady state without predicated loads, so the compiler's vmcnt waits
    // stay exact (a load under a branch makes it wait for every load in
    // flight): every buffer is refilled with a group that exists.
    int gi = g0;
    for (; gi + (2 * NB - 1) * stride < ngroups; gi += NB * stride) { // wave-uniform
#pragma unroll
        for (int q = 0; q < NB; ++q) {
            reduce(B[q], RV[q], gi + q * stride);
            load(B[q], RV[q], gi + (q + NB) * stride);
        }
    }
    // the tail: buffer q holds group gi + q stride; refill only with groups that exist
#pragma unroll
    for (int q = 0; q < NB; ++q) {
        if (gi + q * stride < ngroups)
            reduce(B[q], RV[q], gi + q * stride);
        if (gi + (q + NB) * stride < ngroups)
            load(B[q], RV[q], gi + (q + NB) * stride);
    }
#pragma unroll
    for (int q = 0; q < NB; ++q)
        if (gi + (q + NB) * stride < ngroups)
            reduce(B[q], RV[q], gi + (q + NB) * stride);
}

template <int FMT, int R, bool GATEUP, bool EXT, int NWV, int NB>
__global__ __launch_bounds__(NWV * 64) void k_gemv_kpers(const uint8_t *__restrict__ W,
                                                         const uint8_t *__restrict__ W2,
                                                         const float *__restrict__ x,
                                                         float *y, int outer, int nblk,
                                                         const float *__restrict__ nw, float eps,
                                                         const float *resid, int epi)
{
    __shared__ __attribute__((aligned(16))) uint32_t xbuf[3 * kDigPlaneDw];
    __shared__ __attribute__((aligned(16))) float xsum[128];
    __shared__ __attribute__((aligned(8))) int xexp[128];
    __shared__ float ssw[NWV];
    kpers_run<FMT, R, GATEUP, GATEUP && EXT, !GATEUP && EXT, NWV, NB>(W, W2, x, y, outer, nblk, nw, eps,
                                                                      resid, epi, xbuf, xsum, xexp, ssw);
}

// The persistent kernel with the folded norm on a single weight,
// y = W (rmsnorm(x) .* nw) (as k_gemv_kwide_norm, for rows of at most 16
// blocks past the per-workgroup kernel's row count).
template <int FMT, int R, int NWV, int NB>
__global__ __launch_bounds__(NWV * 64) void k_gemv_kpers_norm(const uint8_t *__restrict__ W,
                                                         const float *__restrict__ x, float *y,
                                                         int outer, int nblk,
                                                         const float *__restrict__ nw, float eps)
{
    __shared__ __attribute__((aligned(16))) uint32_t xbuf[3 * kDigPlaneDw];
    __shared__ __attribute__((aligned(16))) float xsum[128];
    __shared__ __attribute__((aligned(8))) int xexp[128];
    __shared__ float ssw[NWV];
    kpers_run<FMT, R, false, true, false, NWV, NB>(W, nullptr, x, y, outer, nblk, nw, eps, nullptr, 0,
                                                   xbuf, xsum, xexp, ssw);
}

// Persistent form for rows of more than 16 blocks (2..MP passes of 4096
// columns).  One workgroup per CU stages x's digits for every pass once, in
// LDS (x loads of all passes issued together, clamped to the last pass so
// none is predicated).  Each wave then walks items (row group, pass) --
// groups grid-stride, a group's passes in order -- through NB register
// buffers, so the next items' weights are in flight while one is reduced
// and a row's short last pass costs its own bytes rather than a whole
// pass's latency.  Lanes accumulate across a group's passes and the row sum
// is taken after its last pass: the same arithmetic in the same order as
// k_gemv_kwide's serial passes, so the outputs are bit-identical.
template <int FMT, int R, bool GATEUP, bool EXT, int NWV, int NB, int MP>
__global__ __launch_bounds__(NWV * 64) void k_gemv_kpm(const uint8_t *__restrict__ W,
                                                       const uint8_t *__restrict__ W2,
                                                       const float *__restrict__ x,
                                                       float *y, int outer, int nblk,
                                                       const float *__restrict__ nw, float eps,
                                                       const float *resid, int epi)
{
    using F = KFmt<FMT>;
    constexpr int NM = GATEUP ? 2 : 1;
    constexpr bool NORM = GATEUP && EXT, RESID = !GATEUP && EXT;
    constexpr int NT = NWV * 64, NXV = xnv(NT);
    __shared__ __attribute__((aligned(16))) uint32_t xbuf[MP * 3 * kDigPlaneDw];
    __shared__ __attribute__((aligned(16))) float xsum[MP * 128];
    __shared__ __attribute__((aligned(8))) int xexp[MP * 128];
    __shared__ float ssw[NWV];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int b = lane >> 2, j = lane & 3;
    const int inner = nblk * 256;
    const int npass = (nblk + 15) >> 4; // 2..MP (the launcher checks)
    const size_t row_bytes = (size_t)nblk * F::BYTES;
    const int ngroups = (outer + R - 1) / R;
    const int stride = gridDim.x * NWV;
    const int g0 = blockIdx.x * NWV + wave;
    // this wave's items: groups g0, g0 + stride, ... each with npass passes
    const int nitems = g0 < ngroups ? ((ngroups - 1 - g0) / stride + 1) * npass : 0;

    auto load = [&](KBytes (&B)[NM][R], float (&RV)[R], int t) {
        const int k = t / npass, p = t - k * npass; // wave-uniform
        const int gi = min(g0 + k * stride, ngroups - 1);
        const int blk = p * 16 + (b < min(16, nblk - p * 16) ? b : 0);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = min(gi * R + r, outer - 1);
            if constexpr (RESID)
                RV[r] = resid[row]; // wave-uniform: a scalar load
#pragma unroll
            for (int m = 0; m < NM; ++m)
                kbytes_load<FMT>((m == 0 ? W : W2) + (size_t)row * row_bytes + (size_t)blk * F::BYTES,
                                 j, B[m][r]);
        }
    };

    // x of every pass (MP passes of loads, the ones past npass repeating the
    // last), then the first NB items' weights, then the digits into LDS
    float4 xv[MP][NXV];
#pragma unroll
    for (int p = 0; p < MP; ++p)
        x_load_pass<NT>(x, min(p, npass - 1) * 4096, inner, xv[p]);
    float ssq = 0.0f;
    if constexpr (NORM) {
#pragma unroll
        for (int p = 0; p < MP; ++p) {
            float4 wv[NXV];
            x_load_pass<NT>(nw, min(p, npass - 1) * 4096, inner, wv);
            if (p < npass) { // wave-uniform; the loads above are not under it
#pragma unroll
                for (int k = 0; k < NXV; ++k) {
                    ssq = fmaf(xv[p][k].x, xv[p][k].x, ssq);
                    ssq = fmaf(xv[p][k].y, xv[p][k].y, ssq);
                    ssq = fmaf(xv[p][k].z, xv[p][k].z, ssq);
                    ssq = fmaf(xv[p][k].w, xv[p][k].w, ssq);
                    xv[p][k] = make_float4(xv[p][k].x * wv[k].x, xv[p][k].y * wv[k].y,
                                           xv[p][k].z * wv[k].z, xv[p][k].w * wv[k].w);
                }
            }
        }
    }
    KBytes B[NB][NM][R];
    float RV[NB][R];
#pragma unroll
    for (int q = 0; q < NB; ++q)
        load(B[q], RV[q], q);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < MP; ++p)
        if (p < npass)
            x_stage_dig<NT>(xbuf + p * 3 * kDigPlaneDw, xsum + p * 128, xexp + p * 128, xv[p]);
    float scale = 1.0f;
    if constexpr (NORM) {
        const float t = wave_sum(ssq);
        if (lane == 0)
            ssw[wave] = t;
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int i = 0; i < NWV; ++i)
            tot += ssw[i];
        scale = 1.0f / sqrtf(tot / (float)inner + eps);
    } else {
        __syncthreads();
    }

    float acc[NM][R];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;

    auto reduce = [&](const KBytes (&Bq)[NM][R], const float (&RVq)[R], int t) {
        const int k = t / npass, p = t - k * npass; // wave-uniform
        const int gi = g0 + k * stride;
        const bool active = b < min(16, nblk - p * 16);
        XDig X;
        x_from_lds_dig(xbuf + p * 3 * kDigPlaneDw, xsum + p * 128, xexp + p * 128, b, j, X);
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                const float c = kdig_dot<FMT>(Bq[m][r], j, X);
                acc[m][r] += active ? c : 0.0f;
            }
        if (p == npass - 1) { // the group's last pass: its rows are done
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int row = gi * R + r;
                float v[NM];
#pragma unroll
                for (int m = 0; m < NM; ++m) {
                    v[m] = wave_sum(acc[m][r]) * scale;
                    acc[m][r] = 0.0f;
                }
                float o = v[0];
                if constexpr (GATEUP)
                    o = (v[0] / (1.0f + expf(-v[0]))) * v[1]; // src/ModelCPU.jl:492-503
                // every lane holds the row's value: an unpredicated store (a
                // row past `outer` rewrites row outer - 1 with its own value)
                y[min(row, outer - 1)] = RESID ? epi_apply(RVq[r], o, epi) : o;
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    // steady state: every buffer is refilled with an item that exists
    int t = 0;
    for (; t + (2 * NB - 1) < nitems; t += NB) { // wave-uniform
#pragma unroll
        for (int q = 0; q < NB; ++q) {
            reduce(B[q], RV[q], t + q);
            load(B[q], RV[q], t + q + NB);
        }
    }
#pragma unroll
    for (int q = 0; q < NB; ++q) {
        if (t + q < nitems)
            reduce(B[q], RV[q], t + q);
        if (t + q + NB < nitems)
            load(B[q], RV[q], t + q + NB);
    }
#pragma unroll
    for (int q = 0; q < NB; ++q)
        if (t + q + NB < nitems)
            reduce(B[q], RV[q], t + q + NB);
}

// ------------------------------------------------------------------------
// Streamed kernels (Q6_K, Q8_0, IQ4_NL)
// ------------------------------------------------------------------------
// A segment is 8 Q6_K blocks (2048 columns, 1680 B), 64 Q8_0 blocks (2176 B)
// or 64 IQ4_NL blocks (1152 B), the last of a row possibly fewer.  Rows of
// any whole number of blocks stream (16-byte aligned W and x); rows whose byte
// length is not a multiple of 16 leave their segments at byte phases in the
// ring slots (the PH instantiations).
template <int FMT>
struct SFmt;
template <>
struct SFmt<kQ6_K> {
    static constexpr int SEG_BLOCKS = 8, SEG_BYTES = 8 * 210;
};
template <>
struct SFmt<kQ8_0> {
    static constexpr int SEG_BLOCKS = 64, SEG_BYTES = 64 * 34;
};
template <>
struct SFmt<kIQ4_NL> {
    static constexpr int SEG_BLOCKS = 64, SEG_BYTES = 64 * 18;
};
static_assert(SFmt<kQ6_K>::SEG_BYTES % 16 == 0, "Q6_K segment must be 16-byte aligned");
static_assert(SFmt<kQ8_0>::SEG_BYTES % 16 == 0, "Q8_0 segment must be 16-byte aligned");
static_assert(SFmt<kIQ4_NL>::SEG_BYTES % 16 == 0, "IQ4_NL segment must be 16-byte aligned");

// ---- greedy argmax partials ----------------------------------------------
// key = (order-preserving bits of the value << 32) | (0xffffffff - index), so
// the larger key is the larger value and, among equal values, the lower index
// (the strict `>` scan of src/CommonOps.jl:155-158).
struct ArgPart {
    unsigned long long key;
    uint32_t flags; // bit0 NaN, bit1 +Inf, bit2 a value other than -Inf seen
    uint32_t pad;
};
static_assert(sizeof(ArgPart) == 16, "ArgPart layout");
static_assert(kArgMaxParts * sizeof(ArgPart) == IHIP_ARGMAX_WS_BYTES, "argmax workspace size");

__device__ __forceinline__ uint32_t ordered_bits(float v)
{
    if (v == 0.0f)
        v = 0.0f; // -0 == +0 for the strict `>` scan
    const uint32_t b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Fold value v at index i: NaN and +Inf raise a flag and never win.
__device__ __forceinline__ void argmax_fold(float v, uint32_t i, unsigned long long &key,
                                            uint32_t &flags)
{
    if (v != v) {
        flags |= 1u;
        return;
    }
    if (v == INFINITY) {
        flags |= 2u;
        return;
    }
    if (v != -INFINITY)
        flags |= 4u;
    const unsigned long long k =
        ((unsigned long long)ordered_bits(v) << 32) | (unsigned long long)(0xffffffffu - i);
    key = k > key ? k : key;
}

// argmax_fold for a value every lane of the wave holds (a row sum after the
// wave reduction), taken through readfirstlane: the same tests made on the
// value's bits, so the compiler keeps the fold, and key and flags, on the
// scalar unit instead of spending ~20 vector instructions per row on it.
__device__ __forceinline__ void argmax_fold_uniform(float v, uint32_t i, unsigned long long &key,
                                                    uint32_t &flags)
{
    uint32_t b = __builtin_amdgcn_readfirstlane(__float_as_uint(v));
    const uint32_t a = b & 0x7fffffffu;
    if (a > 0x7f800000u) { // NaN
        flags |= 1u;
        return;
    }
    if (b == 0x7f800000u) { // +Inf
        flags |= 2u;
        return;
    }
    if (b != 0xff800000u) // not -Inf
        flags |= 4u;
    if (a == 0u)
        b = 0u; // -0 == +0, as ordered_bits
    const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    const unsigned long long k = ((unsigned long long)ord << 32) | (unsigned long long)(0xffffffffu - i);
    key = k > key ? k : key;
}

__device__ __forceinline__ void argmax_wave_reduce(unsigned long long &key, uint32_t &flags)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const unsigned long long ok = __shfl_xor(key, o, 64);
        key = ok > key ? ok : key;
        flags |= __shfl_xor(flags, o, 64);
    }
}

// Workgroup (4 waves) reduction; thread 0 stores the partial.
__device__ __forceinline__ void argmax_store_partial(unsigned long long key, uint32_t flags,
                                                     ArgPart *part)
{
    __shared__ unsigned long long wkey[4];
    __shared__ uint32_t wflag[4];
    argmax_wave_reduce(key, flags);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        wkey[wave] = key;
        wflag[wave] = flags;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long k = wkey[0];
        uint32_t f = wflag[0];
#pragma unroll
        for (int w = 1; w < 4; ++w) {
            k = wkey[w] > k ? wkey[w] : k;
            f |= wflag[w];
        }
        part->key = k;
        part->flags = f;
        part->pad = 0;
    }
}

// Reduce `nparts` partials with 256 threads, up to 16 16-byte partials in
// flight per thread (the lm_head leaves three per thread); writes the 0-based
// token and the IHIP_FLAG_* bits.
__global__ __launch_bounds__(256) void k_argmax_finalize(const ArgPart *__restrict__ parts,
                                                         int nparts, int32_t *token,
                                                         uint32_t *flags_out)
{
    constexpr int NT = 256, NWV = NT / 64, U = 16;
    unsigned long long key = 0;
    uint32_t fl = 0;
    for (int i0 = threadIdx.x; i0 < nparts; i0 += U * NT) {
        uint4 p[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = i0 + NT * u;
            p[u] = i < nparts ? reinterpret_cast<const uint4 *>(parts)[i] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const unsigned long long k = ((unsigned long long)p[u].y << 32) | p[u].x;
            key = k > key ? k : key;
            fl |= p[u].z;
        }
    }
    argmax_wave_reduce(key, fl);
    __shared__ unsigned long long wkey[NWV];
    __shared__ uint32_t wflag[NWV];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        wkey[wave] = key;
        wflag[wave] = fl;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < NWV; ++w) {
            key = wkey[w] > key ? wkey[w] : key;
            fl |= wflag[w];
        }
    }
    if (threadIdx.x == 0) {
        uint32_t out = fl & 3u;
        int32_t tok = (int32_t)(0xffffffffu - (uint32_t)(key & 0xffffffffull));
        if (!(fl & 4u)) { // every logit was -Inf: index 0 (src/CommonOps.jl:143-161)
            out |= 4u;
            tok = 0;
        }
        *token = tok;
        *flags_out = out;
    }
}

// Standalone argmax over a vector (gpu_argmax!, src/FusedKernels.jl:271-311,
// with the _validate_logits checks of src/CommonOps.jl:142-163).
__global__ __launch_bounds__(256) void k_argmax_partials(const float *__restrict__ v, int64_t n,
                                                         ArgPart *__restrict__ parts)
{
    unsigned long long key = 0;
    uint32_t fl = 0;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        argmax_fold(v[i], (uint32_t)i, key, fl);
    argmax_store_partial(key, fl, parts + blockIdx.x);
}

// ---- persistent streamed kernel with integer-digit activations -----------
// One workgroup per CU (NW waves) walks chunks of rpc rows grid-stride.  The
// K segments of a row (2048 columns each, nseg <= NW) are spread over the
// waves: wave w owns segment w % nseg and, when there are more waves than
// segments, every (NW / nseg)-th row of a chunk.  A wave computes the digits
// of its x slice once, then streams its rows of all its chunks through a
// private D-slot LDS ring of direct-to-LDS copies that runs across chunk
// boundaries (the copy of the row D ahead is issued as soon as a row is
// reduced).  Per chunk the segment sums meet in LDS and the workgroup
// finishes the rows (residual add, argmax fold).
//
// Digits: as for the wide kernels, but each lane scales its own 32 elements
// (one exponent per lane, no cross-lane reduction).  Q6_K's weights q - 32
// and the signed Q8_0 / IQ4_NL weights enter the unsigned digit planes as
// unsigned bytes (q, q + 128, grid + 128); the offsets are taken off exactly
// by starting each integer sum at -offset * (sum of the digits).
struct SXD {
    uint32_t p[3][8]; // digit planes of the lane's 32 elements, 4 per dword
    int init[3][4];   // dot accumulator starts (Q6_K: per 8-element group; else [p][0])
    int e;            // the lane's exponent
    float poison;     // 0, or NaN when the lane's x slice holds a non-finite value
};

// Issue the loads of the lane's 32 elements of x; returns false for a lane
// past the segment's blocks (its loads read block 0 and staged_dig_x zeroes
// them).  The loads are inline assembly the compiler does not track: the
// caller issues them ahead of the ring's direct-to-LDS copies, waits for them
// with an explicit s_waitcnt vmcnt(copies issued since) and then releases the
// registers with staged_dig_pin.  (The compiler's own wait before the first
// use of x would be a vmcnt(0): it treats direct-to-LDS copies and register
// loads as completing out of order, so the digits would wait for every copy.)
typedef float sdig_f4 __attribute__((ext_vector_type(4))); // a register quad for asm operands

__device__ __forceinline__ float4 sdig_gload16(const float *base, int byte_off)
{
    sdig_f4 v;
    switch (byte_off) { // compile-time after unrolling: the immediate offset form
#define IHIP_XL(O)                                                                             \
    case O:                                                                                    \
        asm volatile("global_load_dwordx4 %0, %1, off offset:" #O : "=v"(v) : "v"(base) : "memory"); \
        break;
        IHIP_XL(0) IHIP_XL(16) IHIP_XL(32) IHIP_XL(48) IHIP_XL(64) IHIP_XL(80) IHIP_XL(96) IHIP_XL(112)
        IHIP_XL(128) IHIP_XL(144) IHIP_XL(256) IHIP_XL(272) IHIP_XL(384) IHIP_XL(400)
#undef IHIP_XL
    default:
        asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(base + byte_off / 4) : "memory");
    }
    return __builtin_bit_cast(float4, v);
}

template <int FMT>
__device__ __forceinline__ bool staged_dig_issue(const float *xseg, int lane,
                                                 int seg_blocks, float4 (&v)[8])
{
    bool active;
    const float *base = xseg + sdig_x_lane(FMT, lane, seg_blocks, active);
#pragma unroll
    for (int t = 0; t < 8; ++t)
        v[t] = sdig_gload16(base, sdig_x_load_byte(FMT, t));
    return active;
}

// After the explicit wait for the loads of staged_dig_issue: the registers may
// be read from here on (an empty statement the compiler cannot move them across).
__device__ __forceinline__ void staged_dig_pin(float4 (&v)[8])
{
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        sdig_f4 r = __builtin_bit_cast(sdig_f4, v[t]);
        asm volatile("" : "+v"(r));
        v[t] = __builtin_bit_cast(float4, r);
    }
}

// The lane's digits, exponent and accumulator starts from its loaded x.
template <int FMT>
__device__ __forceinline__ void staged_dig_x(float4 (&v)[8], bool active, SXD &X)
{
    const uint32_t keep = active ? 0xffffffffu : 0u; // a mask, not a branch around loaded registers
#pragma unroll
    for (int t = 0; t < 8; ++t)
        v[t] = make_float4(__uint_as_float(__float_as_uint(v[t].x) & keep),
                           __uint_as_float(__float_as_uint(v[t].y) & keep),
                           __uint_as_float(__float_as_uint(v[t].z) & keep),
                           __uint_as_float(__float_as_uint(v[t].w) & keep));
    uint32_t m = 0;
#pragma unroll
    for (int t = 0; t < 8; ++t)
        m = max(m, abs_bits_max(v[t]));
    const bool finite = m < 0x7f800000u;
    const int e = finite ? __builtin_amdgcn_frexp_expf(__uint_as_float(m)) : 0;
#pragma unroll
    for (int t = 0; t < 8; ++t)
        dig_four(v[t], e, finite, X.p[0][t], X.p[1][t], X.p[2][t]);
    X.e = e;
    X.poison = finite ? 0.0f : __builtin_nanf("");
    constexpr uint32_t ones = 0x01010101u;
    if constexpr (FMT == kQ6_K) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int t = 2 * g;
            X.init[0][g] = -32 * (int)__builtin_amdgcn_udot4(X.p[0][t + 1], ones, __builtin_amdgcn_udot4(X.p[0][t], ones, 0, false), false);
            X.init[1][g] = -32 * (int)__builtin_amdgcn_udot4(X.p[1][t + 1], ones, __builtin_amdgcn_udot4(X.p[1][t], ones, 0, false), false);
            X.init[2][g] = -32 * __builtin_amdgcn_sdot4((int)X.p[2][t + 1], (int)ones, __builtin_amdgcn_sdot4((int)X.p[2][t], (int)ones, 0, false), false);
        }
    } else {
        uint32_t s0 = 0, s1 = 0;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            s0 = __builtin_amdgcn_udot4(X.p[0][t], ones, s0, false);
            s1 = __builtin_amdgcn_udot4(X.p[1][t], ones, s1, false);
        }
        X.init[0][0] = -128 * (int)s0;
        X.init[1][0] = -128 * (int)s1;
        X.init[2][0] = 0; // the signed plane takes the signed weights
    }
}

// a * b + c for a, b in the signed 24-bit range.  The shifts state the range
// to the compiler, which then selects the full-rate v_mad_i32_i24 (it takes
// the low 24 bits of each factor, so the shifts fold away) instead of the
// quarter-rate 32-bit multiply.
__device__ __forceinline__ int mad_i24(int a, int b, int c)
{
    return ((a << 8) >> 8) * ((b << 8) >> 8) + c;
}

// 8 bytes starting `sh` bytes past the dword-aligned LDS address p.
__device__ __forceinline__ void lds_read8_at(const uint8_t *p, uint32_t sh, uint32_t &a,
                                             uint32_t &b)
{
    const uint32_t *q = reinterpret_cast<const uint32_t *>(p);
    const uint32_t w0 = q[0], w1 = q[1], w2 = q[2];
    a = __builtin_amdgcn_alignbyte(w1, w0, sh);
    b = __builtin_amdgcn_alignbyte(w2, w1, sh);
}

// The lane's share of one Q6_K block from its bytes, two dwords each:
// A = ql[64n + l0, +8), B = ql[64n + 32 + l0, +8), H = qh[32n + l0, +8),
// S = sc[8n, 8n + 8); dbits = the block's fp16 d; c = l0 >> 4 (which of the
// scale pairs the lane's positions use).
__device__ __forceinline__ float q6_dot_words(const uint32_t (&A)[2], const uint32_t (&B)[2],
                                              const uint32_t (&H)[2], const uint32_t (&S)[2],
                                              uint32_t dbits, int c, const SXD &X)
{
    const float d = h2f(dbits);
    int acc[3][4];
#pragma unroll
    for (int p = 0; p < 3; ++p)
#pragma unroll
        for (int g = 0; g < 4; ++g) acc[p][g] = X.init[p][g];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const uint32_t v[4] = {
            (A[t] & 0x0f0f0f0fu) | ((H[t] & 0x03030303u) << 4),
            (B[t] & 0x0f0f0f0fu) | ((H[t] & 0x0c0c0c0cu) << 2),
            ((A[t] >> 4) & 0x0f0f0f0fu) | (H[t] & 0x30303030u),
            ((B[t] >> 4) & 0x0f0f0f0fu) | ((H[t] >> 2) & 0x30303030u),
        };
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            acc[0][g] = (int)__builtin_amdgcn_udot4(v[g], X.p[0][2 * g + t], (uint32_t)acc[0][g], false);
            acc[1][g] = (int)__builtin_amdgcn_udot4(v[g], X.p[1][2 * g + t], (uint32_t)acc[1][g], false);
            acc[2][g] = __builtin_amdgcn_sdot4((int)v[g], (int)X.p[2][2 * g + t], acc[2][g], false);
        }
    }
    // scale-weighted sums per plane: |acc| <= 8 * 63 * 255, |sc| <= 128 (24-bit products)
    int T[3] = {0, 0, 0};
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int si = 2 * g + c; // byte of the 8 scales sc[8n..8n+7]
        const int sc = __builtin_amdgcn_sbfe(S[si >> 2], 8 * (si & 3), 8);
#pragma unroll
        for (int p = 0; p < 3; ++p) T[p] = mad_i24(sc, acc[p][g], T[p]);
    }
    const float v = fmaf(fmaf((float)T[2], 256.0f, (float)T[1]), 256.0f, (float)T[0]);
    return d * __builtin_ldexpf(v + X.poison, X.e - 22);
}

// The lane's share of one Q6_K block of the ring slot starting at `slot`
// (dword-aligned).
__device__ __forceinline__ float q6_dot_dig(const uint8_t *slot, const Q6DigLane &L,
                                            const SXD &X)
{
    uint32_t A[2], B[2], H[2], S[2];
    lds_read8_at(slot + L.a, L.sh, A[0], A[1]);
    lds_read8_at(slot + L.a + 32, L.sh, B[0], B[1]);
    lds_read8_at(slot + L.h, L.sh, H[0], H[1]);
    lds_read8_at(slot + L.s, L.sh, S[0], S[1]);
    return q6_dot_words(A, B, H, S, *reinterpret_cast<const uint16_t *>(slot + L.d), L.c, X);
}

// A Q8_0 block from its bytes: w = the 9 dwords from the one at or below its
// first quant, sh = that quant's byte within it, dbits = its fp16 d.
__device__ __forceinline__ float q80_dot_words(const uint32_t (&w)[9], uint32_t sh, uint32_t dbits,
                                               const SXD &X)
{
    const float d = h2f(dbits);
    uint32_t a0 = (uint32_t)X.init[0][0], a1 = (uint32_t)X.init[1][0];
    int a2 = 0;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const uint32_t q = __builtin_amdgcn_alignbyte(w[t + 1], w[t], sh);
        const uint32_t u = q ^ 0x80808080u; // q + 128 as unsigned bytes
        a0 = __builtin_amdgcn_udot4(u, X.p[0][t], a0, false);
        a1 = __builtin_amdgcn_udot4(u, X.p[1][t], a1, false);
        a2 = __builtin_amdgcn_sdot4((int)q, (int)X.p[2][t], a2, false);
    }
    const float v = fmaf(fmaf((float)a2, 256.0f, (float)(int)a1), 256.0f, (float)(int)a0);
    return d * __builtin_ldexpf(v + X.poison, X.e - 22);
}

// Q8_0 block at byte `off` of an LDS row.
__device__ __forceinline__ float q80_dot_dig(const uint8_t *row_lds, uint32_t off, const SXD &X)
{
    const uint32_t o = off + 2;
    const uint32_t *p = reinterpret_cast<const uint32_t *>(row_lds + (o & ~3u));
    uint32_t w[9];
#pragma unroll
    for (int i = 0; i < 9; ++i) w[i] = p[i];
    return q80_dot_words(w, o & 3u, lds_read_u16(row_lds, off), X);
}

// An IQ4_NL block from its bytes (element j = low nibble of qs[j], element
// j + 16 = high nibble): w = the 5 dwords from the one at or below its first
// quant, sh = that quant's byte within it, dbits = its fp16 d.
__device__ __forceinline__ float iq4nl_dot_words(const uint32_t (&w)[5], uint32_t sh, uint32_t dbits,
                                                 const SXD &X)
{
    const float d = h2f(dbits);
    uint32_t a0 = (uint32_t)X.init[0][0], a1 = (uint32_t)X.init[1][0];
    int a2 = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const uint32_t q = __builtin_amdgcn_alignbyte(w[t + 1], w[t], sh); // qs[4t..4t+3]
        uint32_t ul, uh; // grid + 128, elements 4t + b and 16 + 4t + b
        iq4nl_lookup2(q, ul, uh);
        a0 = __builtin_amdgcn_udot4(ul, X.p[0][t], a0, false);
        a1 = __builtin_amdgcn_udot4(ul, X.p[1][t], a1, false);
        a2 = __builtin_amdgcn_sdot4((int)(ul ^ 0x80808080u), (int)X.p[2][t], a2, false);
        a0 = __builtin_amdgcn_udot4(uh, X.p[0][4 + t], a0, false);
        a1 = __builtin_amdgcn_udot4(uh, X.p[1][4 + t], a1, false);
        a2 = __builtin_amdgcn_sdot4((int)(uh ^ 0x80808080u), (int)X.p[2][4 + t], a2, false);
    }
    const float v = fmaf(fmaf((float)a2, 256.0f, (float)(int)a1), 256.0f, (float)(int)a0);
    return d * __builtin_ldexpf(v + X.poison, X.e - 22);
}

// IQ4_NL block at byte `off` of an LDS row.
__device__ __forceinline__ float iq4nl_dot_dig(const uint8_t *row_lds, uint32_t off, const SXD &X)
{
    const uint32_t o = off + 2;
    const uint32_t *p = reinterpret_cast<const uint32_t *>(row_lds + (o & ~3u));
    uint32_t w[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) w[i] = p[i];
    return iq4nl_dot_words(w, o & 3u, lds_read_u16(row_lds, off), X);
}

// Staged digits of one segment in LDS: per lane 24 digit-plane dwords, 12
// accumulator starts, the exponent and the poison value (10 quads, quad-major
// so that a wave's 16-byte reads and writes are conflict-free).

__device__ __forceinline__ void sxd_store(const SXD &X, uint32_t (*d)[64][4], int lane)
{
    uint32_t dw[4 * kDigQuads];
#pragma unroll
    for (int p = 0; p < 3; ++p)
#pragma unroll
        for (int t = 0; t < 8; ++t) dw[8 * p + t] = X.p[p][t];
#pragma unroll
    for (int p = 0; p < 3; ++p)
#pragma unroll
        for (int g = 0; g < 4; ++g) dw[24 + 4 * p + g] = (uint32_t)X.init[p][g];
    dw[36] = (uint32_t)X.e;
    dw[37] = __float_as_uint(X.poison);
    dw[38] = dw[39] = 0;
#pragma unroll
    for (int q = 0; q < kDigQuads; ++q)
        *reinterpret_cast<uint4 *>(d[q][lane]) = make_uint4(dw[4 * q], dw[4 * q + 1], dw[4 * q + 2], dw[4 * q + 3]);
}

__device__ __forceinline__ void sxd_load(SXD &X, const uint32_t (*d)[64][4], int lane)
{
#pragma unroll
    for (int q = 0; q < kDigQuads; ++q) {
        const uint4 v = *reinterpret_cast<const uint4 *>(d[q][lane]);
        const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = 4 * q + e;
            if (i < 24) X.p[i / 8][i % 8] = vv[e];
            else if (i < 36) X.init[(i - 24) / 4][(i - 24) % 4] = (int)vv[e];
            else if (i == 36) X.e = (int)vv[e];
            else if (i == 37) X.poison = __uint_as_float(vv[e]);
        }
    }
}

// The walk itself over LDS the caller declares (ring: NW * D * sdig_slot
// bytes, 16-byte aligned; digs: the staged digits of sdig_share_cap(NW)
// segments unless ARGMAX; part: kSdigMaxRows x NW; wkey / wflag: NW each).
// PH: rows that are not 16-byte multiples (segments at a byte phase in their
// slots); without it every phase is 0 and the lane offsets are fixed.
template <int FMT, int NW, int D, bool ARGMAX, bool RESID, bool PH>
__device__ __forceinline__ void sdig_run(const uint8_t *__restrict__ W, const float *x, float *y,
                                         int outer, int nblk, int rpc, ArgPart *__restrict__ parts,
                                         const float *resid, int epi, uint8_t *ring,
                                         uint32_t (*digs)[kDigQuads][64][4], float (*part)[NW],
                                         unsigned long long *wkey, uint32_t *wflag)
{
    using F = SFmt<FMT>;
    // every copy instruction moves 64 x 16 bytes with all lanes on (lanes past the
    // segment re-read its last 16 bytes into the slot's tail), so the number of
    // copies in flight is a compile-time count and the explicit s_waitcnt vmcnt
    // waits below are exact (x and the copies are inline assembly the compiler
    // does not wait on by itself)
    constexpr int IPR = sdig_ipr(FMT); // copy instructions per row
    constexpr int SLOT = sdig_slot(FMT);
    static_assert(sdig_seg_bytes(FMT) == F::SEG_BYTES && sdig_seg_blocks(FMT) == F::SEG_BLOCKS,
                  "segment geometry");
    static_assert(SLOT >= F::SEG_BYTES + 16, "Q8_0 / IQ4_NL read one dword past a segment");
    // segments whose digits can be staged in LDS for the segment's other waves
    constexpr int SHC = sdig_share_cap(NW);

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int bid = (int)blockIdx.x, grid = (int)gridDim.x;
    const SdigWave g = sdig_wave(FMT, NW, D, SHC, outer, nblk, rpc, bid, grid, w);
    const int nseg = g.nseg, sg = g.sg;
    const bool share = g.share, producer = g.producer;
    const int seg_blocks = g.seg_blocks, nitems = g.nitems;

    // item k's row segment into slot k % D, from the 16-byte unit at or below
    // its first byte
    const uint32_t ring_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)ring;
    auto issue = [&](int k) {
        const size_t off = sdig_copy_row(g, FMT, k, bid, grid, rpc, outer);
        const uint32_t ph = PH ? sdig_phase(off) : 0u;
        const int units = sdig_units(g, ph);
        const uint8_t *src = W + (off - ph);
#pragma unroll
        for (int i = 0; i < IPR; ++i)
            lds_copy16(src + sdig_copy_lane(units, i, lane), ring_lds + sdig_copy_dst(g, FMT, D, k, i));
    };

    // x first, then the first D rows' copies, all in flight together; the
    // digits wait only for x (vmcnt counts completions in issue order).
    float4 xv[8];
    bool xact = false;
    if (producer) // wave-uniform
        xact = staged_dig_issue<FMT>(x + g.x0, lane, seg_blocks, xv);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < D; ++k)
        issue(k);
    SXD X;
    if (producer) {
        wait_vmcnt(D * IPR);
        staged_dig_pin(xv);
        __builtin_amdgcn_sched_barrier(0);
        staged_dig_x<FMT>(xv, xact, X);
        if (share)
            sxd_store(X, digs[sg], lane);
    }
    if (share) { // workgroup-uniform
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        lds_barrier();
        if (!producer)
            sxd_load(X, digs[sg], lane);
    }

    const Q6DigLane q6l = q6_dig_lane(lane); // used by Q6_K only
    // rows of several segments end in the chunk epilogue, one thread per row:
    // the first chunk's epilogue value is loaded now, under the weight stream,
    // instead of as a dependent load at the end (later chunks load theirs in
    // their epilogue)
    float rv0 = 0.0f;
    if constexpr (RESID) {
        if (nseg > 1 && g.my_chunks > 0) {
            const SdigChunk c0 = sdig_chunk(g, 0, bid, grid, rpc, outer);
            if (tid < c0.nrows)
                rv0 = resid[c0.row0 + tid];
        }
    }
    unsigned long long key = 0, ukey = 0; // ukey / ufl: rows a wave holds whole (wave-uniform)
    uint32_t fl = 0, ufl = 0;
    int k = 0;
    for (int ci = 0; ci < g.my_chunks; ++ci) {
        const SdigChunk c = sdig_chunk(g, ci, bid, grid, rpc, outer);
        const int row0 = c.row0, nrows = c.nrows, mine = c.mine;
        // the lane's share of the dot product of the row segment at byte phase
        // ph of ring slot `slot`
        auto dot_at = [&](uint32_t slot, uint32_t ph) {
            float v = 0.0f;
            if constexpr (FMT == kQ6_K) {
                if ((lane >> 3) < seg_blocks)
                    v = q6_dot_dig(ring + slot, PH ? q6_dig_lane_at(q6l, ph) : q6l, X);
            } else if constexpr (FMT == kIQ4_NL) {
                if (lane < seg_blocks)
                    v = iq4nl_dot_dig(ring + slot, sdig_blk_off(FMT, lane) + ph, X);
            } else {
                if (lane < seg_blocks)
                    v = q80_dot_dig(ring + slot, sdig_blk_off(FMT, lane) + ph, X);
            }
            return v;
        };
        auto finish = [&](int rr, float v) {
            if (nseg == 1) { // the wave holds the whole row: finish it here
                const int row = row0 + sdig_chunk_row(g, rr);
                if constexpr (RESID)
                    v = epi_apply(resid[row], v, epi); // wave-uniform: a scalar load
                if (y && lane == 0)
                    y[row] = v;
                if constexpr (ARGMAX)
                    argmax_fold_uniform(v, (uint32_t)row, ukey, ufl);
            } else if (lane == 0) {
                part[sdig_chunk_row(g, rr)][sg] = v;
            }
        };
        for (int rr = 0; rr < mine; ++rr, ++k) {
            const uint32_t ph = PH ? sdig_phase(sdig_seg_off(g, FMT, row0 + sdig_chunk_row(g, rr))) : 0u;
            wait_vmcnt(IPR * sdig_wait_items(g, D, k));
            finish(rr, wave_sum(dot_at(sdig_copy_dst(g, FMT, D, k, 0), ph)));
            if (k + D < nitems)
                issue(k + D); // slot k % D has been read
        }
        if (nseg == 1) // wave-uniform for the whole workgroup: no exchange, no barriers
            continue;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); // part[] writes done
        lds_barrier();
        for (int i = tid; i < nrows; i += NW * 64) { // rpc <= 64: one row per thread
            float v = 0.0f;
            for (int q = 0; q < nseg; ++q)
                v += part[i][q];
            if constexpr (RESID)
                v = epi_apply(ci == 0 ? rv0 : resid[row0 + i], v, epi); // resid may be y
            if (y)
                y[row0 + i] = v;
            if constexpr (ARGMAX)
                argmax_fold(v, (uint32_t)(row0 + i), key, fl);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        lds_barrier(); // part[] is free for the next chunk
    }
    if constexpr (ARGMAX) {
        key = ukey > key ? ukey : key;
        fl |= ufl;
        argmax_wave_reduce(key, fl);
        if (lane == 0) {
            wkey[w] = key;
            wflag[w] = fl;
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        lds_barrier();
        if (tid == 0) {
            unsigned long long kk = wkey[0];
            uint32_t f = wflag[0];
#pragma unroll
            for (int i = 1; i < NW; ++i) {
                kk = wkey[i] > kk ? wkey[i] : kk;
                f |= wflag[i];
            }
            parts[blockIdx.x].key = kk;
            parts[blockIdx.x].flags = f;
            parts[blockIdx.x].pad = 0;
        }
    }
    __builtin_amdgcn_s_waitcnt(0); // every copy has landed before the workgroup ends
}

template <int FMT, int NW, int D, bool ARGMAX, bool RESID, bool PH>
__global__ __launch_bounds__(NW * 64) void k_gemv_sdig(const uint8_t *__restrict__ W,
                                                       const float *x, float *y, int outer, int nblk,
                                                       int rpc, ArgPart *__restrict__ parts,
                                                       const float *resid, int epi)
{
    constexpr int SHC = sdig_share_cap(NW);
    __shared__ __attribute__((aligned(16))) uint8_t ring[NW * D * sdig_slot(FMT)];
    __shared__ __attribute__((aligned(16))) uint32_t digs[SHC > 0 ? SHC : 1][kDigQuads][64][4];
    __shared__ float part[kSdigMaxRows][NW]; // one column per segment (nseg <= NW)
    __shared__ unsigned long long wkey[NW];
    __shared__ uint32_t wflag[NW];
    sdig_run<FMT, NW, D, ARGMAX, RESID, PH>(W, x, y, outer, nblk, rpc, parts, resid, epi, ring, digs,
                                            part, wkey, wflag);
}

// ------------------------------------------------------------------------
// launchers
// ------------------------------------------------------------------------
// CUs of the current device, queried once per device (launch plans ask on
// every launch)
int device_cus()
{
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return 256;
    int ncu = cached[dev].load(std::memory_order_relaxed);
    if (ncu <= 0) {
        ncu = 256;
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
        cached[dev].store(ncu, std::memory_order_relaxed);
    }
    return ncu;
}

// Rows of 17..64 blocks whose 8-wave workgroups (two rows per wave for the
// GEMV, one gate/up row pair for the fused gate/up) would not divide evenly
// over the CUs take the persistent multi-pass kernel; the fused gate/up only
// with more row pairs than one per wave of one workgroup per CU (5120 ->
// 1280 5.5 us serial against 5.9, 8192 -> 1024 6.1 against 6.4; 5120 ->
// 13824 20.6-21.2 against 26.0-26.4).
static bool kwide_takes_kpm(int nblk, int outer, bool gateup)
{
    const int R = gateup ? 1 : 2;
    return nblk > 16 && nblk <= 4 * 16 && ((outer + 8 * R - 1) / (8 * R)) % device_cus() != 0 &&
           (!gateup || (outer + 7) / 8 > device_cus());
}

// Rows of at most 16 blocks with at least four 8-wave row groups per wave
// over one workgroup per CU take the persistent kernel.
static bool kwide_takes_kpers(int nblk, int outer) { return nblk <= 16 && outer >= 4 * 8 * 256; }

// No more one-row workgroups of 8 waves than CUs: one row per wave.
static bool kwide_one_row(int outer) { return (outer + 7) / 8 <= device_cus(); }

// k_gemv_kpm with the smallest pass capacity that holds the row.
template <int FMT, bool GATEUP, bool EXT>
static void launch_kpm(int npass, int grid, const uint8_t *W, const uint8_t *W2, const float *x,
                       float *y, int outer, int nblk, const float *nw, float eps, const float *resid,
                       int epi, hipStream_t s)
{
    constexpr int NWV = 8, NB = 2;
    if (npass <= 2)
        hipLaunchKernelGGL((k_gemv_kpm<FMT, 1, GATEUP, EXT, NWV, NB, 2>), dim3(grid), dim3(NWV * 64), 0, s,
                           W, W2, x, y, outer, nblk, nw, eps, resid, epi);
    else
        hipLaunchKernelGGL((k_gemv_kpm<FMT, 1, GATEUP, EXT, NWV, NB, 4>), dim3(grid), dim3(NWV * 64), 0, s,
                           W, W2, x, y, outer, nblk, nw, eps, resid, epi);
}

// Q4_K / Q5_K: 8-wave workgroups; two rows per wave for the GEMV, one gate and
// one up row per wave for the fused gate/up (measured on MI355X at 4096 x 4096
// and 2 x 12288 x 4096).  Rows of at most 4096 columns with at least four row
// groups per wave over one workgroup per CU take the persistent kernel (2 x
// 12288 x 4096 gate/up 12.7 us against 13.9 us; at 4096 x 4096 one row group
// per wave is all there is and the plain kernel is faster).  Rows of 17..64
// blocks take the persistent multi-pass kernel when the serial kernel's
// workgroups do not divide evenly over the CUs (5120 x 5120 7.8-8.8 us
// against 8.5-8.6, 5120 x 13824 13.9-15.1 against 16.2-16.4, 13824 x 5120
// 14.6-14.9 against 15.4-15.6); at 4096 rows the serial kernel's one
// workgroup per CU is faster (4096 x 11008 9.7-10.0 us against 10.7-11.2).
template <int FMT, bool GATEUP>
static hipError_t launch_kwide(const void *w, const void *w2, const float *x, float *y,
                               int inner, int outer, hipStream_t s, const float *nw = nullptr,
                               float eps = 0.0f, const float *resid = nullptr, int epi = kEpiAdd)
{
    constexpr int NWV = 8, R = GATEUP ? 1 : 2, NB = 2;
    const int nblk = inner / 256;
    const bool ext = GATEUP ? nw != nullptr : resid != nullptr;
    const uint8_t *W = (const uint8_t *)w, *W2 = (const uint8_t *)w2;
    if (kwide_takes_kpers(nblk, outer)) {
        const int grid = std::max(1, std::min(device_cus(), (outer + NWV - 1) / NWV));
        if (ext)
            hipLaunchKernelGGL((k_gemv_kpers<FMT, 1, GATEUP, true, NWV, NB>), dim3(grid), dim3(NWV * 64),
                               0, s, W, W2, x, y, outer, nblk, nw, eps, resid, epi);
        else
            hipLaunchKernelGGL((k_gemv_kpers<FMT, 1, GATEUP, false, NWV, NB>), dim3(grid), dim3(NWV * 64),
                               0, s, W, W2, x, y, outer, nblk, nw, eps, resid, epi);
    } else if (FMT != kIQ4_NL && FMT != kQ8_0 && kwide_takes_kpm(nblk, outer, GATEUP)) {
        if constexpr (FMT != kIQ4_NL && FMT != kQ8_0) {
            const int grid = std::max(1, std::min(device_cus(), (outer + NWV - 1) / NWV));
            const int npass = (nblk + 15) / 16;
            if (ext)
                launch_kpm<FMT, GATEUP, true>(npass, grid, W, W2, x, y, outer, nblk, nw, eps, resid, epi, s);
            else
                launch_kpm<FMT, GATEUP, false>(npass, grid, W, W2, x, y, outer, nblk, nw, eps, resid, epi, s);
        }
    } else if (!GATEUP && kwide_one_row(outer)) {
        // no more one-row workgroups than CUs: one row per wave, all of them
        // at once (2048 x 2048 2.8-3.1 us against 3.5-3.6 with two rows per
        // wave; 3072 x 3072 keeps two rows: 1.5 one-row workgroups per CU
        // measured 4.5 us against 4.1)
        const dim3 grid((outer + NWV - 1) / NWV);
        if (ext)
            hipLaunchKernelGGL((k_gemv_kwide<FMT, 1, false, true, NWV>), grid, dim3(NWV * 64), 0, s, W,
                               W2, x, y, outer, nblk, nw, eps, resid, epi);
        else
            hipLaunchKernelGGL((k_gemv_kwide<FMT, 1, false, false, NWV>), grid, dim3(NWV * 64), 0, s, W,
                               W2, x, y, outer, nblk, nw, eps, resid, epi);
    } else {
        const dim3 grid((outer + NWV * R - 1) / (NWV * R));
        if (ext)
            hipLaunchKernelGGL((k_gemv_kwide<FMT, R, GATEUP, true, NWV>), grid, dim3(NWV * 64), 0, s, W,
                               W2, x, y, outer, nblk, nw, eps, resid, epi);
        else
            hipLaunchKernelGGL((k_gemv_kwide<FMT, R, GATEUP, false, NWV>), grid, dim3(NWV * 64), 0, s, W,
                               W2, x, y, outer, nblk, nw, eps, resid, epi);
    }
    return hipGetLastError();
}

template <int FMT, bool ARGMAX, int NWV, int D, bool PH>
static void launch_sdig_d(const void *w, const float *x, float *y, int nblk, int outer,
                          const SdigPlan &p, void *parts, hipStream_t s, const float *resid, int epi)
{
    if (!ARGMAX && resid) // the lm_head has no residual
        hipLaunchKernelGGL((k_gemv_sdig<FMT, NWV, D, ARGMAX, !ARGMAX, PH>), dim3(p.grid), dim3(NWV * 64), 0,
                           s, (const uint8_t *)w, x, y, outer, nblk, p.rpc, (ArgPart *)parts, resid, epi);
    else
        hipLaunchKernelGGL((k_gemv_sdig<FMT, NWV, D, ARGMAX, false, PH>), dim3(p.grid), dim3(NWV * 64), 0,
                           s, (const uint8_t *)w, x, y, outer, nblk, p.rpc, (ArgPart *)parts, resid, epi);
}

// Ring depth 3 only for the 8-wave (one-segment) plans that pick it.
template <int FMT, bool ARGMAX, int NWV, bool PH>
static void launch_sdig_ph(const void *w, const float *x, float *y, int nblk, int outer,
                           const SdigPlan &p, void *parts, hipStream_t s, const float *resid, int epi)
{
    if constexpr (NWV == 8) {
        if (p.d == 3) {
            launch_sdig_d<FMT, ARGMAX, NWV, 3, PH>(w, x, y, nblk, outer, p, parts, s, resid, epi);
            return;
        }
    }
    launch_sdig_d<FMT, ARGMAX, NWV, 2, PH>(w, x, y, nblk, outer, p, parts, s, resid, epi);
}

template <int FMT, bool ARGMAX, int NWV>
static void launch_sdig_nw(const void *w, const float *x, float *y, int nblk, int outer,
                           const SdigPlan &p, void *parts, hipStream_t s, const float *resid, int epi)
{
    if (sdig_phased(FMT, nblk))
        launch_sdig_ph<FMT, ARGMAX, NWV, true>(w, x, y, nblk, outer, p, parts, s, resid, epi);
    else
        launch_sdig_ph<FMT, ARGMAX, NWV, false>(w, x, y, nblk, outer, p, parts, s, resid, epi);
}

// Q6_K / Q8_0 / IQ4_NL rows of 1..16 segments through the streamed digit
// kernel, with the waves and grid sdig_plan chooses; wider rows through the
// byte-granular kernel (no argmax fusion for them: the caller checks
// lm_head_fusable).
template <int FMT, bool ARGMAX>
static hipError_t launch_sdig(const void *w, const float *x, float *y, int inner, int outer,
                              void *parts, hipStream_t s, const float *resid = nullptr,
                              int epi = kEpiAdd)
{
    const int nblk = inner / block_elems(FMT);
    if (!sdig_rows_ok(FMT, nblk))
        return ARGMAX ? hipErrorInvalidValue : launch_gemv_generic(FMT, w, x, y, inner, outer, s, resid, epi);
    const SdigPlan p = sdig_plan(FMT, nblk, outer, ARGMAX, device_cus());
    if (p.d != 2 && !(p.d == 3 && p.nw == 8))
        return hipErrorInvalidValue; // no such instantiation
    switch (p.nw) {
    case 8: launch_sdig_nw<FMT, ARGMAX, 8>(w, x, y, nblk, outer, p, parts, s, resid, epi); break;
    case 12: launch_sdig_nw<FMT, ARGMAX, 12>(w, x, y, nblk, outer, p, parts, s, resid, epi); break;
    case 16: launch_sdig_nw<FMT, ARGMAX, 16>(w, x, y, nblk, outer, p, parts, s, resid, epi); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gemv(int type, const void *w, const float *x, float *y, int inner, int outer,
                       hipStream_t s, const float *resid, int epi)
{
    switch (type) {
    case kQ4_K: return launch_kwide<kQ4_K, false>(w, nullptr, x, y, inner, outer, s, nullptr, 0.0f, resid, epi);
    case kQ5_K: return launch_kwide<kQ5_K, false>(w, nullptr, x, y, inner, outer, s, nullptr, 0.0f, resid, epi);
    case kQ6_K: return launch_sdig<kQ6_K, false>(w, x, y, inner, outer, nullptr, s, resid, epi);
    case kQ8_0:
        // rows of one pass (at most 4096 columns in whole 256-column units)
        // on the wide lane layout, measured against the streamed kernel in one
        // process: 151936 x 2048 60-62 us against 67.5, 5120 x 3072 6.6 against
        // 8.2, 8192 x 4096 8.9 against 9.4, 4096 x 2048 4.6 against 4.8,
        // 4096 x 4096 6.1-6.2 against 6.1-6.3; rows of several passes stay on
        // the streamed kernel (4096 x 14336 16.2 against 17.7)
        return inner % 256 == 0 && inner <= 4096
                   ? launch_kwide<kQ8_0, false>(w, nullptr, x, y, inner, outer, s, nullptr, 0.0f, resid, epi)
                   : launch_sdig<kQ8_0, false>(w, x, y, inner, outer, nullptr, s, resid, epi);
    case kIQ4_NL:
        // rows of whole 256-column units take the wide kernels' lane layout,
        // except where the persistent multi-pass kernel would run (its IQ4_NL
        // dot from LDS digits measured slower than the streamed kernel:
        // 5120 x 5120 10.9 us against 10.3)
        return inner % 256 == 0 && !kwide_takes_kpm(inner / 256, outer, false)
                   ? launch_kwide<kIQ4_NL, false>(w, nullptr, x, y, inner, outer, s, nullptr, 0.0f, resid, epi)
                   : launch_sdig<kIQ4_NL, false>(w, x, y, inner, outer, nullptr, s, resid, epi);
    default: return hipErrorInvalidValue;
    }
}

bool gemv_norm_fusable(int type, int inner, int)
{
    return (type == kQ4_K || type == kQ5_K) && inner % 256 == 0 && inner / 256 <= 16;
}

template <int FMT>
static void launch_kwide_norm(const void *w, const float *x, const float *nw, float eps, float *y,
                              int inner, int outer, hipStream_t s)
{
    constexpr int NWV = 8;
    const int nblk = inner / 256;
    const uint8_t *W = (const uint8_t *)w;
    if (kwide_takes_kpers(nblk, outer))
        hipLaunchKernelGGL((k_gemv_kpers_norm<FMT, 1, NWV, 2>),
                           dim3(std::max(1, std::min(device_cus(), (outer + NWV - 1) / NWV))),
                           dim3(NWV * 64), 0, s, W, x, y, outer, nblk, nw, eps);
    else if (kwide_one_row(outer))
        hipLaunchKernelGGL((k_gemv_kwide_norm<FMT, 1, NWV>), dim3((outer + NWV - 1) / NWV), dim3(NWV * 64),
                           0, s, W, x, y, outer, nblk, nw, eps);
    else
        hipLaunchKernelGGL((k_gemv_kwide_norm<FMT, 2, NWV>), dim3((outer + 2 * NWV - 1) / (2 * NWV)),
                           dim3(NWV * 64), 0, s, W, x, y, outer, nblk, nw, eps);
}

hipError_t launch_gemv_norm(int type, const void *w, const float *x, const float *nw, float eps,
                            float *y, int inner, int outer, hipStream_t s)
{
    if (!gemv_norm_fusable(type, inner, outer))
        return hipErrorNotSupported;
    if (type == kQ4_K)
        launch_kwide_norm<kQ4_K>(w, x, nw, eps, y, inner, outer, s);
    else
        launch_kwide_norm<kQ5_K>(w, x, nw, eps, y, inner, outer, s);
    return hipGetLastError();
}

bool gate_up_fusable(int gate_type, int up_type)
{
    return gate_type == up_type && (gate_type == kQ4_K || gate_type == kQ5_K);
}

hipError_t launch_gate_up_swiglu(int type, const void *wg, const void *wu, const float *x,
                                 float *h, int hidden, int inter, hipStream_t s,
                                 const float *norm_w, float eps)
{
    switch (type) {
    case kQ4_K: return launch_kwide<kQ4_K, true>(wg, wu, x, h, hidden, inter, s, norm_w, eps);
    case kQ5_K: return launch_kwide<kQ5_K, true>(wg, wu, x, h, hidden, inter, s, norm_w, eps);
    default: return hipErrorInvalidValue;
    }
}

bool lm_head_fusable(int type, int hidden)
{
    return (type == kQ6_K || type == kQ8_0) && sdig_rows_ok(type, hidden / block_elems(type));
}

// 256 threads, four 16-byte partials in flight per thread (measured on MI355X
// for the lm_head's 768 partials: 0.9 us per call less than 1024 threads; a
// single wave gains nothing)
static void launch_argmax_finalize(const void *ws, int nparts, int32_t *token, uint32_t *flags,
                                   hipStream_t s)
{
    hipLaunchKernelGGL(k_argmax_finalize, dim3(1), dim3(256), 0, s, (const ArgPart *)ws, nparts,
                       token, flags);
}

int lm_head_argmax_parts(int type, int hidden, int vocab, bool fused)
{
    if (!fused) // the GEMV, then the standalone argmax over the logits
        return (int)std::min<int64_t>(std::max<int64_t>(1, ((int64_t)vocab + 255) / 256), kArgMaxParts);
    return sdig_plan(type, hidden / block_elems(type), vocab, true, device_cus()).grid;
}

hipError_t launch_lm_head_argmax(int type, const void *w, const float *x, float *logits,
                                 int32_t *token, uint32_t *flags, int hidden, int vocab,
                                 void *ws, hipStream_t s)
{
    if (!lm_head_fusable(type, hidden))
        return hipErrorInvalidValue;
    hipError_t e;
    switch (type) {
    case kQ6_K: e = launch_sdig<kQ6_K, true>(w, x, logits, hidden, vocab, ws, s); break;
    case kQ8_0: e = launch_sdig<kQ8_0, true>(w, x, logits, hidden, vocab, ws, s); break;
    default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess)
        return e;
    launch_argmax_finalize(ws, lm_head_argmax_parts(type, hidden, vocab, true), token, flags, s);
    return hipGetLastError();
}

hipError_t launch_argmax(const float *v, int64_t n, int32_t *token, uint32_t *flags, void *ws,
                         hipStream_t s)
{
    int64_t blocks = (n + 255) / 256;
    if (blocks > kArgMaxParts) blocks = kArgMaxParts;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(k_argmax_partials, dim3((unsigned)blocks), dim3(256), 0, s, v, n,
                       (ArgPart *)ws);
    launch_argmax_finalize(ws, (int)blocks, token, flags, s);
    return hipGetLastError();
}

} // namespace ihip
