// kq_gemv.hip -- gfx950 dequant-fused GEMV kernels for GGML K-quant/Q8_0
// weights and fp32 activations: y[r] = sum_c W[r,c] x[c].
//
// Semantics: the fp32-activation path of Inferno.jl's mul_quant_mat_vec
// (src/ModelCPU.jl:285-379) with the weights of src/Dequant.jl:304-601.
// Activations stay fp32 (the reference C path's int8 re-quantization of x,
// src/kernels/quant_kernels.c:166-194, is not used: it breaks the
// 1e-4*||w_row||*||x|| bound).
//
// A decode GEMV is a single pass over the weight bytes, so every kernel here
// is built to put all of a wave's weight loads in flight before it waits on
// any of them, to reuse each lane's x registers over several rows, and to
// keep the per-weight ALU work at one byte convert plus one FMA (the
// `dmin*m` term of Q4_K/Q5_K and the -32 offset of Q6_K are folded into
// per-sub-block sums of x, which all rows share).
//
//   * Q4_K / Q5_K ("wide" kernels): blocks are 16-byte multiples, so lanes
//     load straight from HBM with 128-bit loads.  A wave covers 16 blocks
//     (4096 columns) of R rows per pass: lane = (block, sub-block pair), 64
//     weights per lane per row.
//   * Q6_K (210 B) and Q8_0 (34 B) blocks are not 16-byte aligned, but 8 of
//     them are (1680 B / 272 B).  Each wave copies its own rows into a
//     private LDS region with gfx950's direct-to-LDS 128-bit loads (no
//     registers, no workgroup barrier), every segment of the row in flight
//     at once, then re-slices blocks from LDS ("staged" kernels).
//   * Greedy argmax (lm_head) is fused into the staged kernel's epilogue:
//     each workgroup writes one (value, index) partial to its own slot and a
//     one-workgroup kernel reduces the partials, so no two workgroups touch
//     the same address.
#include "inferno_hip.h"

#include <algorithm>
#include "kq_common.h"
#include "kq_launch.h"
#include "kq_sdig_plan.h"

namespace ihip {

// ------------------------------------------------------------------------
// Q4_K / Q5_K wide kernels
// ------------------------------------------------------------------------
template <int FMT>
struct KFmt;
template <>
struct KFmt<kQ4_K> {
    static constexpr int BYTES = 144, QS = 16;
};
template <>
struct KFmt<kQ5_K> {
    static constexpr int BYTES = 176, QS = 48;
};

// Lane geometry inside a 16-block (4096-column) pass: block b = lane >> 2,
// sub-block pair j = lane & 3.  The lane's weights are qs[32j, 32j+32) of
// block b: low nibbles are elements 64j + l (sub-block 2j), high nibbles
// 64j + 32 + l (sub-block 2j+1), l = 0..31 (src/Dequant.jl:364-371).
//
// The weight bytes go straight to registers (three 128-bit loads per row and
// lane).  x is read once per workgroup with contiguous loads and kept in LDS
// in a padded layout (4 floats of padding after every 64) under which a
// lane's 16-byte reads hit distinct banks across the wave; the workgroup also
// leaves the sum of every 32-element sub-block of x there.  Loads are issued
// x first, then every row's weights, so x can be staged while the weights are
// still in flight, and each row is reduced as soon as its own bytes land.
struct XWide {
    float a[32], b[32];
    float sa, sb;
};

constexpr int kXPadFloats = 4096 + 4096 / 64 * 4;
// float4s of a 4096-element pass per thread of an NT-thread workgroup (768
// threads: two, the second only for threads below 256)
__host__ __device__ constexpr int xnv(int nt) { return (1024 + nt - 1) / nt; }
__device__ __forceinline__ int xpad(int i) { return i + ((i >> 6) << 2); }

// Stage x[col0, col0 + 4096) (zeros past `inner`) and its 128 sub-block sums.
// `xv` holds this thread's float4s of x (NT threads: 1024 / NT each), loaded
// by the caller.
template <int NT>
__device__ __forceinline__ void x_stage(float *xs, float *xsum, const float4 (&xv)[1024 / NT])
{
    static_assert(1024 % NT == 0, "fp32 staging: NT divides 1024");
    const int tid = threadIdx.x;
#pragma unroll
    for (int k = 0; k < 1024 / NT; ++k) {
        const int i = 4 * (tid + NT * k);
        *reinterpret_cast<float4 *>(xs + xpad(i)) = xv[k];
        // 8 consecutive threads hold one 32-element sub-block
        float t = (xv[k].x + xv[k].y) + (xv[k].z + xv[k].w);
        t = dpp_add<0xb1, 0xf>(t);  // pairs
        t = dpp_add<0x4e, 0xf>(t);  // quads
        t = dpp_add<0x141, 0xf>(t); // 8 lanes (row_half_mirror)
        if ((tid & 7) == 0)
            xsum[(tid + NT * k) >> 3] = t;
    }
}

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

__device__ __forceinline__ void x_from_lds(const float *xs, const float *xsum, int b, int j,
                                           XWide &X)
{
    const int base = 256 * b + 64 * j;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const float4 va = *reinterpret_cast<const float4 *>(xs + xpad(base + 4 * t));
        const float4 vb = *reinterpret_cast<const float4 *>(xs + xpad(base + 32 + 4 * t));
        X.a[4 * t + 0] = va.x; X.a[4 * t + 1] = va.y; X.a[4 * t + 2] = va.z; X.a[4 * t + 3] = va.w;
        X.b[4 * t + 0] = vb.x; X.b[4 * t + 1] = vb.y; X.b[4 * t + 2] = vb.z; X.b[4 * t + 3] = vb.w;
    }
    const float2 s2 = *reinterpret_cast<const float2 *>(xsum + 8 * b + 2 * j);
    X.sa = s2.x;
    X.sb = s2.y;
}

// The block bytes one lane needs for one row: header (d, dmin, scales), its
// 32 qs bytes and (Q5_K) the 32 qh bytes.
struct KBytes {
    uint4 h, q0, q1, e0, e1;
};

template <int FMT>
__device__ __forceinline__ void kbytes_load(const uint8_t *__restrict__ blk, int j, KBytes &B)
{
    using F = KFmt<FMT>;
    B.h = *reinterpret_cast<const uint4 *>(blk);
    B.q0 = *reinterpret_cast<const uint4 *>(blk + F::QS + 32 * j);
    B.q1 = *reinterpret_cast<const uint4 *>(blk + F::QS + 32 * j + 16);
    if constexpr (FMT == kQ5_K) {
        B.e0 = *reinterpret_cast<const uint4 *>(blk + 16);
        B.e1 = *reinterpret_cast<const uint4 *>(blk + 32);
    }
}

typedef float f32x2 __attribute__((ext_vector_type(2)));

// One lane's contribution to one row.
//
// Q4_K converts nibbles with v_cvt_pk_f32_fp8, two per instruction: a byte
// 0000qqqq is the OCP e4m3 encoding of q * 2^-9 exactly (q3 becomes the
// exponent's low bit, q2..q0 the mantissa; 0..7 are e4m3 subnormals, which
// gfx950 converts exactly), so the sums are formed in units of 2^-9 and the
// exact power-of-two factor 512 is applied once per sub-block.  Q5_K's 5-bit
// values are not linear in e4m3 and use v_cvt_f32_ubyte.
template <int FMT>
__device__ __forceinline__ float kwide_dot(const KBytes &B, int j, const XWide &X)
{
    const uint32_t qw[8] = {B.q0.x, B.q0.y, B.q0.z, B.q0.w, B.q1.x, B.q1.y, B.q1.z, B.q1.w};
    float sa0 = 0.0f, sa1 = 0.0f, sb0 = 0.0f, sb1 = 0.0f;
    if constexpr (FMT == kQ4_K) {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t lo = qw[t] & 0x0f0f0f0fu;
            const uint32_t hi = (qw[t] >> 4) & 0x0f0f0f0fu;
            const f32x2 l01 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false);
            const f32x2 l23 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);
            const f32x2 h01 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false);
            const f32x2 h23 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
            sa0 = fmaf(l01[0], X.a[4 * t + 0], sa0);
            sa1 = fmaf(l01[1], X.a[4 * t + 1], sa1);
            sa0 = fmaf(l23[0], X.a[4 * t + 2], sa0);
            sa1 = fmaf(l23[1], X.a[4 * t + 3], sa1);
            sb0 = fmaf(h01[0], X.b[4 * t + 0], sb0);
            sb1 = fmaf(h01[1], X.b[4 * t + 1], sb1);
            sb0 = fmaf(h23[0], X.b[4 * t + 2], sb0);
            sb1 = fmaf(h23[1], X.b[4 * t + 3], sb1);
        }
        sa0 = (sa0 + sa1) * 512.0f;
        sb0 = (sb0 + sb1) * 512.0f;
    } else {
        // qh[l] bit 2j lifts element 64j + l, bit 2j+1 element 64j + 32 + l;
        // shift both bits down to bit positions 0 and 1 of each byte once
        const uint32_t sh = 2 * j;
        const uint32_t ew[8] = {B.e0.x >> sh, B.e0.y >> sh, B.e0.z >> sh, B.e0.w >> sh,
                                B.e1.x >> sh, B.e1.y >> sh, B.e1.z >> sh, B.e1.w >> sh};
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            uint32_t lo = (qw[t] & 0x0f0f0f0fu) | ((ew[t] & 0x01010101u) << 4);
            uint32_t hi = ((qw[t] >> 4) & 0x0f0f0f0fu) | ((ew[t] & 0x02020202u) << 3);
            lo = opaque(lo);
            hi = opaque(hi);
            sa0 = fmaf(ubyte_f(lo, 0), X.a[4 * t + 0], sa0);
            sa1 = fmaf(ubyte_f(lo, 1), X.a[4 * t + 1], sa1);
            sa0 = fmaf(ubyte_f(lo, 2), X.a[4 * t + 2], sa0);
            sa1 = fmaf(ubyte_f(lo, 3), X.a[4 * t + 3], sa1);
            sb0 = fmaf(ubyte_f(hi, 0), X.b[4 * t + 0], sb0);
            sb1 = fmaf(ubyte_f(hi, 1), X.b[4 * t + 1], sb1);
            sb0 = fmaf(ubyte_f(hi, 2), X.b[4 * t + 2], sb0);
            sb1 = fmaf(ubyte_f(hi, 3), X.b[4 * t + 3], sb1);
        }
        sa0 += sa1;
        sb0 += sb1;
    }
    const float d = h2f(B.h.x & 0xffffu), dmin = h2f(B.h.x >> 16);
    float scA, mA, scB, mB;
    k_scale_min_pair(B.h.y, B.h.z, B.h.w, j, scA, mA, scB, mB);
    const float pos = fmaf(scA, sa0, scB * sb0);
    const float neg = fmaf(mA, X.sa, mB * X.sb);
    return fmaf(d, pos, -(dmin * neg));
}

// ---- integer-digit activations -------------------------------------------
// The dot of a lane's nibbles with x can run on the integer dot units
// (v_dot4_{u32_u8,i32_i8}: four byte products and the accumulate in one
// instruction) when x is written as an integer.  Each 32-element sub-block of
// x is scaled by 2^(22-e), e the binary exponent of the sub-block's largest
// |x| (|x| < 2^e), and truncated to an integer X with |X| < 2^22: the error of
// x ~ X * 2^(e-22) is below 2^(e-22) <= |x|max * 2^-21, so a dot product of n
// such values is off by less than sqrt(n) * 2^-21 * ||w||_2 ||x||_2 (3.1e-5
// relative at n = 4096, against the 1e-4 row bound, whatever the data; about
// 1e-7 for random data).  X is split into three byte digits,
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

// One lane's contribution to one row with digit activations: the same sum as
// kwide_dot.
template <int FMT>
__device__ __forceinline__ float kdig_dot(const KBytes &B, int j, const XDig &X)
{
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
template <int FMT, int R, bool GATEUP, bool DIG, bool EXT, int NWV>
__global__ __launch_bounds__(NWV * 64) void k_gemv_kwide(const uint8_t *__restrict__ W,
                                                    const uint8_t *__restrict__ W2,
                                                    const float *__restrict__ x,
                                                    float *y, int outer, int nblk,
                                                    const float *__restrict__ nw, float eps,
                                                    const float *resid, int epi)
{
    using F = KFmt<FMT>;
    constexpr int NW = GATEUP ? 2 : 1;
    constexpr bool NORM = GATEUP && EXT, RESID = !GATEUP && EXT;
    constexpr int NT = NWV * 64, NXV = xnv(NT);
    static_assert(DIG || 1024 % NT == 0, "fp32 staging: NT divides 1024");
    // fp32 x (kXPadFloats) or its three digit planes (3 * kDigPlaneDw dwords)
    __shared__ __attribute__((aligned(16))) uint32_t xbuf[DIG ? 3 * kDigPlaneDw : kXPadFloats];
    __shared__ __attribute__((aligned(16))) float xsum[128];
    __shared__ __attribute__((aligned(8))) int xexp[DIG ? 128 : 1];
    float *xs = reinterpret_cast<float *>(xbuf);

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
        if constexpr (DIG) {
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
        } else {
            x_stage<NT>(xs, xsum, xv);
            __syncthreads();
            XWide X;
            x_from_lds(xs, xsum, b, j, X);
#pragma unroll
            for (int m = 0; m < NW; ++m)
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float c = kwide_dot<FMT>(B[m][r], j, X);
                    acc[m][r] += active ? c : 0.0f;
                }
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

// Persistent form of the digit kernel for matrices of many rows and at most
// 4096 columns (one pass): a workgroup per CU stages x's digits once, each
// lane keeps its 48 digit dwords in registers, and every wave walks row
// groups grid-stride with NB register buffers, so the loads of the next
// NB - 1 groups are in flight while a group is reduced (HBM latency under
// load is a microsecond or more, several group reductions).  A group is R
// rows (GATEUP: R gate rows and the same R up rows).  Same outputs as
// k_gemv_kwide<FMT, R, GATEUP, true, EXT, NWV>.
// The walk itself over LDS the caller declares (xbuf: 3 * kDigPlaneDw
// dwords, xsum / xexp: 128 each, ssw: NWV floats).
template <int FMT, int R, bool GATEUP, bool EXT, int NWV, int NB>
__device__ __forceinline__ void kpers_run(const uint8_t *__restrict__ W, const uint8_t *__restrict__ W2,
                                          const float *__restrict__ x, float *y, int outer, int nblk,
                                          const float *__restrict__ nw, float eps, const float *resid,
                                          int epi, uint32_t *xbuf, float *xsum, int *xexp, float *ssw)
{
    using F = KFmt<FMT>;
    constexpr int NM = GATEUP ? 2 : 1;
    constexpr bool NORM = GATEUP && EXT, RESID = !GATEUP && EXT;
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
    kpers_run<FMT, R, GATEUP, EXT, NWV, NB>(W, W2, x, y, outer, nblk, nw, eps, resid, epi, xbuf, xsum,
                                            xexp, ssw);
}

// ------------------------------------------------------------------------
// Staged kernels (Q6_K, Q8_0)
// ------------------------------------------------------------------------
// A segment is 8 Q6_K blocks (2048 columns, 1680 B) or 64 Q8_0 blocks (2048
// columns, 2176 B); rows of a whole number of 8-block groups are 16-byte
// aligned, which the host checks before choosing these kernels.
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
__host__ __device__ constexpr int SFmtSegBlocks(int fmt)
{
    return fmt == kQ6_K ? SFmt<kQ6_K>::SEG_BLOCKS : fmt == kQ8_0 ? SFmt<kQ8_0>::SEG_BLOCKS
         : SFmt<kIQ4_NL>::SEG_BLOCKS;
}
static_assert(SFmt<kQ6_K>::SEG_BYTES % 16 == 0, "Q6_K segment must be 16-byte aligned");
static_assert(SFmt<kQ8_0>::SEG_BYTES % 16 == 0, "Q8_0 segment must be 16-byte aligned");
static_assert(SFmt<kIQ4_NL>::SEG_BYTES % 16 == 0, "IQ4_NL segment must be 16-byte aligned");

// Q6_K lane geometry: block bs = lane>>3; unit u = lane&7: half n = u>>2,
// positions l0 = 8*(u&3) .. +7.  Group g (0..3) of the unit holds the
// elements 128n + 32g + l0 + i (src/Dequant.jl:584-597): g=0 low nibble of
// ql[64n+l0+i], g=1 low nibble of ql[64n+32+l0+i], g=2/3 the high nibbles,
// with qh[32n+l0+i] bits 2g..2g+1 on top and scale sc[8n + 2g + (l0>>4)].
// Q8_0 and IQ4_NL lane geometry: lane = block of the 64-block segment, 32
// weights (IQ4_NL also keeps the sum of its 32 x values).
template <int FMT>
struct SX;
template <>
struct SX<kQ6_K> {
    float x[4][8];
    float s[4];
};
template <>
struct SX<kQ8_0> {
    float x[32];
};
template <>
struct SX<kIQ4_NL> {
    float x[32];
    float s;
};

// All loads first, then the selects and sums, so that the loads are in
// flight together.
template <int FMT>
__device__ __forceinline__ void staged_load_x(const float *__restrict__ xseg, int lane,
                                              int seg_blocks, SX<FMT> &X)
{
    float4 v[8];
    bool active;
    if constexpr (FMT == kQ6_K) {
        const int bs = lane >> 3, n = (lane >> 2) & 1, l0 = 8 * (lane & 3);
        active = bs < seg_blocks;
        const float *base = xseg + (active ? 256 * bs + 128 * n + l0 : 0);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const float4 *p = reinterpret_cast<const float4 *>(base + 32 * g);
            v[2 * g] = p[0];
            v[2 * g + 1] = p[1];
        }
    } else {
        active = lane < seg_blocks;
        const float4 *p = reinterpret_cast<const float4 *>(xseg + (active ? 32 * lane : 0));
#pragma unroll
        for (int t = 0; t < 8; ++t) v[t] = p[t];
    }
#pragma unroll
    for (int t = 0; t < 8; ++t)
        if (!active) v[t] = make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (FMT == kQ6_K) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const float4 a = v[2 * g], b = v[2 * g + 1];
            X.x[g][0] = a.x; X.x[g][1] = a.y; X.x[g][2] = a.z; X.x[g][3] = a.w;
            X.x[g][4] = b.x; X.x[g][5] = b.y; X.x[g][6] = b.z; X.x[g][7] = b.w;
            X.s[g] = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
        }
    } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            X.x[4 * t] = v[t].x; X.x[4 * t + 1] = v[t].y;
            X.x[4 * t + 2] = v[t].z; X.x[4 * t + 3] = v[t].w;
        }
        if constexpr (FMT == kIQ4_NL) {
            float a = 0.0f;
#pragma unroll
            for (int t = 0; t < 8; ++t)
                a += (v[t].x + v[t].y) + (v[t].z + v[t].w);
            X.s = a;
        }
    }
}

// `tile` is the 16-byte-aligned LDS array, `bo` the block's byte offset in it.
__device__ __forceinline__ float q6_dot(const uint8_t *tile, uint32_t bo, int n, int l0,
                                        const SX<kQ6_K> &X)
{
    uint32_t A[2], B[2], H[2], S[2];
    lds_read8_even(tile, bo + 64 * n + l0, A[0], A[1]);
    lds_read8_even(tile, bo + 64 * n + 32 + l0, B[0], B[1]);
    lds_read8_even(tile, bo + 128 + 32 * n + l0, H[0], H[1]);
    lds_read8_even(tile, bo + 192 + 8 * n, S[0], S[1]);
    const float d = h2f(lds_read_u16(tile, bo + 208));
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const uint32_t v[4] = {
            (A[t] & 0x0f0f0f0fu) | ((H[t] & 0x03030303u) << 4),
            (B[t] & 0x0f0f0f0fu) | ((H[t] & 0x0c0c0c0cu) << 2),
            ((A[t] >> 4) & 0x0f0f0f0fu) | (H[t] & 0x30303030u),
            ((B[t] >> 4) & 0x0f0f0f0fu) | ((H[t] >> 2) & 0x30303030u),
        };
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int b = 0; b < 4; ++b)
                acc[g] = fmaf(ubyte_f(v[g], b), X.x[g][4 * t + b], acc[g]);
    }
    const int c = l0 >> 4;
    float r = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int si = 2 * g + c; // byte of the 8 scales sc[8n..8n+7]
        const float ds = d * sbyte_f(S[si >> 2], si & 3);
        r = fmaf(ds, fmaf(-32.0f, X.s[g], acc[g]), r);
    }
    return r;
}

// Q8_0 block at byte `off` of the 16-byte-aligned LDS row `row_lds`.
__device__ __forceinline__ float q80_dot(const uint8_t *row_lds, uint32_t off, const float *xr)
{
    const float d = h2f(lds_read_u16(row_lds, off));
    const uint32_t o = off + 2;
    const uint32_t *p = reinterpret_cast<const uint32_t *>(row_lds + (o & ~3u));
    const uint32_t sh = o & 3u;
    uint32_t w[9];
#pragma unroll
    for (int i = 0; i < 9; ++i) w[i] = p[i];
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const uint32_t q = __builtin_amdgcn_alignbyte(w[t + 1], w[t], sh);
        a0 = fmaf(sbyte_f(q, 0), xr[4 * t + 0], a0);
        a1 = fmaf(sbyte_f(q, 1), xr[4 * t + 1], a1);
        a0 = fmaf(sbyte_f(q, 2), xr[4 * t + 2], a0);
        a1 = fmaf(sbyte_f(q, 3), xr[4 * t + 3], a1);
    }
    return d * (a0 + a1);
}

// IQ4_NL block at byte `off` of the 16-byte-aligned LDS row `row_lds`
// (src/Dequant.jl:683-693: element j = low nibble of qs[j], element j + 16 =
// high nibble; weight = d * grid[nibble], grid src/QuantsData.jl:384).  The
// grid, biased by +128 to unsigned bytes, is looked up four nibbles at a time
// with byte permutes (grid[0..7] and grid[8..15], then a choice by the
// nibble's bit 3); the bias comes back off through the lane's x sum.
constexpr uint32_t kIQ4G0 = 0x3F2D1801u; // grid + 128: 1, 24, 45, 63
constexpr uint32_t kIQ4G1 = 0x766A5D4Fu; // 79, 93, 106, 118
constexpr uint32_t kIQ4G2 = 0xA6998D81u; // 129, 141, 153, 166
constexpr uint32_t kIQ4G3 = 0xF1D9C5B5u; // 181, 197, 217, 241

__device__ __forceinline__ uint32_t iq4nl_lookup(uint32_t nib) // four nibbles in bytes
{
    const uint32_t n7 = nib & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(kIQ4G1, kIQ4G0, n7); // bytes 0-3 of G0, 4-7 of G1
    const uint32_t hi = __builtin_amdgcn_perm(kIQ4G3, kIQ4G2, n7);
    const uint32_t pick = 0x03020100u + ((nib & 0x08080808u) >> 1); // byte i of lo or of hi
    return __builtin_amdgcn_perm(hi, lo, pick);
}

__device__ __forceinline__ float iq4nl_dot(const uint8_t *row_lds, uint32_t off,
                                           const SX<kIQ4_NL> &X)
{
    const float d = h2f(lds_read_u16(row_lds, off));
    const uint32_t o = off + 2;
    const uint32_t *p = reinterpret_cast<const uint32_t *>(row_lds + (o & ~3u));
    const uint32_t sh = o & 3u;
    uint32_t w[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) w[i] = p[i];
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const uint32_t q = __builtin_amdgcn_alignbyte(w[t + 1], w[t], sh); // qs[4t..4t+3]
        const uint32_t vl = opaque(iq4nl_lookup(q & 0x0f0f0f0fu));         // elements 4t + b
        const uint32_t vh = opaque(iq4nl_lookup((q >> 4) & 0x0f0f0f0fu));  // elements 16 + 4t + b
        a0 = fmaf(ubyte_f(vl, 0), X.x[4 * t + 0], a0);
        a1 = fmaf(ubyte_f(vl, 1), X.x[4 * t + 1], a1);
        a0 = fmaf(ubyte_f(vl, 2), X.x[4 * t + 2], a0);
        a1 = fmaf(ubyte_f(vl, 3), X.x[4 * t + 3], a1);
        a0 = fmaf(ubyte_f(vh, 0), X.x[16 + 4 * t + 0], a0);
        a1 = fmaf(ubyte_f(vh, 1), X.x[16 + 4 * t + 1], a1);
        a0 = fmaf(ubyte_f(vh, 2), X.x[16 + 4 * t + 2], a0);
        a1 = fmaf(ubyte_f(vh, 3), X.x[16 + 4 * t + 3], a1);
    }
    return d * fmaf(-128.0f, X.s, a0 + a1);
}

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

// Reduce `nparts` partials with NT threads, U 16-byte partials in flight per
// thread; writes the 0-based token and the IHIP_FLAG_* bits.  With NT = 64
// there is no LDS exchange and no barrier; NT = 256 (four partials per thread
// for the lm_head's ~1000) is the default.
template <int NT>
__global__ __launch_bounds__(NT) void k_argmax_finalize(const ArgPart *__restrict__ parts,
                                                        int nparts, int32_t *token,
                                                        uint32_t *flags_out)
{
    constexpr int NWV = NT / 64, U = NT >= 1024 ? 4 : 16;
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
    if constexpr (NWV > 1) {
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

// ---- the streamed staged GEMV --------------------------------------------
// Workgroup = NW waves; wave w owns K segments w, w + NW, ... so the x slice
// of its segment stays in registers while it streams the workgroup's rows
// through a D-slot LDS ring filled by direct-to-LDS 128-bit loads: the copy
// of row i + D is issued as soon as row i has been reduced, so D rows per
// wave are always in flight.  Per-row partial sums meet in LDS and the
// workgroup's threads finish the rows (and, ARGMAX, fold them into one
// partial per workgroup).  Workgroups walk chunks of `rpc` rows grid-stride.

constexpr int kStreamMaxRows = 64; // rows per chunk (one partial slot per row and wave)
static_assert(kStreamMaxRows <= 64, "the epilogue gives every row its own thread");

template <int FMT, int NW, int D, bool ARGMAX>
__global__ __launch_bounds__(NW * 64) void k_gemv_stream(const uint8_t *__restrict__ W,
                                                         const float *__restrict__ x,
                                                         float *y, int outer,
                                                         int nblk, int rpc,
                                                         ArgPart *__restrict__ parts,
                                                         const float *resid, int epi)
{
    using F = SFmt<FMT>;
    constexpr int SLOT = F::SEG_BYTES + 16; // Q8_0 reads one dword past a segment
    __shared__ __attribute__((aligned(16))) uint8_t ring[NW * D * SLOT];
    __shared__ float part[kStreamMaxRows][NW];
    __shared__ unsigned long long wkey[NW];
    __shared__ uint32_t wflag[NW];

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6); // wave-uniform (scalar)
    const int bb = block_bytes(FMT);
    const size_t row_bytes = (size_t)nblk * bb;
    const int nseg = (nblk + F::SEG_BLOCKS - 1) / F::SEG_BLOCKS;
    const int nchunks = (outer + rpc - 1) / rpc;
    const uint32_t my_ring = (uint32_t)(w * D * SLOT);

    unsigned long long key = 0;
    uint32_t fl = 0;
    SX<FMT> X;
    int x_seg = -1; // segment whose x slice X holds

    for (int chunk = blockIdx.x; chunk < nchunks; chunk += gridDim.x) {
        const int row0 = chunk * rpc;
        const int nrows = min(rpc, outer - row0);
        // the residual of this thread's row (the epilogue below has one row
        // per thread) is loaded now, under the weight stream; the segment
        // loop's first s_waitcnt(0) completes it before the copy waits start
        const float rv = (resid && tid < nrows) ? resid[row0 + tid] : 0.0f;
        for (int i = tid; i < kStreamMaxRows * NW; i += NW * 64)
            (&part[0][0])[i] = 0.0f;
        __syncthreads();
        for (int sg = w; sg < nseg; sg += NW) { // wave-uniform
            const int seg_blocks = min(F::SEG_BLOCKS, nblk - sg * F::SEG_BLOCKS);
            // whole 8-block groups (checked on the host): a multiple of 16 bytes
            const int chunks16 = seg_blocks * bb / 16;
            const int ipr = (chunks16 + 63) >> 6; // copy instructions per row
            const uint8_t *src0 = W + (size_t)row0 * row_bytes + (size_t)sg * F::SEG_BYTES;
            auto issue = [&](int i) {
                const uint8_t *src = src0 + (size_t)i * row_bytes;
                uint8_t *dst = ring + my_ring + (i % D) * SLOT;
                for (int c0 = 0; c0 < chunks16; c0 += 64) {
                    const int c = c0 + lane;
                    if (c < chunks16)
                        __builtin_amdgcn_global_load_lds(
                            (const void *)(src + 16 * (size_t)c),
                            (__attribute__((address_space(3))) void *)(dst + 16 * c0), 16, 0, 0);
                }
            };
            const int pre = min(D, nrows);
            for (int i = 0; i < pre; ++i)
                issue(i);
            if (x_seg != sg) {
                staged_load_x<FMT>(x + (size_t)sg * 2048, lane, seg_blocks, X);
                x_seg = sg;
            }
            // x (and the prologue rows) complete here, so that inside the row loop
            // only ring copies are outstanding and the explicit waits below are
            // the only ones
            __builtin_amdgcn_s_waitcnt(0);
            for (int i = 0; i < nrows; ++i) {
                wait_vmcnt(ipr * min(D - 1, nrows - 1 - i)); // row i has landed
                const uint32_t slot = my_ring + (uint32_t)((i % D) * SLOT);
                float v = 0.0f;
                if constexpr (FMT == kQ6_K) {
                    const int bs = lane >> 3, n = (lane >> 2) & 1, l0 = 8 * (lane & 3);
                    if (bs < seg_blocks)
                        v = q6_dot(ring, slot + (uint32_t)(210 * bs), n, l0, X);
                } else if constexpr (FMT == kIQ4_NL) {
                    if (lane < seg_blocks)
                        v = iq4nl_dot(ring + slot, 18u * lane, X);
                } else {
                    if (lane < seg_blocks)
                        v = q80_dot(ring + slot, 34u * lane, X.x);
                }
                v = wave_sum(v);
                if (lane == 0)
                    part[i][w] += v;
                if (i + D < nrows)
                    issue(i + D); // slot i % D has been read
            }
        }
        __syncthreads();
        for (int i = tid; i < nrows; i += NW * 64) {
            float v = 0.0f;
#pragma unroll
            for (int k = 0; k < NW; ++k)
                v += part[i][k];
            if (y)
                y[row0 + i] = resid ? epi_apply(rv, v, epi) : v; // i == tid; resid may be y
            if constexpr (ARGMAX)
                argmax_fold(v, (uint32_t)(row0 + i), key, fl);
        }
        __syncthreads(); // part is cleared for the next chunk
    }
    if constexpr (ARGMAX) {
        argmax_wave_reduce(key, fl);
        if (lane == 0) {
            wkey[w] = key;
            wflag[w] = fl;
        }
        __syncthreads();
        if (tid == 0) {
            unsigned long long k = wkey[0];
            uint32_t f = wflag[0];
#pragma unroll
            for (int i = 1; i < NW; ++i) {
                k = wkey[i] > k ? wkey[i] : k;
                f |= wflag[i];
            }
            parts[blockIdx.x].key = k;
            parts[blockIdx.x].flags = f;
            parts[blockIdx.x].pad = 0;
        }
    }
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
    const float d = h2f(*reinterpret_cast<const uint16_t *>(slot + L.d));
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
    const int c = L.c;
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

// Q8_0 block at byte `off` of an LDS row.
__device__ __forceinline__ float q80_dot_dig(const uint8_t *row_lds, uint32_t off, const SXD &X)
{
    const float d = h2f(lds_read_u16(row_lds, off));
    const uint32_t o = off + 2;
    const uint32_t *p = reinterpret_cast<const uint32_t *>(row_lds + (o & ~3u));
    const uint32_t sh = o & 3u;
    constexpr int NDW = sdig_blk_dwords(kQ8_0);
    uint32_t w[NDW];
#pragma unroll
    for (int i = 0; i < NDW; ++i) w[i] = p[i];
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

// IQ4_NL block at byte `off` of an LDS row (element j = low nibble of qs[j],
// element j + 16 = high nibble).
__device__ __forceinline__ float iq4nl_dot_dig(const uint8_t *row_lds, uint32_t off, const SXD &X)
{
    const float d = h2f(lds_read_u16(row_lds, off));
    const uint32_t o = off + 2;
    const uint32_t *p = reinterpret_cast<const uint32_t *>(row_lds + (o & ~3u));
    const uint32_t sh = o & 3u;
    constexpr int NDW = sdig_blk_dwords(kIQ4_NL);
    uint32_t w[NDW];
#pragma unroll
    for (int i = 0; i < NDW; ++i) w[i] = p[i];
    uint32_t a0 = (uint32_t)X.init[0][0], a1 = (uint32_t)X.init[1][0];
    int a2 = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const uint32_t q = __builtin_amdgcn_alignbyte(w[t + 1], w[t], sh); // qs[4t..4t+3]
        const uint32_t ul = iq4nl_lookup(q & 0x0f0f0f0fu);          // grid + 128, elements 4t + b
        const uint32_t uh = iq4nl_lookup((q >> 4) & 0x0f0f0f0fu);   // elements 16 + 4t + b
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
// segments unless ARGMAX; part: kSdigMaxRows x 8; wkey / wflag: NW each).
template <int FMT, int NW, int D, bool ARGMAX, bool RESID>
__device__ __forceinline__ void sdig_run(const uint8_t *__restrict__ W, const float *x, float *y,
                                         int outer, int nblk, int rpc, ArgPart *__restrict__ parts,
                                         const float *resid, int epi, uint8_t *ring,
                                         uint32_t (*digs)[kDigQuads][64][4], float (*part)[8],
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
    // segments whose digits can be staged in LDS (none for the lm_head: its 32 KB
    // workgroups run four to a CU, which the staging area would halve)
    constexpr int SHC = ARGMAX ? 0 : sdig_share_cap(NW);

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int bid = (int)blockIdx.x, grid = (int)gridDim.x;
    const SdigWave g = sdig_wave(FMT, NW, D, SHC, outer, nblk, rpc, bid, grid, w);
    const int nseg = g.nseg, sg = g.sg;
    const bool share = g.share, producer = g.producer;
    const int seg_blocks = g.seg_blocks, nitems = g.nitems;

    // item k's row segment into slot k % D
    const uint32_t ring_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)ring;
    auto issue = [&](int k) {
        const uint8_t *src = W + sdig_copy_row(g, FMT, k, bid, grid, rpc, outer);
#pragma unroll
        for (int i = 0; i < IPR; ++i)
            lds_copy16(src + sdig_copy_lane(g, i, lane), ring_lds + sdig_copy_dst(g, FMT, D, k, i));
    };

    // x first, then the first D rows' copies, all in flight together; the
    // digits wait only for x (vmcnt counts completions in issue order).
    float4 xv[8];
    bool xact = false;
    if (producer) // wave-uniform
        xact = staged_dig_issue<FMT>(x + (size_t)sg * 2048, lane, seg_blocks, xv);
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
    unsigned long long key = 0;
    uint32_t fl = 0;
    int k = 0;
    for (int ci = 0; ci < g.my_chunks; ++ci) {
        const SdigChunk c = sdig_chunk(g, ci, bid, grid, rpc, outer);
        const int row0 = c.row0, nrows = c.nrows, mine = c.mine;
        // the lane's share of the dot product of the row in ring slot `slot`
        auto dot_at = [&](uint32_t slot) {
            float v = 0.0f;
            if constexpr (FMT == kQ6_K) {
                if ((lane >> 3) < seg_blocks)
                    v = q6_dot_dig(ring + slot, q6l, X);
            } else if constexpr (FMT == kIQ4_NL) {
                if (lane < seg_blocks)
                    v = iq4nl_dot_dig(ring + slot, sdig_blk_off(FMT, lane), X);
            } else {
                if (lane < seg_blocks)
                    v = q80_dot_dig(ring + slot, sdig_blk_off(FMT, lane), X);
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
                    argmax_fold(v, (uint32_t)row, key, fl); // every lane folds the same row
            } else if (lane == 0) {
                part[sdig_chunk_row(g, rr)][sg] = v;
            }
        };
        for (int rr = 0; rr < mine; ++rr, ++k) {
            wait_vmcnt(IPR * sdig_wait_items(g, D, k));
            finish(rr, wave_sum(dot_at(sdig_copy_dst(g, FMT, D, k, 0))));
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

template <int FMT, int NW, int D, bool ARGMAX, bool RESID>
__global__ __launch_bounds__(NW * 64) void k_gemv_sdig(const uint8_t *__restrict__ W,
                                                       const float *x, float *y, int outer, int nblk,
                                                       int rpc, ArgPart *__restrict__ parts,
                                                       const float *resid, int epi)
{
    constexpr int SHC = ARGMAX ? 0 : sdig_share_cap(NW);
    __shared__ __attribute__((aligned(16))) uint8_t ring[NW * D * sdig_slot(FMT)];
    __shared__ __attribute__((aligned(16))) uint32_t digs[SHC > 0 ? SHC : 1][kDigQuads][64][4];
    __shared__ float part[kSdigMaxRows][8];
    __shared__ unsigned long long wkey[NW];
    __shared__ uint32_t wflag[NW];
    sdig_run<FMT, NW, D, ARGMAX, RESID>(W, x, y, outer, nblk, rpc, parts, resid, epi, ring, digs, part,
                                        wkey, wflag);
}

// ------------------------------------------------------------------------
// launchers
// ------------------------------------------------------------------------
// Rows per wave of the wide kernels and rows per chunk of the streamed
// kernels; 0 = the measured default.
static int g_rows_wide = 0;   // Q4_K/Q5_K GEMV (default 2)
static int g_rows_gateup = 0; // fused gate/up (default 1)
static int g_stream_rows = 0; // Q6_K/Q8_0 rows per chunk (default: see stream_rows())
static int g_wide_fp32 = 0;   // Q4_K/Q5_K: 1 = fp32 activations instead of integer digits
static int g_wide_waves = 0;  // Q4_K/Q5_K waves per workgroup (4 or 8; default 8)
static int g_wide_persist = 0; // Q4_K/Q5_K persistent kernel: 1 = always, -1 = never, 0 = by size
static int g_pers_wg_per_cu = 1; // workgroups per CU of the persistent kernel
static int g_pers_bufs = 0;      // register buffers per wave of the persistent kernel (2..4)
static int g_stream_wg_per_cu = 0; // streamed kernel: cap on workgroups per CU (0 = one per chunk)
// persistent digit streamed kernel: rows per chunk, ring depth (0 = default), 1 = not used
static int g_sdig_rows = 0, g_sdig_depth = 0, g_sdig_off = 0, g_sdig_wg_per_cu = 0, g_sdig_waves = 0;
static int g_argmax_threads = 0; // argmax finalize: 64, 256 or 1024 threads (0 = 256)

void set_tuning(const char *name, int value)
{
    if (!__builtin_strcmp(name, "rows_wide")) g_rows_wide = value;
    if (!__builtin_strcmp(name, "rows_gateup")) g_rows_gateup = value;
    if (!__builtin_strcmp(name, "stream_rows")) g_stream_rows = value;
    if (!__builtin_strcmp(name, "wide_fp32")) g_wide_fp32 = value;
    if (!__builtin_strcmp(name, "wide_waves")) g_wide_waves = value;
    if (!__builtin_strcmp(name, "wide_persist")) g_wide_persist = value;
    if (!__builtin_strcmp(name, "pers_wg_per_cu")) g_pers_wg_per_cu = value > 0 ? value : 1;
    if (!__builtin_strcmp(name, "pers_bufs")) g_pers_bufs = value;
    if (!__builtin_strcmp(name, "stream_wg_per_cu")) g_stream_wg_per_cu = value;
    if (!__builtin_strcmp(name, "sdig_rows")) g_sdig_rows = value;
    if (!__builtin_strcmp(name, "sdig_depth")) g_sdig_depth = value;
    if (!__builtin_strcmp(name, "sdig_off")) g_sdig_off = value;
    if (!__builtin_strcmp(name, "sdig_wg_per_cu")) g_sdig_wg_per_cu = value;
    if (!__builtin_strcmp(name, "sdig_waves")) g_sdig_waves = value;
    if (!__builtin_strcmp(name, "argmax_threads")) g_argmax_threads = value;
}

template <int FMT, bool GATEUP>
static hipError_t launch_kwide(const void *w, const void *w2, const float *x, float *y,
                               int inner, int outer, hipStream_t s, const float *nw = nullptr,
                               float eps = 0.0f, const float *resid = nullptr, int epi = kEpiAdd)
{
    const int nblk = inner / 256;
    int R = GATEUP ? g_rows_gateup : g_rows_wide;
    if (R <= 0) // measured on MI355X: 4096 x 4096 GEMV and 2 x 12288 x 4096 gate/up
        R = GATEUP ? 1 : 2;
    if (FMT == kQ5_K && GATEUP && R > 2)
        R = 2; // register budget
    const bool dig = g_wide_fp32 <= 0;
    const bool ext = GATEUP ? nw != nullptr : resid != nullptr;
    const int nwv = g_wide_waves == 4 ? 4 : 8;
#define IHIP_KW(RR, DG, EX, NV)                                                              \
    hipLaunchKernelGGL((k_gemv_kwide<FMT, RR, GATEUP, DG, EX, NV>),                          \
                       dim3((outer + NV * RR - 1) / (NV * RR)), dim3(NV * 64), 0, s,          \
                       (const uint8_t *)w, (const uint8_t *)w2, x, y, outer, nblk, nw, eps, resid, epi)
#define IHIP_KW_R(DG, EX)                                                                    \
    do {                                                                                     \
        if (nwv == 8) {                                                                      \
            if (R == 1) IHIP_KW(1, DG, EX, 8); else if (R == 4) IHIP_KW(4, DG, EX, 8); else IHIP_KW(2, DG, EX, 8); \
        } else {                                                                             \
            if (R == 1) IHIP_KW(1, DG, EX, 4); else if (R == 4) IHIP_KW(4, DG, EX, 4); else IHIP_KW(2, DG, EX, 4); \
        }                                                                                    \
    } while (0)
    // the persistent kernel once every wave has at least four rows (measured on
    // MI355X: 2 x 12288 x 4096 gate/up 12.7 us against 13.9 us; at 4096 x 4096
    // one row group per wave is all there is and the plain kernel is faster)
    const bool pers = dig && nblk <= 16 && (g_wide_persist > 0 || (g_wide_persist == 0 && outer >= 4 * nwv * 256));
    if (pers) {
        int dev = 0, ncu = 256;
        if (hipGetDevice(&dev) == hipSuccess)
            hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
        const int nbuf = g_pers_bufs >= 2 && g_pers_bufs <= 4 ? g_pers_bufs : 2;
        const int grid = max(1, min(ncu * g_pers_wg_per_cu, (outer + nwv - 1) / nwv));
#define IHIP_KP(RR, EX, NV, NBB)                                                             \
    hipLaunchKernelGGL((k_gemv_kpers<FMT, RR, GATEUP, EX, NV, NBB>), dim3(grid), dim3(NV * 64), 0, s, \
                       (const uint8_t *)w, (const uint8_t *)w2, x, y, outer, nblk, nw, eps, resid, epi)
#define IHIP_KP_R(EX)                                                                        \
    do {                                                                                     \
        if (nwv == 8) {                                                                      \
            if (nbuf == 2) IHIP_KP(1, EX, 8, 2); else if (nbuf == 3) IHIP_KP(1, EX, 8, 3); else IHIP_KP(1, EX, 8, 4); \
        } else {                                                                             \
            if (nbuf == 2) IHIP_KP(1, EX, 4, 2); else if (nbuf == 3) IHIP_KP(1, EX, 4, 3); else IHIP_KP(1, EX, 4, 4); \
        }                                                                                    \
    } while (0)
        if (ext) IHIP_KP_R(true); else IHIP_KP_R(false);
#undef IHIP_KP_R
#undef IHIP_KP
    } else if (dig) {
        if (ext) IHIP_KW_R(true, true); else IHIP_KW_R(true, false);
    } else {
        if (ext) IHIP_KW_R(false, true); else IHIP_KW_R(false, false);
    }
#undef IHIP_KW_R
#undef IHIP_KW
    return hipGetLastError();
}

// Waves per workgroup of the streamed kernel: one per K segment, at most 8.
static int stream_waves(int nseg) { return nseg >= 8 ? 8 : nseg >= 6 ? 6 : nseg >= 4 ? 4 : nseg; }

// Rows per chunk: outer / 1024 within 4..16 (at least four workgroups per
// CU; measured on MI355X at 4096 x 4096 Q8_0, 4096 x 12288 Q6_K and
// 151936 x 2048 Q6_K).  With the fused argmax every chunk leaves one partial,
// so the chunk count is kept within kArgMaxParts.
static int stream_rows(int outer, bool argmax)
{
    int r;
    if (g_stream_rows > 0) {
        r = min(g_stream_rows, kStreamMaxRows);
    } else {
        r = outer / 1024;
        r = r < 4 ? 4 : r > 16 ? 16 : r;
    }
    if (argmax)
        r = max(r, (outer + kArgMaxParts - 1) / kArgMaxParts);
    return r;
}

// One workgroup per chunk, or at most g_stream_wg_per_cu workgroups per CU that
// walk the chunks grid-stride (each keeps its x slice across its chunks).
static int stream_grid(int outer, int rpc)
{
    const int nchunks = (outer + rpc - 1) / rpc;
    if (g_stream_wg_per_cu <= 0)
        return nchunks;
    int dev = 0, ncu = 256;
    if (hipGetDevice(&dev) == hipSuccess)
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
    return max(1, min(nchunks, g_stream_wg_per_cu * ncu));
}

static SdigKnobs sdig_knobs()
{
    SdigKnobs k;
    k.rows = g_sdig_rows;
    k.depth = g_sdig_depth;
    k.wg_per_cu = g_sdig_wg_per_cu;
    k.waves = g_sdig_waves;
    return k;
}

static int device_cus()
{
    int dev = 0, ncu = 256;
    if (hipGetDevice(&dev) == hipSuccess)
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
    return ncu;
}

static bool sdig_usable(int fmt, int nblk) { return g_sdig_off <= 0 && sdig_rows_ok(fmt, nblk); }

template <int FMT, bool ARGMAX, int NWV, int DD>
static void launch_sdig_nd(const void *w, const float *x, float *y, int nblk, int outer,
                           const SdigPlan &p, void *parts, hipStream_t s, const float *resid, int epi)
{
    if (resid)
        hipLaunchKernelGGL((k_gemv_sdig<FMT, NWV, DD, ARGMAX, true>), dim3(p.grid), dim3(NWV * 64), 0,
                           s, (const uint8_t *)w, x, y, outer, nblk, p.rpc, (ArgPart *)parts, resid, epi);
    else
        hipLaunchKernelGGL((k_gemv_sdig<FMT, NWV, DD, ARGMAX, false>), dim3(p.grid), dim3(NWV * 64), 0,
                           s, (const uint8_t *)w, x, y, outer, nblk, p.rpc, (ArgPart *)parts, resid, epi);
}

// The instantiation sdig_plan chose (ring depths that do not fit the LDS are
// never instantiated; the plan never picks them).
template <int FMT, bool ARGMAX>
static hipError_t launch_sdig(const void *w, const float *x, float *y, int inner, int outer,
                              void *parts, hipStream_t s, const float *resid, int epi)
{
    const int nblk = inner / block_elems(FMT);
    const SdigPlan p = sdig_plan(FMT, nblk, outer, ARGMAX, sdig_knobs(), device_cus());
    switch (p.nw * 16 + p.d) {
    case 12 * 16 + 6:
        if constexpr (sdig_fits(FMT, 12, 6))
            launch_sdig_nd<FMT, ARGMAX, 12, 6>(w, x, y, nblk, outer, p, parts, s, resid, epi);
        break;
    case 12 * 16 + 4:
        if constexpr (sdig_fits(FMT, 12, 4))
            launch_sdig_nd<FMT, ARGMAX, 12, 4>(w, x, y, nblk, outer, p, parts, s, resid, epi);
        break;
    case 12 * 16 + 2: launch_sdig_nd<FMT, ARGMAX, 12, 2>(w, x, y, nblk, outer, p, parts, s, resid, epi); break;
    case 16 * 16 + 2: launch_sdig_nd<FMT, ARGMAX, 16, 2>(w, x, y, nblk, outer, p, parts, s, resid, epi); break;
    case 6 * 16 + 2: launch_sdig_nd<FMT, ARGMAX, 6, 2>(w, x, y, nblk, outer, p, parts, s, resid, epi); break;
    case 6 * 16 + 4: launch_sdig_nd<FMT, ARGMAX, 6, 4>(w, x, y, nblk, outer, p, parts, s, resid, epi); break;
    case 8 * 16 + 2: launch_sdig_nd<FMT, ARGMAX, 8, 2>(w, x, y, nblk, outer, p, parts, s, resid, epi); break;
    case 8 * 16 + 4: launch_sdig_nd<FMT, ARGMAX, 8, 4>(w, x, y, nblk, outer, p, parts, s, resid, epi); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int FMT, bool ARGMAX>
static hipError_t launch_stream(const void *w, const float *x, float *y, int inner, int outer,
                                void *parts, hipStream_t s, const float *resid = nullptr,
                                int epi = kEpiAdd)
{
    if (sdig_usable(FMT, inner / block_elems(FMT)))
        return launch_sdig<FMT, ARGMAX>(w, x, y, inner, outer, parts, s, resid, epi);
    const int nblk = inner / block_elems(FMT);
    const int nseg = (nblk + SFmt<FMT>::SEG_BLOCKS - 1) / SFmt<FMT>::SEG_BLOCKS;
    const int nw = stream_waves(nseg);
    const int rpc = stream_rows(outer, ARGMAX);
    const int grid = stream_grid(outer, rpc);
#define IHIP_ST(NWV, DD)                                                                         if (nw == NWV) {                                                                                 hipLaunchKernelGGL((k_gemv_stream<FMT, NWV, DD, ARGMAX>), dim3(grid), dim3(NWV * 64),                            0, s, (const uint8_t *)w, x, y, outer, nblk, rpc, (ArgPart *)parts, resid, epi);         return hipGetLastError();                                                                }
    IHIP_ST(1, 2) IHIP_ST(2, 2) IHIP_ST(3, 2) IHIP_ST(4, 2) IHIP_ST(6, 2) IHIP_ST(8, 2)
#undef IHIP_ST
    return hipErrorInvalidValue;
}

hipError_t launch_gemv(int type, const void *w, const float *x, float *y, int inner, int outer,
                       hipStream_t s, const float *resid, int epi)
{
    switch (type) {
    case kQ4_K: return launch_kwide<kQ4_K, false>(w, nullptr, x, y, inner, outer, s, nullptr, 0.0f, resid, epi);
    case kQ5_K: return launch_kwide<kQ5_K, false>(w, nullptr, x, y, inner, outer, s, nullptr, 0.0f, resid, epi);
    case kQ6_K: return launch_stream<kQ6_K, false>(w, x, y, inner, outer, nullptr, s, resid, epi);
    case kQ8_0: return launch_stream<kQ8_0, false>(w, x, y, inner, outer, nullptr, s, resid, epi);
    case kIQ4_NL: return launch_stream<kIQ4_NL, false>(w, x, y, inner, outer, nullptr, s, resid, epi);
    default: return hipErrorInvalidValue;
    }
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

bool lm_head_fusable(int vocab) { return stream_rows(vocab, true) <= kStreamMaxRows; }

static void launch_argmax_finalize(const void *ws, int nparts, int32_t *token, uint32_t *flags,
                                   hipStream_t s)
{
    // 256 measured fastest for the lm_head's 1024 partials (against 1024 threads:
    // -0.9 us per call; a single wave gains nothing)
    int nt = g_argmax_threads;
    if (nt != 64 && nt != 256 && nt != 1024)
        nt = 256;
    const ArgPart *parts = (const ArgPart *)ws;
    switch (nt) {
    case 64:
        hipLaunchKernelGGL(k_argmax_finalize<64>, dim3(1), dim3(64), 0, s, parts, nparts, token, flags);
        break;
    case 256:
        hipLaunchKernelGGL(k_argmax_finalize<256>, dim3(1), dim3(256), 0, s, parts, nparts, token, flags);
        break;
    default:
        hipLaunchKernelGGL(k_argmax_finalize<1024>, dim3(1), dim3(1024), 0, s, parts, nparts, token, flags);
    }
}

int lm_head_argmax_parts(int type, int hidden, int vocab, bool fused)
{
    if (!fused) // the GEMV, then the standalone argmax over the logits
        return (int)std::min<int64_t>(std::max<int64_t>(1, ((int64_t)vocab + 255) / 256), kArgMaxParts);
    const int nblk = hidden / block_elems(type);
    return sdig_usable(type, nblk) ? sdig_plan(type, nblk, vocab, true, sdig_knobs(), device_cus()).grid
                                   : stream_grid(vocab, stream_rows(vocab, true));
}

hipError_t launch_lm_head_argmax(int type, const void *w, const float *x, float *logits,
                                 int32_t *token, uint32_t *flags, int hidden, int vocab,
                                 void *ws, hipStream_t s)
{
    if (!lm_head_fusable(vocab))
        return hipErrorInvalidValue;
    hipError_t e;
    switch (type) {
    case kQ6_K: e = launch_stream<kQ6_K, true>(w, x, logits, hidden, vocab, ws, s); break;
    case kQ8_0: e = launch_stream<kQ8_0, true>(w, x, logits, hidden, vocab, ws, s); break;
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
