// kq_common.h -- shared definitions for the gfx950 K-quant kernels.
//
// Block layouts (src/kernels/quant_kernels.c:24-62, src/Dequant.jl:311-316,
// 336-341, 392-400, 570-574 of Inferno.jl), little-endian:
//   Q4_K 144 B: d f16 @0, dmin f16 @2, scales[12] @4, qs[128] @16
//   Q5_K 176 B: d @0, dmin @2, scales[12] @4, qh[32] @16, qs[128] @48
//   Q6_K 210 B: ql[128] @0, qh[64] @128, scales int8[16] @192, d f16 @208
//   Q8_0  34 B: d f16 @0, qs int8[32] @2
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ihip {

constexpr int kQ8_0 = 8, kQ4_K = 12, kQ5_K = 13, kQ6_K = 14, kIQ4_NL = 20;

constexpr int kBytesQ4K = 144, kBytesQ5K = 176, kBytesQ6K = 210, kBytesQ80 = 34;

__host__ __device__ constexpr int block_bytes(int t)
{
    return t == kQ4_K ? 144 : t == kQ5_K ? 176 : t == kQ6_K ? 210 : t == kQ8_0 ? 34
         : t == kIQ4_NL ? 18 : 0;
}
__host__ __device__ constexpr int block_elems(int t)
{
    return (t == kQ4_K || t == kQ5_K || t == kQ6_K) ? 256 : (t == kQ8_0 || t == kIQ4_NL) ? 32 : 0;
}

// fp16 bits -> fp32.  v_cvt_f32_f16 widens exactly, fp16 subnormals
// included (the kernels run with fp16/fp64 denormals enabled, the HIP
// default; the exhaustive dequant test checks all 65536 patterns).
__device__ __forceinline__ float h2f(uint32_t bits16)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// The 6-bit scale (sc) and min (m) of sub-block i of a Q4_K/Q5_K block,
// from the 12 packed bytes held as three dwords s0 (bytes 0-3), s1 (4-7)
// and s2 (8-11): src/Dequant.jl:345-362.
//   i < 4:  sc = s[i] & 63,                        m = s[i+4] & 63
//   i >= 4: sc = (s[i+4] & 15) | (s[i-4] >> 6) << 4, m = (s[i+4] >> 4) | (s[i] >> 6) << 4
// Branch-free: `i` may differ between lanes.
__device__ __forceinline__ void k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int i,
                                            uint32_t &sc, uint32_t &m)
{
    const uint32_t k = 8u * (uint32_t)(i & 3);
    const uint32_t sc_lo = __builtin_amdgcn_ubfe(s0, k, 6), m_lo = __builtin_amdgcn_ubfe(s1, k, 6);
    const uint32_t sc_hi = __builtin_amdgcn_ubfe(s2, k, 4) | (__builtin_amdgcn_ubfe(s0, k + 6, 2) << 4);
    const uint32_t m_hi = __builtin_amdgcn_ubfe(s2, k + 4, 4) | (__builtin_amdgcn_ubfe(s1, k + 6, 2) << 4);
    sc = i < 4 ? sc_lo : sc_hi;
    m = i < 4 ? m_lo : m_hi;
}

// v + (v moved across lanes by a DPP pattern); lanes outside row_mask add 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v)
{
    const int moved = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false);
    return v + __int_as_float(moved);
}

// Sum over the 64 lanes of a wavefront; every lane gets the total.  DPP lane
// moves (no LDS traffic): pairs, quads, half-rows and rows of 16 by
// quad_perm / row_half_mirror / row_mirror, then row_bcast:15 and
// row_bcast:31 carry the row sums up to lane 63, whose value is broadcast.
__device__ __forceinline__ float wave_sum(float v)
{
    v = dpp_add<0xb1, 0xf>(v);  // quad_perm [1,0,3,2]
    v = dpp_add<0x4e, 0xf>(v);  // quad_perm [2,3,0,1]
    v = dpp_add<0x141, 0xf>(v); // row_half_mirror
    v = dpp_add<0x140, 0xf>(v); // row_mirror
    v = dpp_add<0x142, 0xa>(v); // row_bcast:15 into rows 1 and 3
    v = dpp_add<0x143, 0xc>(v); // row_bcast:31 into rows 2 and 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Unsigned maximum of a value and its DPP-moved copy (lanes the move does
// not write contribute 0): the x staging chains these over a sub-block's
// lanes for its largest magnitude.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_max_u32(uint32_t v)
{
    const uint32_t moved = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xf, false);
    return v > moved ? v : moved;
}

// fmaxf over the 64 lanes of a wavefront for values >= 0 (or NaN, which
// fmaxf skips in any order), by the wave_sum pattern: lanes a DPP move does
// not write see 0.  Every lane gets the maximum.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_fmax(float v)
{
    const int moved = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false);
    return fmaxf(v, __int_as_float(moved));
}
__device__ __forceinline__ float wave_fmax_nonneg(float v)
{
    v = dpp_fmax<0xb1, 0xf>(v);
    v = dpp_fmax<0x4e, 0xf>(v);
    v = dpp_fmax<0x141, 0xf>(v);
    v = dpp_fmax<0x140, 0xf>(v);
    v = dpp_fmax<0x142, 0xa>(v);
    v = dpp_fmax<0x143, 0xc>(v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Read 8 bytes starting at byte `off` of a 4-byte-aligned LDS array as two
// dwords.  The dword reads stay 4-byte aligned; the byte phase (off & 3) is
// taken out with v_alignbyte.  `off` must be relative to the aligned array
// base, not to a block inside it (Q6_K blocks are 210 bytes, so odd blocks
// start 2 bytes past a dword boundary).
__device__ __forceinline__ void lds_read8_even(const uint8_t *lds, uint32_t off, uint32_t &a,
                                               uint32_t &b)
{
    const uint32_t *p = reinterpret_cast<const uint32_t *>(lds + (off & ~3u));
    const uint32_t w0 = p[0], w1 = p[1], w2 = p[2];
    const uint32_t sh = off & 3u;
    a = __builtin_amdgcn_alignbyte(w1, w0, sh);
    b = __builtin_amdgcn_alignbyte(w2, w1, sh);
}

__device__ __forceinline__ uint32_t lds_read_u16(const uint8_t *lds, uint32_t off)
{
    return *reinterpret_cast<const uint16_t *>(lds + off);
}

// One direct-to-LDS copy: lane l's 16 bytes at `src` land at LDS byte address
// lds + 16 l.  Inline assembly, so that the compiler does not track it: as a
// compiler-visible LDS write it would make later LDS reads it cannot prove
// disjoint wait for every copy in flight (vmcnt(0)), including copies issued
// ahead for later rows; kernels using it wait with explicit s_waitcnt vmcnt.
__device__ __forceinline__ void lds_copy16(const void *src, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(src), "s"(lds)
                 : "memory", "m0");
}

// Workgroup execution barrier without a memory fence.  __syncthreads()
// carries a workgroup-scope release fence, which makes the compiler wait for
// every outstanding direct-to-LDS copy (they count as LDS writes), including
// copies issued ahead for the next stage.  Kernels that track their copies
// with explicit s_waitcnt use this instead; the empty asm statements keep the
// compiler from moving LDS accesses across the barrier.
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Signed byte k (0..3) of a dword, as float.
__device__ __forceinline__ float sbyte_f(uint32_t w, int k)
{
    return (float)(int32_t)(int8_t)(w >> (8 * k));
}
// Unsigned byte k of a dword, as float (v_cvt_f32_ubyte{k}).
__device__ __forceinline__ float ubyte_f(uint32_t w, int k)
{
    return (float)((w >> (8 * k)) & 0xffu);
}

// 6-bit scale and min of sub-blocks 2j and 2j+1 as floats (src/Dequant.jl:345-362),
// from header dwords s0 = scales[0..3], s1 = scales[4..7], s2 = scales[8..11].
__device__ __forceinline__ void k_scale_min_pair(uint32_t s0, uint32_t s1, uint32_t s2, int j,
                                                 float &scA, float &mA, float &scB, float &mB)
{
    const uint32_t sh = 16u * (uint32_t)(j & 1); // bytes 2(j&1), 2(j&1)+1
    const uint32_t w0 = s0 >> sh, w1 = s1 >> sh, w2 = s2 >> sh;
    // sub-blocks 0..3: low 6 bits of scales[i] / scales[i+4]
    const uint32_t sc_lo = w0 & 0x3f3fu, m_lo = w1 & 0x3f3fu;
    // sub-blocks 4..7: nibbles of scales[i+4], top bits of scales[i-4] / scales[i]
    const uint32_t sc_hi = (w2 & 0x0f0fu) | ((w0 >> 2) & 0x3030u);
    const uint32_t m_hi = ((w2 >> 4) & 0x0f0fu) | ((w1 >> 2) & 0x3030u);
    const uint32_t sc = j >= 2 ? sc_hi : sc_lo, m = j >= 2 ? m_hi : m_lo;
    scA = ubyte_f(sc, 0);
    scB = ubyte_f(sc, 1);
    mA = ubyte_f(m, 0);
    mB = ubyte_f(m, 1);
}

// Row epilogues of the GEMV kernels that read one value r per output row
// (r may be the output row itself):
//   kEpiAdd:    y = r + v, the residual add of src/ModelCPU.jl:913-920;
//   kEpiSwiglu: y = silu(r) * v = r / (1 + exp(-r)) * v, the SwiGLU of an
//               unfused gate/up pair (r: the gate row already in y, v: the up
//               row), src/ModelCPU.jl:492-503.
constexpr int kEpiAdd = 0, kEpiSwiglu = 1;
__device__ __forceinline__ float epi_apply(float r, float v, int epi)
{
    return epi == kEpiSwiglu ? (r / (1.0f + expf(-r))) * v : r + v;
}

// Wait until at most n of this wave's vector-memory operations are
// outstanding (n <= 31; expcnt and lgkmcnt are not waited on).
__device__ __forceinline__ void wait_vmcnt(int n)
{
#define IHIP_VM(N)                                                                             \
    case N:                                                                                    \
        __builtin_amdgcn_s_waitcnt(((N)&15) | (((N) >> 4) << 14) | 0x0F70);                    \
        break;
    switch (n) {
        IHIP_VM(0) IHIP_VM(1) IHIP_VM(2) IHIP_VM(3) IHIP_VM(4) IHIP_VM(5) IHIP_VM(6) IHIP_VM(7)
        IHIP_VM(8) IHIP_VM(9) IHIP_VM(10) IHIP_VM(11) IHIP_VM(12) IHIP_VM(13) IHIP_VM(14)
        IHIP_VM(15) IHIP_VM(16) IHIP_VM(17) IHIP_VM(18) IHIP_VM(19) IHIP_VM(20) IHIP_VM(21)
        IHIP_VM(22) IHIP_VM(23) IHIP_VM(24) IHIP_VM(25) IHIP_VM(26) IHIP_VM(27) IHIP_VM(28)
        IHIP_VM(29) IHIP_VM(30) IHIP_VM(31)
    default:
        __builtin_amdgcn_s_waitcnt(0);
    }
#undef IHIP_VM
}

// ---- Q4_K / Q5_K (and IQ4_NL) blocks as lanes load them -----------------
// Lane (block b, sub-block pair j): the block header (d, dmin, scales), the 32
// qs bytes of pair j (low nibbles: sub-block 2j, high: 2j + 1) and (Q5_K) the
// 32 qh bytes, as 128-bit loads (both block sizes are 16-byte multiples).
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

// IQ4_NL as eight 18-byte blocks per 256 columns (144 bytes, a 16-byte
// multiple): lane j's 36 bytes are blocks 2j and 2j + 1, which start j dwords
// into the three 16-byte units at or below byte 36 j.
template <>
struct KFmt<kIQ4_NL> {
    static constexpr int BYTES = 144, QS = 0;
};

// Q8_0: eight 34-byte blocks per 256 columns (272 bytes); lane j's 68 bytes
// are blocks 2j and 2j + 1, from byte 68 j (a dword boundary), loaded exactly:
// four 16-byte loads and one dword at dword alignment.
template <>
struct KFmt<kQ8_0> {
    static constexpr int BYTES = 272, QS = 0;
};

struct KBytes {
    uint4 h, q0, q1, e0, e1;
};

template <int FMT>
__device__ __forceinline__ void kbytes_load(const uint8_t *__restrict__ blk, int j, KBytes &B)
{
    using F = KFmt<FMT>;
    if constexpr (FMT == kIQ4_NL) {
        const uint8_t *u = blk + ((36 * j) & ~15);
        B.h = *reinterpret_cast<const uint4 *>(u);
        B.q0 = *reinterpret_cast<const uint4 *>(u + 16);
        B.q1 = *reinterpret_cast<const uint4 *>(u + 32);
        return;
    }
    if constexpr (FMT == kQ8_0) {
        typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
        const uint8_t *u = blk + 68 * j;
        auto ld16 = [](const uint8_t *p) {
            const u32x4_a4 v = *reinterpret_cast<const u32x4_a4 *>(p);
            return make_uint4(v.x, v.y, v.z, v.w);
        };
        B.h = ld16(u);
        B.q0 = ld16(u + 16);
        B.q1 = ld16(u + 32);
        B.e0 = ld16(u + 48);
        B.e1 = make_uint4(*reinterpret_cast<const uint32_t *>(u + 64), 0u, 0u, 0u);
        return;
    }
    B.h = *reinterpret_cast<const uint4 *>(blk);
    B.q0 = *reinterpret_cast<const uint4 *>(blk + F::QS + 32 * j);
    B.q1 = *reinterpret_cast<const uint4 *>(blk + F::QS + 32 * j + 16);
    if constexpr (FMT == kQ5_K) {
        B.e0 = *reinterpret_cast<const uint4 *>(blk + 16);
        B.e1 = *reinterpret_cast<const uint4 *>(blk + 32);
    }
}

} // namespace ihip
