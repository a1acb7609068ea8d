// kq_q8k.hip -- the int8-activation numerics of the reference C kernels, bit
// for bit: quantize_row_q8_K (src/kernels/quant_kernels.c:166-194 of
// Inferno.jl) and the q{4,5,6}_k_gemv drivers (:602-650) over
// vec_dot_q{4,5,6}_K_q8_K (AVX2 branches, :212-277, :319-397, :444-521).
//
// Every integer product and sum of those routines is exact, so the only
// roundings are in a few fp32 operations whose order is fixed: per 256-block
// d = amax / 127, id = 1 / d, q = roundf(x * id); per row, for each block in
// order, d = y.d * d_w and acc[t] = fma(d, float(sumi[t]), acc[t]) on eight
// lane accumulators t (integer lane t of the AVX2 code holds bytes 4t..4t+3 of
// every 32-byte chunk), then the AVX2 horizontal sums.  Here a wave takes one
// row: its lanes form the exact integer lane sums of every block with
// v_dot4_i32_i8 in parallel and stage (d, float(sumi)) in LDS, then eight
// lanes run the eight fp32 chains in block order and lane 0 adds them up in
// the horizontal-sum order.  Q4_K keeps four more chains for the dmin terms
// (accm, :262-270), Q5_K one (summs, :352-360).
#include "kq_common.h"
#include "kq_launch.h"

namespace ihip {

constexpr int kQ8KBytes = 292; // float d, int8 qs[256], int16 bsums[16]

// One 256-element block of quantize_row_q8_K across a wave: lane l holds
// elements 4l..4l+3 and gets their four quants packed in a dword, the block's
// d, and (lanes l % 4 == 0) the sum of the 16 quants of elements 4l..4l+15.
struct Q8KLane {
    uint32_t q;
    int bsum;
    float d;
};

__device__ __forceinline__ Q8KLane q8k_quantize_lane(float v0, float v1, float v2, float v3)
{
    // amax: the strict `>` scan from 0 skips NaN, as fmaxf does (in any order)
    const float amax =
        wave_fmax_nonneg(fmaxf(fmaxf(fabsf(v0), fabsf(v1)), fmaxf(fabsf(v2), fabsf(v3))));
    Q8KLane L;
    L.d = amax / 127.0f;
    const float id = L.d != 0.0f ? 1.0f / L.d : 0.0f;
    const int q0 = (int)roundf(v0 * id), q1 = (int)roundf(v1 * id);
    const int q2 = (int)roundf(v2 * id), q3 = (int)roundf(v3 * id);
    L.q = (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) | ((uint32_t)(q2 & 0xff) << 16) |
          ((uint32_t)(q3 & 0xff) << 24);
    int s = q0 + q1 + q2 + q3; // bsums: 16 elements = 4 lanes (a quad)
    s += __builtin_amdgcn_mov_dpp(s, 0xb1, 0xf, 0xf, false); // lane ^ 1
    s += __builtin_amdgcn_mov_dpp(s, 0x4e, 0xf, 0xf, false); // lane ^ 2
    L.bsum = s;
    return L;
}

// Store a lane's share of Q8_K block yb (292 bytes, 4-byte aligned).
__device__ __forceinline__ void q8k_store_lane(uint8_t *yb, const Q8KLane &L, int lane)
{
    *reinterpret_cast<uint32_t *>(yb + 4 + 4 * lane) = L.q;
    if ((lane & 3) == 0)
        *reinterpret_cast<int16_t *>(yb + 260 + 2 * (lane >> 2)) = (int16_t)L.bsum;
    if (lane == 0)
        *reinterpret_cast<float *>(yb) = L.d;
}

// One wave per 256-element block: lane l quantizes elements 4l..4l+3.
// x needs 4-byte alignment, y (the Q8_K blocks) 4-byte alignment.
__global__ __launch_bounds__(64) void k_quantize_q8k(const float *__restrict__ x,
                                                     uint8_t *__restrict__ y)
{
    const int lane = threadIdx.x;
    const size_t blk = blockIdx.x;
    const float *src = x + blk * 256 + 4 * lane;
    const Q8KLane L = q8k_quantize_lane(src[0], src[1], src[2], src[3]);
    q8k_store_lane(y + blk * kQ8KBytes, L, lane);
}

__device__ __forceinline__ int q8k_dword(const uint8_t *by, int off)
{
    return *reinterpret_cast<const int *>(by + 4 + off);
}

__device__ __forceinline__ int q8k_bsum(const uint8_t *by, int g)
{
    return *reinterpret_cast<const int16_t *>(by + 260 + 2 * g);
}

// 32 bits at a 2-byte-aligned address (Q6_K blocks are 210 bytes).
__device__ __forceinline__ uint32_t ld32_a2(const uint8_t *p)
{
    const uint16_t *h = reinterpret_cast<const uint16_t *>(p);
    return (uint32_t)h[0] | ((uint32_t)h[1] << 16);
}

__device__ __forceinline__ int sdot4(uint32_t a, int b, int c)
{
    return __builtin_amdgcn_sdot4((int)a, b, c, false);
}

// The exact integer part of block `bx` against Q8_K block `by` for integer
// lane t: sumi[t], plus (Q4_K, t < 4) the dmin product of accm[t] and
// (Q5_K, t == 0) the dmin sum.  d and dmin are y.d * d_w and -y.d * dmin_w.
template <int FMT>
__device__ __forceinline__ void q8k_item(const uint8_t *bx, const uint8_t *by, int t, int &sumi,
                                         int &mterm, float &d, float &dmin)
{
    const float yd = *reinterpret_cast<const float *>(by);
    sumi = 0;
    mterm = 0;
    if constexpr (FMT == kQ6_K) {
        d = yd * h2f(*reinterpret_cast<const uint16_t *>(bx + 208));
        dmin = 0.0f;
        const int8_t *sc = reinterpret_cast<const int8_t *>(bx + 192);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t hq = ld32_a2(bx + 128 + 32 * j + 4 * t);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t lb = ld32_a2(bx + 64 * j + 32 * (k & 1) + 4 * t);
                const uint32_t lo = k < 2 ? (lb & 0x0f0f0f0fu) : ((lb >> 4) & 0x0f0f0f0fu);
                const uint32_t q = lo | (((hq >> (2 * k)) & 0x03030303u) << 4);
                const int q8 = q8k_dword(by, 128 * j + 32 * k + 4 * t);
                // sum of (q - 32) * q8 over the four bytes, exactly
                const int p = sdot4(q, q8, 0) - 32 * sdot4(0x01010101u, q8, 0);
                sumi += (int)sc[2 * (4 * j + k) + (t >= 4)] * p;
            }
        }
        return;
    } else {
        const uint4 hd = *reinterpret_cast<const uint4 *>(bx);
        d = yd * h2f(hd.x & 0xffffu);
        dmin = -yd * h2f(hd.x >> 16);
        uint32_t sc[8], mn[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            k_scale_min(hd.y, hd.z, hd.w, i, sc[i], mn[i]);
        const uint8_t *qs = bx + (FMT == kQ4_K ? 16 : 48);
        const uint32_t qh = FMT == kQ5_K ? *reinterpret_cast<const uint32_t *>(bx + 16 + 4 * t) : 0u;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t qw = *reinterpret_cast<const uint32_t *>(qs + 32 * j + 4 * t);
            uint32_t lo = qw & 0x0f0f0f0fu, hi = (qw >> 4) & 0x0f0f0f0fu;
            if constexpr (FMT == kQ5_K) {
                lo |= ((qh >> (2 * j)) & 0x01010101u) << 4;
                hi |= ((qh >> (2 * j + 1)) & 0x01010101u) << 4;
            }
            const int pl = sdot4(lo, q8k_dword(by, 64 * j + 4 * t), 0);
            const int ph = sdot4(hi, q8k_dword(by, 64 * j + 32 + 4 * t), 0);
            sumi += (int)sc[2 * j] * pl + (int)sc[2 * j + 1] * ph;
        }
        if constexpr (FMT == kQ4_K) {
            if (t < 4) { // accm[t]: sub-blocks 2t, 2t+1
                const int s0 = (int16_t)(q8k_bsum(by, 4 * t) + q8k_bsum(by, 4 * t + 1));
                const int s1 = (int16_t)(q8k_bsum(by, 4 * t + 2) + q8k_bsum(by, 4 * t + 3));
                mterm = (int)mn[2 * t] * s0 + (int)mn[2 * t + 1] * s1;
            }
        } else {
            if (t == 0) {
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    mterm += (int)mn[k] * (int16_t)(q8k_bsum(by, 2 * k) + q8k_bsum(by, 2 * k + 1));
            }
        }
    }
}

constexpr int kQ8KChunk = 64; // blocks staged per pass

// One row per wave, four rows per workgroup.  Rows past `outer` exit (the
// waves of a workgroup never synchronise with each other).
template <int FMT>
__global__ __launch_bounds__(256) void k_gemv_q8k(const uint8_t *__restrict__ W,
                                                  const uint8_t *__restrict__ Q,
                                                  float *__restrict__ out, int outer, int nb)
{
    constexpr int BB = FMT == kQ4_K ? 144 : FMT == kQ5_K ? 176 : 210;
    __shared__ float s_sum[4][kQ8KChunk][8];
    __shared__ float s_m[4][kQ8KChunk][4];
    __shared__ float s_d[4][kQ8KChunk];
    __shared__ float s_dm[4][kQ8KChunk];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row = blockIdx.x * 4 + w;
    if (row >= outer)
        return; // wave-uniform
    const int t = lane & 7, slot = lane >> 3;
    const uint8_t *wr = W + (size_t)row * (size_t)nb * BB;
    float acc = 0.0f; // lane t < 8: acc[t]; Q4_K lanes 8..11: accm[lane - 8]; Q5_K lane 8: summs
    for (int c0 = 0; c0 < nb; c0 += kQ8KChunk) {
        const int cn = min(kQ8KChunk, nb - c0);
        for (int ii = slot; ii < cn; ii += 8) {
            const int i = c0 + ii;
            int sumi, mterm;
            float d, dmin;
            q8k_item<FMT>(wr + (size_t)i * BB, Q + (size_t)i * kQ8KBytes, t, sumi, mterm, d, dmin);
            s_sum[w][ii][t] = (float)sumi;
            if (t < 4)
                s_m[w][ii][t] = (float)mterm;
            if (t == 0) {
                s_d[w][ii] = d;
                s_dm[w][ii] = dmin;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane < 8) {
            for (int ii = 0; ii < cn; ++ii)
                acc = fmaf(s_d[w][ii], s_sum[w][ii][lane], acc);
        } else if ((FMT == kQ4_K && lane < 12) || (FMT == kQ5_K && lane == 8)) {
            for (int ii = 0; ii < cn; ++ii)
                acc = fmaf(s_dm[w][ii], s_m[w][ii][lane - 8], acc);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier(); // the next pass overwrites the stage
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    float a[12];
#pragma unroll
    for (int k = 0; k < 12; ++k)
        a[k] = __shfl(acc, k);
    if (lane == 0) {
        // AVX2 horizontal sums (quant_kernels.c:91-98, 274-275)
        const float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
        float r = (s0 + s2) + (s1 + s3);
        if constexpr (FMT == kQ4_K)
            r = r + ((a[8] + a[10]) + (a[9] + a[11]));
        else if constexpr (FMT == kQ5_K)
            r = r + a[8];
        out[row] = r;
    }
}

// Q4_K / Q5_K rows in the same numerics with the loads of the fp32 kernels:
// lane (block b, sub-block pair j) of a 16-block pass takes its 48 (Q5_K 80)
// weight bytes with 128-bit loads, and 8 waves x 2 rows share x as Q8_K blocks
// in LDS.  QX: the workgroup quantizes x itself (q8k_quantize_lane, the
// arithmetic of k_quantize_q8k), its first blocks loaded ahead of the first
// pass's weights, and workgroup 0 writes the blocks to q8out when given;
// otherwise the Q8_K blocks are read from q8.  A lane forms, for all eight
// integer lanes t, sc[2j] * sum(lo * q8) + sc[2j + 1] * sum(hi * q8) of its
// pair; the four pairs of a block meet in exact integer adds (any grouping
// gives the reference's sumi[t]), and the block's terms are staged in LDS for
// the fp32 chains, which run as in k_gemv_q8k: eight lanes (plus the dmin
// chains) per row, block by block in order.
constexpr int kQ8WMaxBlocks = 128; // rows of up to 32768 columns
constexpr int kQ8WRows = 2;        // rows per wave

template <int FMT, bool QX>
__global__ __launch_bounds__(512) void k_gemv_q8kw(const uint8_t *__restrict__ W,
                                                   const float *__restrict__ x,
                                                   const uint8_t *__restrict__ q8,
                                                   uint8_t *__restrict__ q8out, float *__restrict__ out,
                                                   int outer, int nb)
{
    using F = KFmt<FMT>;
    constexpr int NWV = 8, R = kQ8WRows;
    __shared__ __attribute__((aligned(16))) uint32_t s_qs[kQ8WMaxBlocks * 64]; // quants, 256 B a block
    __shared__ float s_yd[kQ8WMaxBlocks];
    __shared__ __attribute__((aligned(16))) int16_t s_bs[kQ8WMaxBlocks * 16];
    // per wave and row, per block of the pass: float(sumi[0..7]), d, dmin, the dmin terms
    __shared__ float s_st[NWV][R][16][14];

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int b = lane >> 2, j = lane & 3;
    const size_t row_bytes = (size_t)nb * F::BYTES;
    const int row0 = (blockIdx.x * NWV + w) * R;

    // x of this wave's first two blocks, ahead of the weights (QX)
    float4 xa = make_float4(0.f, 0.f, 0.f, 0.f), xb = xa;
    if constexpr (QX) {
        if (w < nb)
            xa = *reinterpret_cast<const float4 *>(x + (size_t)w * 256 + 4 * lane);
        if (w + NWV < nb)
            xb = *reinterpret_cast<const float4 *>(x + (size_t)(w + NWV) * 256 + 4 * lane);
    }
    KBytes B[R];
    auto load_pass = [&](int p) {
        const int blk = 16 * p + (b < nb - 16 * p ? b : 0);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = min(row0 + r, outer - 1);
            kbytes_load<FMT>(W + (size_t)row * row_bytes + (size_t)blk * F::BYTES, j, B[r]);
        }
    };
    load_pass(0);
    __builtin_amdgcn_sched_barrier(0);

    // x as Q8_K blocks in LDS
    if constexpr (QX) {
        auto quantize = [&](int blk, float4 v) {
            const Q8KLane L = q8k_quantize_lane(v.x, v.y, v.z, v.w);
            s_qs[blk * 64 + lane] = L.q;
            if ((lane & 3) == 0)
                s_bs[blk * 16 + (lane >> 2)] = (int16_t)L.bsum;
            if (lane == 0)
                s_yd[blk] = L.d;
            if (q8out && blockIdx.x == 0)
                q8k_store_lane(q8out + (size_t)blk * kQ8KBytes, L, lane);
        };
        // the two preloaded blocks first, outside any loop that loads: the
        // compiler then waits for x alone (a load in the same loop would make
        // it wait for every load in flight, the weights included)
        if (w < nb)
            quantize(w, xa);
        if (w + NWV < nb)
            quantize(w + NWV, xb);
        for (int blk = w + 2 * NWV; blk < nb; blk += NWV) // rows of more than 16 blocks
            quantize(blk, *reinterpret_cast<const float4 *>(x + (size_t)blk * 256 + 4 * lane));
    } else {
        for (int i = tid; i < nb * 73; i += NWV * 64) { // 73 dwords a block
            const int blk = i / 73, o = i - 73 * blk;
            const uint32_t v = reinterpret_cast<const uint32_t *>(q8 + (size_t)blk * kQ8KBytes)[o];
            if (o == 0)
                s_yd[blk] = __uint_as_float(v);
            else if (o <= 64)
                s_qs[blk * 64 + o - 1] = v;
            else
                reinterpret_cast<uint32_t *>(s_bs)[blk * 8 + o - 65] = v;
        }
    }
    __syncthreads();

    float acc = 0.0f; // lane 16 r + i: row r's chain i (0..7 acc[t]; Q4_K 8..11 accm, Q5_K 8 summs)
    const int npass = (nb + 15) >> 4;
    for (int p = 0; p < npass; ++p) {
        const int nbp = min(16, nb - 16 * p);
        const bool active = b < nbp;
        const int blk = 16 * p + (active ? b : 0);
        if (p > 0)
            load_pass(p);
        uint32_t q[16]; // quants 64j .. 64j + 63 of the block: 32j + 4t (low nibbles), + 32 (high)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint4 v = *reinterpret_cast<const uint4 *>(&s_qs[blk * 64 + 16 * j + 4 * i]);
            q[4 * i] = v.x;
            q[4 * i + 1] = v.y;
            q[4 * i + 2] = v.z;
            q[4 * i + 3] = v.w;
        }
        const float yd = s_yd[blk];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const KBytes &K = B[r];
            uint32_t sc0, m0, sc1, m1;
            k_scale_min(K.h.y, K.h.z, K.h.w, 2 * j, sc0, m0);
            k_scale_min(K.h.y, K.h.z, K.h.w, 2 * j + 1, sc1, m1);
            const uint32_t qw[8] = {K.q0.x, K.q0.y, K.q0.z, K.q0.w, K.q1.x, K.q1.y, K.q1.z, K.q1.w};
            int part[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                uint32_t lo = qw[t] & 0x0f0f0f0fu, hi = (qw[t] >> 4) & 0x0f0f0f0fu;
                if constexpr (FMT == kQ5_K) {
                    const uint32_t e[8] = {K.e0.x, K.e0.y, K.e0.z, K.e0.w, K.e1.x, K.e1.y, K.e1.z, K.e1.w};
                    lo |= ((e[t] >> (2 * j)) & 0x01010101u) << 4;
                    hi |= ((e[t] >> (2 * j + 1)) & 0x01010101u) << 4;
                }
                part[t] = (int)sc0 * sdot4(lo, (int)q[t], 0) + (int)sc1 * sdot4(hi, (int)q[8 + t], 0);
            }
            // the four pairs of the block (lanes 4b .. 4b + 3): exact integer sums,
            // lane pairs then pairs of pairs by DPP quad permutes
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                part[t] += __builtin_amdgcn_mov_dpp(part[t], 0xb1, 0xf, 0xf, false); // lane ^ 1
                part[t] += __builtin_amdgcn_mov_dpp(part[t], 0x4e, 0xf, 0xf, false); // lane ^ 2
            }
            // the dmin terms from this pair's mins: Q4_K accm[j] (sub-blocks 2j,
            // 2j + 1: bsums 4j .. 4j + 3), Q5_K its share of summs
            const int16_t *bs = &s_bs[blk * 16 + 4 * j];
            const int s0 = (int16_t)(bs[0] + bs[1]), s1 = (int16_t)(bs[2] + bs[3]);
            int mt = (int)m0 * s0 + (int)m1 * s1;
            if constexpr (FMT == kQ5_K) { // summs: the four pairs' shares, exactly
                mt += __builtin_amdgcn_mov_dpp(mt, 0xb1, 0xf, 0xf, false);
                mt += __builtin_amdgcn_mov_dpp(mt, 0x4e, 0xf, 0xf, false);
            }
            if (active) { // lane j stages sums 2j and 2j + 1 and its dmin term
                float *st = s_st[w][r][b];
                st[2 * j] = (float)(j == 0 ? part[0] : j == 1 ? part[2] : j == 2 ? part[4] : part[6]);
                st[2 * j + 1] = (float)(j == 0 ? part[1] : j == 1 ? part[3] : j == 2 ? part[5] : part[7]);
                if (j == 0) {
                    st[8] = yd * h2f(K.h.x & 0xffffu);
                    st[9] = -yd * h2f(K.h.x >> 16);
                }
                if (FMT == kQ4_K || j == 0)
                    st[10 + j] = (float)mt;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        {
            const int r = lane >> 4, i = lane & 15;
            if (r < R && (i < 8 || (FMT == kQ4_K && i < 12) || (FMT == kQ5_K && i == 8))) {
                // every stage read first, then the chain of fmas in block order
                const int cd = i < 8 ? 8 : 9, cs = i < 8 ? i : 10 + i - 8;
                float dv[16], sv[16];
#pragma unroll
                for (int bb = 0; bb < 16; ++bb) {
                    dv[bb] = bb < nbp ? s_st[w][r][bb][cd] : 0.0f;
                    sv[bb] = bb < nbp ? s_st[w][r][bb][cs] : 0.0f;
                }
#pragma unroll
                for (int bb = 0; bb < 16; ++bb)
                    if (bb < nbp)
                        acc = fmaf(dv[bb], sv[bb], acc);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier(); // the next pass overwrites the stage
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float a[12]; // the row's chains, read across lanes without LDS
#pragma unroll
        for (int k = 0; k < 12; ++k)
            a[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 16 * r + k));
        const int row = row0 + r;
        if (lane == 0 && row < outer) {
            // AVX2 horizontal sums (quant_kernels.c:91-98, 274-275)
            const float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
            float v = (s0 + s2) + (s1 + s3);
            if constexpr (FMT == kQ4_K)
                v = v + ((a[8] + a[10]) + (a[9] + a[11]));
            else
                v = v + a[8];
            out[row] = v;
        }
    }
}

template <bool QX>
static hipError_t launch_q8kw(int type, const void *w, const float *x, const void *q8, void *q8out,
                              float *out, int nb, int outer, hipStream_t s)
{
    const dim3 grid((unsigned)((outer + 8 * kQ8WRows - 1) / (8 * kQ8WRows))), block(512);
    if (type == kQ4_K)
        hipLaunchKernelGGL((k_gemv_q8kw<kQ4_K, QX>), grid, block, 0, s, (const uint8_t *)w, x,
                           (const uint8_t *)q8, (uint8_t *)q8out, out, outer, nb);
    else
        hipLaunchKernelGGL((k_gemv_q8kw<kQ5_K, QX>), grid, block, 0, s, (const uint8_t *)w, x,
                           (const uint8_t *)q8, (uint8_t *)q8out, out, outer, nb);
    return hipGetLastError();
}

static bool q8kw_ok(int type, const void *w, int nb)
{
    return (type == kQ4_K || type == kQ5_K) && nb >= 1 && nb <= kQ8WMaxBlocks &&
           ((uintptr_t)w & 15u) == 0;
}

hipError_t launch_quantize_q8k(const float *x, void *y, int64_t k, hipStream_t s)
{
    if (k <= 0 || k % 256)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_quantize_q8k, dim3((unsigned)(k / 256)), dim3(64), 0, s, x, (uint8_t *)y);
    return hipGetLastError();
}

hipError_t launch_gemv_q8k(int type, const void *w, const void *q8, float *out, int inner,
                           int outer, hipStream_t s)
{
    const int nb = inner / 256;
    if (q8kw_ok(type, w, nb) && ((uintptr_t)q8 & 3u) == 0)
        return launch_q8kw<false>(type, w, nullptr, q8, nullptr, out, nb, outer, s);
    const dim3 grid((unsigned)((outer + 3) / 4)), block(256);
    switch (type) {
    case kQ4_K:
        hipLaunchKernelGGL(k_gemv_q8k<kQ4_K>, grid, block, 0, s, (const uint8_t *)w,
                           (const uint8_t *)q8, out, outer, nb);
        break;
    case kQ5_K:
        hipLaunchKernelGGL(k_gemv_q8k<kQ5_K>, grid, block, 0, s, (const uint8_t *)w,
                           (const uint8_t *)q8, out, outer, nb);
        break;
    case kQ6_K:
        hipLaunchKernelGGL(k_gemv_q8k<kQ6_K>, grid, block, 0, s, (const uint8_t *)w,
                           (const uint8_t *)q8, out, outer, nb);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gemv_q8k_x(int type, const void *w, const float *x, void *q8out, void *q8tmp,
                             float *out, int inner, int outer, hipStream_t s)
{
    if (inner <= 0 || inner % 256)
        return hipErrorInvalidValue;
    const int nb = inner / 256;
    if (q8kw_ok(type, w, nb) && ((uintptr_t)x & 15u) == 0 && ((uintptr_t)q8out & 3u) == 0)
        return launch_q8kw<true>(type, w, x, nullptr, q8out, out, nb, outer, s);
    void *q8 = q8out ? q8out : q8tmp;
    if (!q8)
        return hipErrorInvalidValue;
    hipError_t e = launch_quantize_q8k(x, q8, inner, s);
    return e == hipSuccess ? launch_gemv_q8k(type, w, q8, out, inner, outer, s) : e;
}

} // namespace ihip
