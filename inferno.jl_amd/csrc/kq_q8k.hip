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

// One wave per 256-element block: lane l quantizes elements 4l..4l+3.
// x needs 4-byte alignment, y (the Q8_K blocks) 4-byte alignment.
__global__ __launch_bounds__(64) void k_quantize_q8k(const float *__restrict__ x,
                                                     uint8_t *__restrict__ y)
{
    const int lane = threadIdx.x;
    const size_t blk = blockIdx.x;
    const float *src = x + blk * 256 + 4 * lane;
    const float v0 = src[0], v1 = src[1], v2 = src[2], v3 = src[3];
    // amax: the strict `>` scan from 0 skips NaN, as fmaxf does
    float amax = fmaxf(fmaxf(fabsf(v0), fabsf(v1)), fmaxf(fabsf(v2), fabsf(v3)));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
        amax = fmaxf(amax, __shfl_xor(amax, o));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const int q0 = (int)roundf(v0 * id), q1 = (int)roundf(v1 * id);
    const int q2 = (int)roundf(v2 * id), q3 = (int)roundf(v3 * id);
    uint8_t *yb = y + blk * kQ8KBytes;
    *reinterpret_cast<uint32_t *>(yb + 4 + 4 * lane) =
        (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) | ((uint32_t)(q2 & 0xff) << 16) |
        ((uint32_t)(q3 & 0xff) << 24);
    int s = q0 + q1 + q2 + q3; // bsums: 16 elements = 4 lanes
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    if ((lane & 3) == 0)
        *reinterpret_cast<int16_t *>(yb + 260 + 2 * (lane >> 2)) = (int16_t)s;
    if (lane == 0)
        *reinterpret_cast<float *>(yb) = d;
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

} // namespace ihip
