// kq_dequant.hip -- bit-exact GGML block -> fp32 dequantization on gfx950,
// the generic (any alignment) GEMV fallback, and the element-wise SwiGLU
// kernels.
//
// Dequant semantics: src/Dequant.jl:304-601 (Inferno.jl).  Every product
// in those formulas is exact in fp32 (d*sc <= 17 significant bits, times a
// <= 6-bit quant), so forming the same products and the single final
// subtraction gives the reference bits whether or not the compiler fuses
// them into an FMA.
#include "kq_common.h"
#include "kq_launch.h"

namespace ihip {

// ---- element-at-a-time decode (generic paths) ---------------------------
__device__ __forceinline__ uint32_t rd16(const uint8_t *p) { return p[0] | (p[1] << 8); }

__device__ __forceinline__ void k_scale_min_bytes(const uint8_t *s, int i, uint32_t &sc,
                                                  uint32_t &m)
{
    if (i < 4) {
        sc = s[i] & 63u;
        m = s[i + 4] & 63u;
    } else {
        sc = (s[i + 4] & 15u) | ((uint32_t)(s[i - 4] >> 6) << 4);
        m = (uint32_t)(s[i + 4] >> 4) | ((uint32_t)(s[i] >> 6) << 4);
    }
}

// Element e of one block, src/Dequant.jl element order.
// IQ4_NL's non-linear 4-bit grid (src/QuantsData.jl:384).
__constant__ int8_t kIQ4NLValues[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                        1,    13,   25,  38,  53,  69,  89,  113};

template <int FMT>
__device__ __forceinline__ float elem(const uint8_t *b, int e)
{
    if constexpr (FMT == kQ8_0) {
        return h2f(rd16(b)) * (float)(int8_t)b[2 + e];
    } else if constexpr (FMT == kIQ4_NL) {
        // src/Dequant.jl:683-693: element j low nibble of qs[j], element
        // j + 16 high nibble; d * value (exact in fp32)
        const uint32_t qb = b[2 + (e & 15)];
        return h2f(rd16(b)) * (float)kIQ4NLValues[e < 16 ? (qb & 15u) : (qb >> 4)];
    } else if constexpr (FMT == kQ6_K) {
        const int n = e >> 7, r = e & 127, g = r >> 5, l = r & 31;
        const uint32_t lb = b[64 * n + l + 32 * (g & 1)];
        const uint32_t nib = g < 2 ? (lb & 15u) : (lb >> 4);
        const uint32_t h = (b[128 + 32 * n + l] >> (2 * g)) & 3u;
        const int q = (int)(nib | (h << 4)) - 32;
        const int sc = (int8_t)b[192 + 8 * n + 2 * g + (l >> 4)];
        return (h2f(rd16(b + 208)) * (float)sc) * (float)q;
    } else {
        const int j = e >> 6, hi = (e >> 5) & 1, l = e & 31, sub = 2 * j + hi;
        uint32_t sc, m;
        k_scale_min_bytes(b + 4, sub, sc, m);
        constexpr int QS = FMT == kQ5_K ? 48 : 16;
        const uint32_t qb = b[QS + 32 * j + l];
        uint32_t q = hi ? (qb >> 4) : (qb & 15u);
        if constexpr (FMT == kQ5_K)
            q += ((b[16 + l] >> sub) & 1u) << 4;
        const float d1 = h2f(rd16(b)) * (float)sc, m1 = h2f(rd16(b + 2)) * (float)m;
        return d1 * (float)q - m1;
    }
}

// Generic GEMV: one wave per row, lanes stride over the row's elements with
// byte loads.  Used only when a pointer or row stride rules out the
// 128-bit paths.
template <int FMT>
__global__ __launch_bounds__(256) void k_gemv_generic(const uint8_t *__restrict__ W,
                                                      const float *__restrict__ x,
                                                      float *y, int outer, int inner,
                                                      const float *resid, int epi)
{
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= outer)
        return;
    constexpr int BE = block_elems(FMT), BB = block_bytes(FMT);
    const uint8_t *rp = W + (size_t)row * (size_t)(inner / BE) * BB;
    float acc = 0.0f;
    for (int c = lane; c < inner; c += 64)
        acc = fmaf(elem<FMT>(rp + (size_t)(c / BE) * BB, c % BE), x[c], acc);
    acc = wave_sum(acc);
    if (lane == 0)
        y[row] = resid ? epi_apply(resid[row], acc, epi) : acc; // resid may be y
}

template <int FMT>
__global__ __launch_bounds__(256) void k_dequant_generic(const uint8_t *__restrict__ src,
                                                         float *__restrict__ dst, int64_t n)
{
    constexpr int BE = block_elems(FMT), BB = block_bytes(FMT);
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n;
         e += (int64_t)gridDim.x * 256)
        dst[e] = elem<FMT>(src + (e / BE) * BB, (int)(e % BE));
}

// ---- fast dequant: Q4_K / Q5_K, one 16-byte qs chunk per thread ---------
template <int FMT>
__global__ __launch_bounds__(256) void k_dequant_kdirect(const uint8_t *__restrict__ src,
                                                         float *__restrict__ dst, int64_t nblocks)
{
    constexpr int BB = FMT == kQ5_K ? 176 : 144, QS = FMT == kQ5_K ? 48 : 16;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t b = t >> 3;
    if (b >= nblocks)
        return;
    const int k = (int)(t & 7), j = k >> 1, l0 = 16 * (k & 1);
    const uint8_t *bp = src + b * BB;
    const uint4 h = *reinterpret_cast<const uint4 *>(bp);
    const uint4 q = *reinterpret_cast<const uint4 *>(bp + QS + 16 * k);
    uint4 qh = make_uint4(0, 0, 0, 0);
    if constexpr (FMT == kQ5_K)
        qh = *reinterpret_cast<const uint4 *>(bp + 16 + l0);
    const float d = h2f(h.x & 0xffffu), dmin = h2f(h.x >> 16);
    uint32_t scA, mA, scB, mB;
    k_scale_min(h.y, h.z, h.w, 2 * j, scA, mA);
    k_scale_min(h.y, h.z, h.w, 2 * j + 1, scB, mB);
    const float dA = d * (float)scA, minA = dmin * (float)mA;
    const float dB = d * (float)scB, minB = dmin * (float)mB;
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
    const uint32_t hw[4] = {qh.x, qh.y, qh.z, qh.w};
    float4 *oa = reinterpret_cast<float4 *>(dst + b * 256 + 64 * j + l0);
    float4 *ob = reinterpret_cast<float4 *>(dst + b * 256 + 64 * j + 32 + l0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t lo = qw[i] & 0x0f0f0f0fu, hi = (qw[i] >> 4) & 0x0f0f0f0fu;
        if constexpr (FMT == kQ5_K) {
            lo |= ((hw[i] >> (2 * j)) & 0x01010101u) << 4;
            hi |= ((hw[i] >> (2 * j + 1)) & 0x01010101u) << 4;
        }
        oa[i] = make_float4(dA * ubyte_f(lo, 0) - minA, dA * ubyte_f(lo, 1) - minA,
                            dA * ubyte_f(lo, 2) - minA, dA * ubyte_f(lo, 3) - minA);
        ob[i] = make_float4(dB * ubyte_f(hi, 0) - minB, dB * ubyte_f(hi, 1) - minB,
                            dB * ubyte_f(hi, 2) - minB, dB * ubyte_f(hi, 3) - minB);
    }
}

// ---- fast dequant: Q6_K / Q8_0 via an LDS-staged group of 8 blocks ------
// 8 blocks are 1680 B (Q6_K) / 272 B (Q8_0): a 16-byte multiple, so a group
// starting on a 16-byte boundary can be copied with 128-bit loads.
template <int FMT>
__global__ __launch_bounds__(256) void k_dequant_staged(const uint8_t *__restrict__ src,
                                                        float *__restrict__ dst, int64_t ngroups)
{
    constexpr int GB = 8 * block_bytes(FMT), CH = GB / 16;
    constexpr int GPW = FMT == kQ6_K ? 1 : 8; // groups per workgroup
    __shared__ __attribute__((aligned(16))) uint8_t tile[GPW * GB + 16];
    const int64_t g0 = (int64_t)blockIdx.x * GPW;
    for (int c = threadIdx.x; c < GPW * CH; c += 256) {
        const int64_t g = g0 + c / CH;
        if (g < ngroups)
            *reinterpret_cast<uint4 *>(tile + 16 * c) =
                *reinterpret_cast<const uint4 *>(src + g0 * GB + 16 * (int64_t)c);
    }
    __syncthreads();
    if constexpr (FMT == kQ6_K) {
        if (g0 >= ngroups)
            return;
        // 8 blocks x 32 units of 8 consecutive outputs = 256 threads
        const int bs = threadIdx.x >> 5, u = threadIdx.x & 31;
        const int n = u >> 4, g = (u >> 2) & 3, l0 = 8 * (u & 3);
        const uint32_t bo = 210u * bs; // block offset in the 16-byte-aligned tile
        uint32_t L[2], H[2], S[2];
        lds_read8_even(tile, bo + 64 * n + 32 * (g & 1) + l0, L[0], L[1]);
        lds_read8_even(tile, bo + 128 + 32 * n + l0, H[0], H[1]);
        lds_read8_even(tile, bo + 192 + 8 * n, S[0], S[1]);
        const float d = h2f(lds_read_u16(tile, bo + 208));
        const int si = 2 * g + (l0 >> 4);
        const float ds = d * sbyte_f(S[si >> 2], si & 3);
        float *out = dst + (g0 * 8 + bs) * 256 + 128 * n + 32 * g + l0;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const uint32_t nib = g < 2 ? (L[t] & 0x0f0f0f0fu) : ((L[t] >> 4) & 0x0f0f0f0fu);
            const uint32_t hb = ((H[t] >> (2 * g)) & 0x03030303u) << 4;
            const uint32_t v = nib | hb;
            reinterpret_cast<float4 *>(out)[t] =
                make_float4(ds * (float)((int)((v >> 0) & 0xff) - 32),
                            ds * (float)((int)((v >> 8) & 0xff) - 32),
                            ds * (float)((int)((v >> 16) & 0xff) - 32),
                            ds * (float)((int)((v >> 24) & 0xff) - 32));
        }
    } else {
        // 64 blocks x 8 quads of 4 outputs = 512 float4 per workgroup
        for (int i = threadIdx.x; i < GPW * 64; i += 256) {
            const int b = i >> 3, quad = i & 7; // b: block in the workgroup tile
            if (g0 * 8 + b >= ngroups * 8)
                break;
            const uint32_t off = 34u * b;
            const float d = h2f(lds_read_u16(tile, off));
            const uint32_t o = off + 2 + 4 * quad;
            const uint32_t *p = reinterpret_cast<const uint32_t *>(tile + (o & ~3u));
            const uint32_t q = __builtin_amdgcn_alignbyte(p[1], p[0], o & 3u);
            reinterpret_cast<float4 *>(dst + (g0 * 8 + b) * 32)[quad] =
                make_float4(d * sbyte_f(q, 0), d * sbyte_f(q, 1), d * sbyte_f(q, 2),
                            d * sbyte_f(q, 3));
        }
    }
}

// ---- element-wise SwiGLU (FusedKernels.jl:203-230) ---------------------
__global__ __launch_bounds__(256) void k_mlp_gate_mul(float *__restrict__ gate,
                                                      const float *__restrict__ up, int64_t n)
{
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * 256) {
        const float g = gate[i];
        gate[i] = g / (1.0f + expf(-g)) * up[i];
    }
}

__global__ __launch_bounds__(256) void k_silu_gate_mul(float *__restrict__ out,
                                                       const float *__restrict__ x,
                                                       const float *__restrict__ gate, int64_t n)
{
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * 256) {
        const float v = x[i];
        out[i] = v / (1.0f + expf(-v)) * gate[i];
    }
}

static unsigned grid_for(int64_t n, int64_t per_block, int64_t cap = 65535)
{
    int64_t g = (n + per_block - 1) / per_block;
    if (g > cap) g = cap;
    if (g < 1) g = 1;
    return (unsigned)g;
}

hipError_t launch_gemv_generic(int type, const void *w, const float *x, float *y, int inner,
                               int outer, hipStream_t s, const float *resid, int epi)
{
    const dim3 grid((outer + 3) / 4), block(256);
    const uint8_t *W = (const uint8_t *)w;
    switch (type) {
    case kQ4_K: hipLaunchKernelGGL(k_gemv_generic<kQ4_K>, grid, block, 0, s, W, x, y, outer, inner, resid, epi); break;
    case kQ5_K: hipLaunchKernelGGL(k_gemv_generic<kQ5_K>, grid, block, 0, s, W, x, y, outer, inner, resid, epi); break;
    case kQ6_K: hipLaunchKernelGGL(k_gemv_generic<kQ6_K>, grid, block, 0, s, W, x, y, outer, inner, resid, epi); break;
    case kQ8_0: hipLaunchKernelGGL(k_gemv_generic<kQ8_0>, grid, block, 0, s, W, x, y, outer, inner, resid, epi); break;
    case kIQ4_NL: hipLaunchKernelGGL(k_gemv_generic<kIQ4_NL>, grid, block, 0, s, W, x, y, outer, inner, resid, epi); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_dequant(int type, const void *src, float *dst, int64_t n, bool aligned,
                          hipStream_t s)
{
    const uint8_t *S = (const uint8_t *)src;
    const int64_t nb = n / block_elems(type);
    if (aligned && (type == kQ4_K || type == kQ5_K)) {
        const unsigned grid = (unsigned)((nb * 8 + 255) / 256);
        if (type == kQ4_K)
            hipLaunchKernelGGL(k_dequant_kdirect<kQ4_K>, dim3(grid), dim3(256), 0, s, S, dst, nb);
        else
            hipLaunchKernelGGL(k_dequant_kdirect<kQ5_K>, dim3(grid), dim3(256), 0, s, S, dst, nb);
        return hipGetLastError();
    }
    if (aligned && (type == kQ6_K || type == kQ8_0) && nb % 8 == 0) {
        const int64_t ng = nb / 8;
        if (type == kQ6_K)
            hipLaunchKernelGGL(k_dequant_staged<kQ6_K>, dim3((unsigned)ng), dim3(256), 0, s, S, dst, ng);
        else
            hipLaunchKernelGGL(k_dequant_staged<kQ8_0>, dim3((unsigned)((ng + 7) / 8)), dim3(256), 0, s,
                               S, dst, ng);
        return hipGetLastError();
    }
    const unsigned grid = grid_for(n, 256, 1 << 20);
    switch (type) {
    case kQ4_K: hipLaunchKernelGGL(k_dequant_generic<kQ4_K>, dim3(grid), dim3(256), 0, s, S, dst, n); break;
    case kQ5_K: hipLaunchKernelGGL(k_dequant_generic<kQ5_K>, dim3(grid), dim3(256), 0, s, S, dst, n); break;
    case kQ6_K: hipLaunchKernelGGL(k_dequant_generic<kQ6_K>, dim3(grid), dim3(256), 0, s, S, dst, n); break;
    case kQ8_0: hipLaunchKernelGGL(k_dequant_generic<kQ8_0>, dim3(grid), dim3(256), 0, s, S, dst, n); break;
    case kIQ4_NL: hipLaunchKernelGGL(k_dequant_generic<kIQ4_NL>, dim3(grid), dim3(256), 0, s, S, dst, n); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- rmsnorm_cpu! (src/ModelCPU.jl:111-123) --------------------------------
// One workgroup: sum of squares, scale = 1 / sqrt(ss / n + eps), then
// out[i] = x[i] * scale * w[i] in the reference's order.  out may alias x.
__global__ __launch_bounds__(1024) void k_rmsnorm(const float *x, const float *__restrict__ w,
                                                  float eps, float *out, int n)
{
    __shared__ float part[16];
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += 1024)
        ss = fmaf(x[i], x[i], ss);
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0)
        part[threadIdx.x >> 6] = ss;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k)
        t += part[k];
    const float scale = 1.0f / sqrtf(t / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += 1024)
        out[i] = x[i] * scale * w[i];
}

hipError_t launch_rmsnorm(const float *x, const float *w, float eps, float *out, int n,
                          hipStream_t s)
{
    hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(1024), 0, s, x, w, eps, out, n);
    return hipGetLastError();
}

hipError_t launch_mlp_gate_mul(float *gate, const float *up, int64_t n, hipStream_t s)
{
    hipLaunchKernelGGL(k_mlp_gate_mul, dim3(grid_for(n, 256)), dim3(256), 0, s, gate, up, n);
    return hipGetLastError();
}

hipError_t launch_silu_gate_mul(float *out, const float *x, const float *gate, int64_t n,
                                hipStream_t s)
{
    hipLaunchKernelGGL(k_silu_gate_mul, dim3(grid_for(n, 256)), dim3(256), 0, s, out, x, gate, n);
    return hipGetLastError();
}

} // namespace ihip
