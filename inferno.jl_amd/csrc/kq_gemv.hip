// kq_gemv.hip -- gfx950 dequant-fused GEMV kernels for GGML K-quant/Q8_0
// weights and fp32 activations: y[r] = sum_c W[r,c] x[c].
//
// Semantics: the fp32-activation path of Inferno.jl's mul_quant_mat_vec
// (src/ModelCPU.jl:285-379) with the weights of src/Dequant.jl:304-601.
// Activations stay fp32 (the reference C path's int8 re-quantization of x,
// src/kernels/quant_kernels.c:166-194, is not used: it breaks the
// 1e-4*||w_row||*||x|| bound).
//
// Work decomposition (wave64):
//   * the K axis is cut into 2048-column segments; within a segment each of
//     the 64 lanes owns 32 columns for the whole kernel, keeps those 32 x
//     values in registers and reuses them across the R rows its wave owns;
//   * per row, a lane reduces its 32 weights against its 32 x values; a
//     wave-wide butterfly gives the row total.
//   * Q4_K / Q5_K blocks are 16-byte multiples, so lanes load their bytes
//     straight from HBM with 128-bit loads ("direct" kernels): 8 lanes per
//     block, one 16-byte qs chunk (32 weights) each, plus the block header.
//   * Q6_K (210 B) and Q8_0 (34 B) blocks are not 16-byte aligned; the
//     workgroup streams its rows' bytes into LDS with coalesced 128-bit
//     loads and lanes re-slice blocks from LDS ("staged" kernels).
// Per-sub-block sums of x (shared by all rows) absorb the `dmin*m` term of
// Q4_K/Q5_K and the -32 offset of Q6_K, so the inner loop is one convert and
// one FMA per weight.
#include "kq_common.h"
#include "kq_launch.h"

namespace ihip {

// ------------------------------------------------------------------------
// Q4_K / Q5_K direct kernels
// ------------------------------------------------------------------------
template <int FMT>
struct KDirect;
template <>
struct KDirect<kQ4_K> {
    static constexpr int BYTES = 144, QS = 16;
};
template <>
struct KDirect<kQ5_K> {
    static constexpr int BYTES = 176, QS = 48, QH = 16;
};

// Lane geometry inside a 2048-column segment: block bs = lane>>3 (8 blocks),
// qs chunk k = lane&7 covering qs[16k, 16k+16) = sub-block pair j = k>>1,
// positions l0..l0+15 (l0 = 16*(k&1)); low nibbles are elements 64j+l0+i
// (sub-block 2j), high nibbles 64j+32+l0+i (sub-block 2j+1).
struct KLane {
    int bs, k, j, l0;
    __device__ KLane(int lane) : bs(lane >> 3), k(lane & 7), j((lane & 7) >> 1), l0(16 * (lane & 1)) {}
};

struct XSlice {
    float a[16], b[16];
    float sa, sb;
};

__device__ __forceinline__ void load_x_slice(const float *__restrict__ xblk, const KLane &L,
                                             bool active, XSlice &X)
{
    if (active) {
        const float4 *pa = reinterpret_cast<const float4 *>(xblk + 64 * L.j + L.l0);
        const float4 *pb = reinterpret_cast<const float4 *>(xblk + 64 * L.j + 32 + L.l0);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float4 va = pa[t], vb = pb[t];
            X.a[4 * t + 0] = va.x; X.a[4 * t + 1] = va.y; X.a[4 * t + 2] = va.z; X.a[4 * t + 3] = va.w;
            X.b[4 * t + 0] = vb.x; X.b[4 * t + 1] = vb.y; X.b[4 * t + 2] = vb.z; X.b[4 * t + 3] = vb.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) X.a[i] = X.b[i] = 0.0f;
    }
    float sa = 0.0f, sb = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) { sa += X.a[i]; sb += X.b[i]; }
    X.sa = sa;
    X.sb = sb;
}

// One lane's contribution for one row: header h, qs chunk q, (Q5_K) qh chunk.
template <int FMT>
__device__ __forceinline__ float kdot(const uint4 &h, const uint4 &q, const uint4 &qh,
                                      const KLane &L, const XSlice &X)
{
    float sa = 0.0f, sb = 0.0f;
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
    const uint32_t hw[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        uint32_t lo = qw[t] & 0x0f0f0f0fu;
        uint32_t hi = (qw[t] >> 4) & 0x0f0f0f0fu;
        if (FMT == kQ5_K) {
            lo |= ((hw[t] >> (2 * L.j)) & 0x01010101u) << 4;
            hi |= ((hw[t] >> (2 * L.j + 1)) & 0x01010101u) << 4;
        }
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            sa = fmaf(ubyte_f(lo, b), X.a[4 * t + b], sa);
            sb = fmaf(ubyte_f(hi, b), X.b[4 * t + b], sb);
        }
    }
    const float d = h2f(h.x & 0xffffu), dmin = h2f(h.x >> 16);
    uint32_t scA, mA, scB, mB;
    k_scale_min(h.y, h.z, h.w, 2 * L.j, scA, mA);
    k_scale_min(h.y, h.z, h.w, 2 * L.j + 1, scB, mB);
    float r = (d * (float)scA) * sa;
    r = fmaf(d * (float)scB, sb, r);
    r = fmaf(-(dmin * (float)mA), X.sa, r);
    r = fmaf(-(dmin * (float)mB), X.sb, r);
    return r;
}

// Plain GEMV (GATEUP == false) or fused gate/up + SwiGLU (GATEUP == true:
// W2 is the up weight, y[r] = silu(g[r]) * u[r]).
template <int FMT, int R, bool GATEUP>
__global__ __launch_bounds__(256) void k_gemv_kdirect(const uint8_t *__restrict__ W,
                                                      const uint8_t *__restrict__ W2,
                                                      const float *__restrict__ x,
                                                      float *__restrict__ y, int outer, int nblk)
{
    using F = KDirect<FMT>;
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
    if (row0 >= outer)
        return; // wave-uniform
    const KLane L(lane);
    const size_t row_bytes = (size_t)nblk * F::BYTES;
    constexpr int NW = GATEUP ? 2 : 1;
    float acc[NW][R];
#pragma unroll
    for (int m = 0; m < NW; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;

    const int nseg = (nblk + 7) >> 3;
    for (int seg = 0; seg < nseg; ++seg) {
        const int blk = seg * 8 + L.bs;
        const bool active = blk < nblk;
        uint4 hh[NW][R], qq[NW][R], qh[NW][R];
#pragma unroll
        for (int m = 0; m < NW; ++m) {
            const uint8_t *Wm = m == 0 ? W : W2;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int row = row0 + r;
                if (active && row < outer) {
                    const uint8_t *bp = Wm + (size_t)row * row_bytes + (size_t)blk * F::BYTES;
                    hh[m][r] = *reinterpret_cast<const uint4 *>(bp);
                    qq[m][r] = *reinterpret_cast<const uint4 *>(bp + F::QS + 16 * L.k);
                    if constexpr (FMT == kQ5_K)
                        qh[m][r] = *reinterpret_cast<const uint4 *>(bp + 16 + L.l0);
                    else
                        qh[m][r] = make_uint4(0, 0, 0, 0);
                } else {
                    hh[m][r] = qq[m][r] = qh[m][r] = make_uint4(0, 0, 0, 0);
                }
            }
        }
        XSlice X;
        load_x_slice(x + (size_t)blk * 256, L, active, X);
#pragma unroll
        for (int m = 0; m < NW; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r)
                acc[m][r] += kdot<FMT>(hh[m][r], qq[m][r], qh[m][r], L, X);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float g = wave_sum(acc[0][r]);
        float v = g;
        if constexpr (GATEUP) {
            const float u = wave_sum(acc[NW - 1][r]);
            // src/ModelCPU.jl:492-503: g / (1 + exp(-g)), then * u
            v = (g / (1.0f + expf(-g))) * u;
        }
        const int row = row0 + r;
        if (lane == 0 && row < outer)
            y[row] = v;
    }
}

// ------------------------------------------------------------------------
// Staged kernels (Q6_K, Q8_0): WG = 4 waves x R rows; each 2048-column
// segment of the WG's rows is copied to LDS with 128-bit loads first.
// ------------------------------------------------------------------------
template <int FMT>
struct KStaged;
template <>
struct KStaged<kQ6_K> {
    static constexpr int SEG_BLOCKS = 8, SEG_BYTES = 8 * 210, CHUNKS = SEG_BYTES / 16;
};
template <>
struct KStaged<kQ8_0> {
    static constexpr int SEG_BLOCKS = 64, SEG_BYTES = 64 * 34, CHUNKS = SEG_BYTES / 16;
};
static_assert(KStaged<kQ6_K>::SEG_BYTES % 16 == 0, "Q6_K segment must be 16-byte aligned");
static_assert(KStaged<kQ8_0>::SEG_BYTES % 16 == 0, "Q8_0 segment must be 16-byte aligned");

// Q6_K lane geometry: block bs = lane>>3; unit u = lane&7: half n = u>>2,
// positions l0 = 8*(u&3) .. +7.  Group g (0..3) of the unit holds the
// elements 128n + 32g + l0 + i (src/Dequant.jl:584-597): g=0 low nibble of
// ql[64n+l0+i], g=1 low nibble of ql[64n+32+l0+i], g=2/3 the high nibbles,
// with qh[32n+l0+i] bits 2g..2g+1 on top and scale sc[8n + 2g + (l0>>4)].
struct Q6Slice {
    float x[4][8];
    float s[4];
};

__device__ __forceinline__ void q6_load_x(const float *__restrict__ xblk, int n, int l0,
                                          bool active, Q6Slice &X)
{
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        if (active) {
            const float4 *p = reinterpret_cast<const float4 *>(xblk + 128 * n + 32 * g + l0);
            const float4 v0 = p[0], v1 = p[1];
            X.x[g][0] = v0.x; X.x[g][1] = v0.y; X.x[g][2] = v0.z; X.x[g][3] = v0.w;
            X.x[g][4] = v1.x; X.x[g][5] = v1.y; X.x[g][6] = v1.z; X.x[g][7] = v1.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) X.x[g][i] = 0.0f;
        }
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) s += X.x[g][i];
        X.s[g] = s;
    }
}

// `tile` is the 16-byte-aligned LDS array, `bo` the block's byte offset in it.
__device__ __forceinline__ float q6_dot(const uint8_t *tile, uint32_t bo, int n, int l0,
                                        const Q6Slice &X)
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
        r = fmaf(ds, acc[g] - 32.0f * X.s[g], r);
    }
    return r;
}

// Q8_0: lane = block within the 64-block segment, 32 weights.
__device__ __forceinline__ float q80_dot(const uint8_t *blk_lds, uint32_t off, const float *xr)
{
    const float d = h2f(lds_read_u16(blk_lds, off));
    const uint32_t o = off + 2;
    const uint32_t *p = reinterpret_cast<const uint32_t *>(blk_lds + (o & ~3u));
    const uint32_t sh = o & 3u;
    uint32_t w[9];
#pragma unroll
    for (int i = 0; i < 9; ++i) w[i] = p[i];
    float acc = 0.0f;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const uint32_t q = __builtin_amdgcn_alignbyte(w[t + 1], w[t], sh);
#pragma unroll
        for (int b = 0; b < 4; ++b)
            acc = fmaf(sbyte_f(q, b), xr[4 * t + b], acc);
    }
    return d * acc;
}

struct ArgmaxWS {
    unsigned long long key; // (ordered value << 32) | (0xffffffff - index)
    unsigned int count;     // workgroups finished
    unsigned int flags;     // bit0 NaN, bit1 +Inf, bit2 a value other than -Inf seen
};

__device__ __forceinline__ uint32_t ordered_bits(float v)
{
    if (v == 0.0f)
        v = 0.0f; // -0 == +0 for the strict `>` scan of src/CommonOps.jl:155-158
    const uint32_t b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Fold value v at index i into a (key, flags) pair: NaN and +Inf raise a
// flag and never win; ties keep the lower index.
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

// Workgroup-level result -> global workspace; the last workgroup writes the
// token and flags and returns the workspace to zero for the next call.
__device__ void argmax_commit(ArgmaxWS *ws, unsigned long long key, uint32_t flags,
                              int32_t *token, uint32_t *flags_out)
{
    // called by one thread per workgroup
    if (flags)
        atomicOr(&ws->flags, flags);
    if (key)
        atomicMax(&ws->key, key);
    __threadfence();
    const unsigned int done = atomicAdd(&ws->count, 1u);
    if (done == gridDim.x - 1) {
        __threadfence();
        const unsigned long long k = atomicAdd(&ws->key, 0ull);
        const uint32_t f = atomicOr(&ws->flags, 0u);
        *token = (int32_t)(0xffffffffu - (uint32_t)(k & 0xffffffffull));
        uint32_t out = 0;
        if (f & 1u) out |= 1u;
        if (f & 2u) out |= 2u;
        if (!(f & 4u)) out |= 4u; // every logit was -Inf: index 0 (CommonOps.jl:143-161)
        if (!(f & 4u)) *token = 0;
        *flags_out = out;
        atomicExch(&ws->key, 0ull);
        atomicExch(&ws->flags, 0u);
        atomicExch(&ws->count, 0u);
    }
}

template <int FMT, int R, bool ARGMAX>
__global__ __launch_bounds__(256) void k_gemv_staged(const uint8_t *__restrict__ W,
                                                     const float *__restrict__ x,
                                                     float *__restrict__ y, int outer, int nblk,
                                                     ArgmaxWS *ws, int32_t *token,
                                                     uint32_t *flags_out)
{
    using F = KStaged<FMT>;
    constexpr int ROWS = 4 * R;
    __shared__ __attribute__((aligned(16))) uint8_t tile[ROWS * F::SEG_BYTES + 16];
    __shared__ unsigned long long wkey[4];
    __shared__ uint32_t wflag[4];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wg_row0 = blockIdx.x * ROWS;
    const size_t row_bytes = (size_t)nblk * block_bytes(FMT);
    const int nseg = (nblk + F::SEG_BLOCKS - 1) / F::SEG_BLOCKS;

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    for (int seg = 0; seg < nseg; ++seg) {
        const int seg_blocks = min(F::SEG_BLOCKS, nblk - seg * F::SEG_BLOCKS);
        const int seg_chunks = (seg_blocks * block_bytes(FMT) + 15) / 16;
        // cooperative 128-bit copy of the WG's rows' segment into LDS
        for (int c = tid; c < ROWS * F::CHUNKS; c += 256) {
            const int rr = c / F::CHUNKS, cc = c - rr * F::CHUNKS;
            const int row = wg_row0 + rr;
            if (row < outer && cc < seg_chunks) {
                const uint8_t *src = W + (size_t)row * row_bytes +
                                     (size_t)seg * F::SEG_BYTES + 16 * (size_t)cc;
                *reinterpret_cast<uint4 *>(tile + rr * F::SEG_BYTES + 16 * cc) =
                    *reinterpret_cast<const uint4 *>(src);
            }
        }
        __syncthreads();
        const float *xs = x + (size_t)seg * 2048;
        if constexpr (FMT == kQ6_K) {
            const int bs = lane >> 3, n = (lane >> 2) & 1, l0 = 8 * (lane & 3);
            const bool active = bs < seg_blocks;
            Q6Slice X;
            q6_load_x(xs + 256 * bs, n, l0, active, X);
            if (active) {
#pragma unroll
                for (int r = 0; r < R; ++r)
                    acc[r] += q6_dot(tile, (wave * R + r) * F::SEG_BYTES + 210 * bs, n, l0, X);
            }
        } else {
            const bool active = lane < seg_blocks;
            float xr[32];
            if (active) {
                const float4 *p = reinterpret_cast<const float4 *>(xs + 32 * lane);
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const float4 v = p[t];
                    xr[4 * t] = v.x; xr[4 * t + 1] = v.y; xr[4 * t + 2] = v.z; xr[4 * t + 3] = v.w;
                }
#pragma unroll
                for (int r = 0; r < R; ++r)
                    acc[r] += q80_dot(tile + (wave * R + r) * F::SEG_BYTES, 34u * lane, xr);
            }
        }
        __syncthreads();
    }

    unsigned long long key = 0;
    uint32_t fl = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float v = wave_sum(acc[r]);
        const int row = wg_row0 + wave * R + r;
        if (row < outer) {
            if (y && lane == 0)
                y[row] = v;
            if (ARGMAX)
                argmax_fold(v, (uint32_t)row, key, fl);
        }
    }
    if constexpr (ARGMAX) {
        if (lane == 0) {
            wkey[wave] = key;
            wflag[wave] = fl;
        }
        __syncthreads();
        if (tid == 0) {
            unsigned long long k = wkey[0];
            uint32_t f = wflag[0];
#pragma unroll
            for (int w = 1; w < 4; ++w) {
                k = wkey[w] > k ? wkey[w] : k;
                f |= wflag[w];
            }
            argmax_commit(ws, k, f, token, flags_out);
        }
    }
}

// Standalone argmax over a logits vector (gpu_argmax!, FusedKernels.jl:271-311,
// with the _validate_logits checks of CommonOps.jl:142-163).
__global__ __launch_bounds__(256) void k_argmax(const float *__restrict__ v, int64_t n,
                                                ArgmaxWS *ws, int32_t *token, uint32_t *flags_out)
{
    __shared__ unsigned long long wkey[4];
    __shared__ uint32_t wflag[4];
    unsigned long long key = 0;
    uint32_t fl = 0;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        argmax_fold(v[i], (uint32_t)i, key, fl);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const unsigned long long ok = __shfl_xor(key, o, 64);
        key = ok > key ? ok : key;
        fl |= __shfl_xor(fl, o, 64);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        wkey[wave] = key;
        wflag[wave] = fl;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long k = wkey[0];
        uint32_t f = wflag[0];
        for (int w = 1; w < 4; ++w) {
            k = wkey[w] > k ? wkey[w] : k;
            f |= wflag[w];
        }
        argmax_commit(ws, k, f, token, flags_out);
    }
}

// ------------------------------------------------------------------------
// launchers
// ------------------------------------------------------------------------
static int g_rows_direct = 4; // rows per wave, direct kernels
static int g_rows_staged = 2; // rows per wave, staged kernels

void set_tuning(const char *name, int value)
{
    if (!__builtin_strcmp(name, "rows_direct")) g_rows_direct = value;
    if (!__builtin_strcmp(name, "rows_staged")) g_rows_staged = value;
}

template <int FMT, bool GATEUP>
static hipError_t launch_kdirect(const void *w, const void *w2, const float *x, float *y,
                                 int inner, int outer, hipStream_t s)
{
    const int nblk = inner / 256;
    const int R = g_rows_direct;
#define IHIP_KD(RR)                                                                          \
    case RR:                                                                                 \
        hipLaunchKernelGGL((k_gemv_kdirect<FMT, RR, GATEUP>),                                \
                           dim3((outer + 4 * RR - 1) / (4 * RR)), dim3(256), 0, s,            \
                           (const uint8_t *)w, (const uint8_t *)w2, x, y, outer, nblk);      \
        break;
    switch (R) {
        IHIP_KD(1)
        IHIP_KD(2)
        IHIP_KD(8)
    default:
        IHIP_KD(4)
    }
#undef IHIP_KD
    return hipGetLastError();
}

template <int FMT, bool ARGMAX>
static hipError_t launch_staged(const void *w, const float *x, float *y, int inner, int outer,
                                void *ws, int32_t *token, uint32_t *flags, hipStream_t s)
{
    const int nblk = inner / block_elems(FMT);
    const int R = g_rows_staged;
#define IHIP_KS(RR)                                                                          \
    case RR:                                                                                 \
        hipLaunchKernelGGL((k_gemv_staged<FMT, RR, ARGMAX>),                                 \
                           dim3((outer + 4 * RR - 1) / (4 * RR)), dim3(256), 0, s,            \
                           (const uint8_t *)w, x, y, outer, nblk, (ArgmaxWS *)ws, token,      \
                           flags);                                                           \
        break;
    switch (R) {
        IHIP_KS(1)
        IHIP_KS(4)
    default:
        IHIP_KS(2)
    }
#undef IHIP_KS
    return hipGetLastError();
}

hipError_t launch_gemv(int type, const void *w, const float *x, float *y, int inner, int outer,
                       hipStream_t s)
{
    switch (type) {
    case kQ4_K: return launch_kdirect<kQ4_K, false>(w, nullptr, x, y, inner, outer, s);
    case kQ5_K: return launch_kdirect<kQ5_K, false>(w, nullptr, x, y, inner, outer, s);
    case kQ6_K: return launch_staged<kQ6_K, false>(w, x, y, inner, outer, nullptr, nullptr, nullptr, s);
    case kQ8_0: return launch_staged<kQ8_0, false>(w, x, y, inner, outer, nullptr, nullptr, nullptr, s);
    default: return hipErrorInvalidValue;
    }
}

bool gate_up_fusable(int gate_type, int up_type)
{
    return gate_type == up_type && (gate_type == kQ4_K || gate_type == kQ5_K);
}

hipError_t launch_gate_up_swiglu(int type, const void *wg, const void *wu, const float *x,
                                 float *h, int hidden, int inter, hipStream_t s)
{
    switch (type) {
    case kQ4_K: return launch_kdirect<kQ4_K, true>(wg, wu, x, h, hidden, inter, s);
    case kQ5_K: return launch_kdirect<kQ5_K, true>(wg, wu, x, h, hidden, inter, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_lm_head_argmax(int type, const void *w, const float *x, float *logits,
                                 int32_t *token, uint32_t *flags, int hidden, int vocab,
                                 void *ws, hipStream_t s)
{
    switch (type) {
    case kQ6_K: return launch_staged<kQ6_K, true>(w, x, logits, hidden, vocab, ws, token, flags, s);
    case kQ8_0: return launch_staged<kQ8_0, true>(w, x, logits, hidden, vocab, ws, token, flags, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_argmax(const float *v, int64_t n, int32_t *token, uint32_t *flags, void *ws,
                         hipStream_t s)
{
    int64_t blocks = (n + 255) / 256;
    if (blocks > 1024) blocks = 1024;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(k_argmax, dim3((unsigned)blocks), dim3(256), 0, s, v, n, (ArgmaxWS *)ws,
                       token, flags);
    return hipGetLastError();
}

} // namespace ihip
