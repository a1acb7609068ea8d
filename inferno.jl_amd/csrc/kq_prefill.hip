// kq_prefill.hip -- batched prefill GEMM on gfx950 matrix cores:
//   Y[t, n] = sum_k W[n, k] * X[t, k],  W: N x K Q4_K,  X: T x K fp32.
//
// The reference has no GEMM here: src/ModelCPU.jl:1001-1017 (Inferno.jl)
// runs T independent GEMVs, so the semantics are the Q4_K GEMV applied row
// by row.  On MI355X the T tokens share every weight byte, which makes this
// a dense contraction: X is rounded once to fp16 (the matrix-core operand
// type; fp16 keeps the 1e-4*||w||*||x|| bound where bf16 does not), each
// K-step dequantizes one Q4_K super-block column of the W tile into LDS as
// fp16, and v_mfma_f32_32x32x16_f16 accumulates in fp32.
//
// Tile: BM = 64 tokens x BN = 128 weight rows per workgroup of 4 waves; wave
// w owns rows [32w, 32w+32) of the BN tile and both 32-token halves of BM.
// K-step = 256 (one super-block).  Workgroups are mapped so that the 32
// workgroups of one XCD (blockIdx % 8) share a contiguous band of W rows.
#include "kq_common.h"
#include "kq_launch.h"

namespace ihip {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int PF_BM = 64, PF_BN = 128, PF_BK = 256;
constexpr int PF_LDA = PF_BK + 8; // halves per LDS row (16-byte pad against bank conflicts)

__global__ __launch_bounds__(256) void k_x_to_f16(const float *__restrict__ X,
                                                  _Float16 *__restrict__ Xh, int64_t n)
{
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i + 3 < n) {
        const float4 v = *reinterpret_cast<const float4 *>(X + i);
        Xh[i] = (_Float16)v.x;
        Xh[i + 1] = (_Float16)v.y;
        Xh[i + 2] = (_Float16)v.z;
        Xh[i + 3] = (_Float16)v.w;
    } else {
        for (int64_t j = i; j < n; ++j)
            Xh[j] = (_Float16)X[j];
    }
}

__global__ __launch_bounds__(256) void k_prefill_q4k(const uint8_t *__restrict__ W,
                                                     const _Float16 *__restrict__ Xh,
                                                     float *__restrict__ Y, int T, int K, int N,
                                                     int mtiles, int ntiles)
{
    __shared__ __attribute__((aligned(16))) _Float16 As[PF_BM * PF_LDA];
    __shared__ __attribute__((aligned(16))) _Float16 Bs[PF_BN * PF_LDA];

    // XCD-aware tile order: consecutive workgroups of one XCD walk the
    // M tiles of one N band.
    const int bid = blockIdx.x;
    const int nxcd = 8;
    const int per_xcd = (mtiles * ntiles + nxcd - 1) / nxcd;
    const int lin = (bid % nxcd) * per_xcd + bid / nxcd;
    if (lin >= mtiles * ntiles)
        return;
    const int mt = lin % mtiles, nt = lin / mtiles;
    const int m0 = mt * PF_BM, n0 = nt * PF_BN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nblk = K / 256;
    const size_t row_bytes = (size_t)nblk * 144;

    float16v acc[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[i][j] = 0.0f;

    for (int kb = 0; kb < nblk; ++kb) {
        // ---- A tile: 64 x 256 halves, 16-byte pieces (2048 of them)
#pragma unroll
        for (int it = 0; it < 8; ++it) {
            const int p = tid + 256 * it; // piece index
            const int r = p >> 5, c = (p & 31) * 8;
            const int t = m0 + r;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (t < T)
                v = *reinterpret_cast<const uint4 *>(Xh + (size_t)t * K + (size_t)kb * 256 + c);
            *reinterpret_cast<uint4 *>(As + r * PF_LDA + c) = v;
        }
        // ---- B tile: 128 rows x one Q4_K block -> fp16; 4 (row, chunk) per thread
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int u = tid + 256 * it;
            const int r = u >> 3, k = u & 7, j = k >> 1, l0 = 16 * (k & 1);
            const int n = n0 + r;
            uint4 h = make_uint4(0, 0, 0, 0), q = make_uint4(0, 0, 0, 0);
            if (n < N) {
                const uint8_t *bp = W + (size_t)n * row_bytes + (size_t)kb * 144;
                h = *reinterpret_cast<const uint4 *>(bp);
                q = *reinterpret_cast<const uint4 *>(bp + 16 + 16 * k);
            }
            const float d = h2f(h.x & 0xffffu), dmin = h2f(h.x >> 16);
            uint32_t scA, mA, scB, mB;
            k_scale_min(h.y, h.z, h.w, 2 * j, scA, mA);
            k_scale_min(h.y, h.z, h.w, 2 * j + 1, scB, mB);
            const float dA = d * (float)scA, minA = dmin * (float)mA;
            const float dB = d * (float)scB, minB = dmin * (float)mB;
            const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
            half8 va[2], vb[2];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t lo = qw[t] & 0x0f0f0f0fu, hi = (qw[t] >> 4) & 0x0f0f0f0fu;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    va[t >> 1][4 * (t & 1) + b] = (_Float16)(dA * ubyte_f(lo, b) - minA);
                    vb[t >> 1][4 * (t & 1) + b] = (_Float16)(dB * ubyte_f(hi, b) - minB);
                }
            }
            _Float16 *row = Bs + r * PF_LDA;
            *reinterpret_cast<half8 *>(row + 64 * j + l0) = va[0];
            *reinterpret_cast<half8 *>(row + 64 * j + l0 + 8) = va[1];
            *reinterpret_cast<half8 *>(row + 64 * j + 32 + l0) = vb[0];
            *reinterpret_cast<half8 *>(row + 64 * j + 32 + l0 + 8) = vb[1];
        }
        __syncthreads();
        // ---- 16 MFMA K-steps of 16
        const int li = lane & 31, kh = 8 * (lane >> 5);
        const _Float16 *bp = Bs + (32 * wave + li) * PF_LDA + kh;
        const _Float16 *ap0 = As + li * PF_LDA + kh;
        const _Float16 *ap1 = As + (32 + li) * PF_LDA + kh;
#pragma unroll 4
        for (int ks = 0; ks < PF_BK; ks += 16) {
            const half8 b = *reinterpret_cast<const half8 *>(bp + ks);
            const half8 a0 = *reinterpret_cast<const half8 *>(ap0 + ks);
            const half8 a1 = *reinterpret_cast<const half8 *>(ap1 + ks);
            acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b, acc[0], 0, 0, 0);
            acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b, acc[1], 0, 0, 0);
        }
        __syncthreads();
    }
    // ---- store: D[m][n], lane l, reg j: n = l % 32, m = 8*(j/4) + 4*(l/32) + j%4
    const int n = n0 + 32 * wave + (lane & 31);
    if (n < N) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int m = m0 + 32 * i + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
                if (m < T)
                    Y[(size_t)m * N + n] = acc[i][j];
            }
    }
}

void set_prefill_tuning(const char *, int) {}

hipError_t launch_prefill_q4k(const void *w, const float *X, void *xh, float *Y, int T,
                              int inner, int outer, hipStream_t s)
{
    const int64_t n = (int64_t)T * inner;
    hipLaunchKernelGGL(k_x_to_f16, dim3((unsigned)((n / 4 + 255) / 256 + 1)), dim3(256), 0, s, X,
                       (_Float16 *)xh, n);
    const int mtiles = (T + PF_BM - 1) / PF_BM, ntiles = (outer + PF_BN - 1) / PF_BN;
    const int per_xcd = (mtiles * ntiles + 7) / 8;
    hipLaunchKernelGGL(k_prefill_q4k, dim3(per_xcd * 8), dim3(256), 0, s, (const uint8_t *)w,
                       (const _Float16 *)xh, Y, T, inner, outer, mtiles, ntiles);
    return hipGetLastError();
}

} // namespace ihip
