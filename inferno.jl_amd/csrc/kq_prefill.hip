// kq_prefill.hip -- batched prefill GEMM on gfx950 matrix cores:
//   Y[t, n] = sum_k W[n, k] * X[t, k],  W: N x K Q4_K,  X: T x K fp32.
//
// The reference has no GEMM here: src/ModelCPU.jl:1001-1017 (Inferno.jl)
// runs T independent GEMVs, so the semantics are the Q4_K GEMV applied row
// by row.  On MI355X the T tokens share every weight byte, which makes this
// a dense contraction: X is rounded once to fp16 (the matrix-core operand
// type; fp16 keeps the 1e-4*||w||*||x|| bound where bf16 does not) and
// v_mfma_f32_32x32x16_f16 accumulates in fp32.
//
// Tile: 64 tokens x 128 weight rows per workgroup of 4 waves (256 workgroups
// at 512 x 4096 x 4096); wave w owns weight rows [32w, 32w+32) of the tile
// and both 32-token halves.  The activations stream through a double-
// buffered, bank-swizzled LDS stage one Q4_K block column (256 k) ahead;
// each lane dequantizes the B operand it feeds the matrix core (one weight
// row, 8 k per 16-wide step) straight into registers from the block bytes,
// also loaded one block ahead, so the weights are dequantized exactly once
// per workgroup and never pass through LDS.  Workgroups are mapped so that
// those of one XCD (blockIdx % 8) share a contiguous band of W rows.
#include "kq_common.h"
#include "kq_launch.h"

namespace ihip {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int PF_BM = 64, PF_BN = 128; // workgroup tile: tokens x weight rows

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

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// One 64-token x 256-column stage of the fp16 activations in LDS: row m
// holds 32 chunks of 16 bytes, chunk c at slot c ^ (m & 15), so that the 16
// lanes of a 128-bit read (same chunk, consecutive rows) hit distinct banks.
constexpr int PF_ROW_BYTES = 512;
constexpr int PF_A_STAGE = 64 * PF_ROW_BYTES;   // 32 KB
constexpr int PF_B_STAGE = PF_BN * 144;          // 18 KB: one Q4_K block of 128 rows
constexpr int PF_THREADS = 512;                  // 8 waves

// Register double-buffering of one block column: each of the 512 threads
// loads 4 chunks (16 bytes) of the 64-token activation stage and up to 3 of
// the 128-row weight stage for block kb + 1 while block kb is reduced, then
// writes them to the other stage.
struct PfRegs {
    uint4 a0, a1, a2, a3, b0, b1, b2; // plain members: the registers must not become an array
};

__device__ __forceinline__ uint4 pf_load_a(const _Float16 *__restrict__ Xh, int m0, int T, int K,
                                           int kb, int q)
{
    const int rp = q >> 5, slot = q & 31; // stage row q/32, slot q%32
    const int c = slot ^ (rp & 15);       // the activation chunk that lives in this slot
    const int row = min(m0 + rp, T - 1);  // rows past T re-read row T-1
    return *reinterpret_cast<const uint4 *>(Xh + (size_t)row * K + (size_t)kb * 256 + 8 * c);
}

__device__ __forceinline__ uint4 pf_load_b(const uint8_t *__restrict__ W, int n0, int N,
                                           size_t row_bytes, int kb, int q)
{
    // chunk q of the 128 x 144-byte weight stage (q < 1152; callers clamp)
    const int row = q / 9, piece = q - 9 * (q / 9);
    return *reinterpret_cast<const uint4 *>(W + (size_t)min(n0 + row, N - 1) * row_bytes +
                                            (size_t)kb * 144 + 16 * piece);
}

__device__ __forceinline__ void pf_load(const _Float16 *__restrict__ Xh,
                                        const uint8_t *__restrict__ W, int m0, int n0, int T,
                                        int N, int K, size_t row_bytes, int kb, int tid, PfRegs &R)
{
    R.a0 = pf_load_a(Xh, m0, T, K, kb, tid);
    R.a1 = pf_load_a(Xh, m0, T, K, kb, tid + PF_THREADS);
    R.a2 = pf_load_a(Xh, m0, T, K, kb, tid + 2 * PF_THREADS);
    R.a3 = pf_load_a(Xh, m0, T, K, kb, tid + 3 * PF_THREADS);
    R.b0 = pf_load_b(W, n0, N, row_bytes, kb, tid);
    R.b1 = pf_load_b(W, n0, N, row_bytes, kb, tid + PF_THREADS);
    // the third round covers chunks 1024..1151: threads past it re-load chunk 1151
    R.b2 = pf_load_b(W, n0, N, row_bytes, kb, min(tid + 2 * PF_THREADS, PF_BN * 9 - 1));
}

__device__ __forceinline__ void pf_store(uint8_t *sa, uint8_t *sb, int tid, const PfRegs &R)
{
    *reinterpret_cast<uint4 *>(sa + 16 * tid) = R.a0;
    *reinterpret_cast<uint4 *>(sa + 16 * (tid + PF_THREADS)) = R.a1;
    *reinterpret_cast<uint4 *>(sa + 16 * (tid + 2 * PF_THREADS)) = R.a2;
    *reinterpret_cast<uint4 *>(sa + 16 * (tid + 3 * PF_THREADS)) = R.a3;
    *reinterpret_cast<uint4 *>(sb + 16 * tid) = R.b0;
    *reinterpret_cast<uint4 *>(sb + 16 * (tid + PF_THREADS)) = R.b1;
    if (tid + 2 * PF_THREADS < PF_BN * 9)
        *reinterpret_cast<uint4 *>(sb + 16 * (tid + 2 * PF_THREADS)) = R.b2;
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

// Y[t, n] = sum_k W[n, k] Xh[t, k].  Workgroup tile: 64 tokens x 128 weight
// rows, 8 waves: wave w owns weight rows n0 + 32 (w & 3) .. +32, both
// 32-token halves, and half (w >> 2) of every block column (sub-block pairs
// 2 (w >> 2) and 2 (w >> 2) + 1); the two halves' sums meet in LDS at the
// end.  Both operands stream through double-buffered LDS stages filled by
// direct-to-LDS loads one block column ahead; each lane dequantizes the B
// operand it feeds the matrix core (one weight row, 8 k per 16-wide step)
// from the stage into registers, so the weights are dequantized exactly once
// per workgroup.  v_mfma_f32_32x32x16_f16, fp32 accumulation.
// Reduce sub-block pair j of block column kb from one stage into the
// accumulators: this lane's B operands are weight rows `blk0` and `blk1`
// (rows li and li + 32 of the wave's 64), 8 k of every 16-wide step.
__device__ __forceinline__ void pf_pair(const uint8_t *sa, const uint8_t *blk0,
                                        const uint8_t *blk1, int j, int h, int li,
                                        float16v (&acc)[2][2])
{
    half2v dsA[2], dmA[2], dsB[2], dmB[2];
    uint2 q0[2], q1[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const uint8_t *blk = u ? blk1 : blk0;
        const uint4 hd = *reinterpret_cast<const uint4 *>(blk);
        const float d = h2f(hd.x & 0xffffu), dmin = h2f(hd.x >> 16);
        float scA, mA, scB, mB;
        k_scale_min_pair(hd.y, hd.z, hd.w, j, scA, mA, scB, mB);
        const _Float16 a = (_Float16)(d * scA), ma = (_Float16)(-(dmin * mA));
        const _Float16 bb = (_Float16)(d * scB), mb = (_Float16)(-(dmin * mB));
        dsA[u] = half2v{a, a};
        dmA[u] = half2v{ma, ma};
        dsB[u] = half2v{bb, bb};
        dmB[u] = half2v{mb, mb};
        q0[u] = *reinterpret_cast<const uint2 *>(blk + 16 + 32 * j + 8 * h);
        q1[u] = *reinterpret_cast<const uint2 *>(blk + 16 + 32 * j + 16 + 8 * h);
    }
    // four 16-wide K steps: k = 64j + 16s + 8h + (0..7)
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int c = 8 * j + 2 * s + h; // 16-byte chunk of the stage row
        half8 a[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int m = 32 * t + li;
            a[t] = *reinterpret_cast<const half8 *>(sa + m * PF_ROW_BYTES + 16 * (c ^ (m & 15)));
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const half8 b = pf_dequant8((s & 1) ? q1[u] : q0[u], s >= 2, s >= 2 ? dsB[u] : dsA[u],
                                        s >= 2 ? dmB[u] : dmA[u]);
#pragma unroll
            for (int t = 0; t < 2; ++t)
                acc[u][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[t], b, acc[u][t], 0, 0, 0);
        }
    }
}

// Y[t, n] = sum_k W[n, k] Xh[t, k].  Workgroup tile: 64 tokens x 128 weight
// rows, 8 waves: wave w owns weight rows n0 + 64 (w & 1) .. +64 (two 32-row
// MFMA tiles), both 32-token halves, and sub-block pair w >> 1 of every block
// column; the four pairs' sums meet in LDS at the end.  Both operands stream
// through double-buffered LDS stages filled by register double-buffering
// (block kb + 1 is loaded into registers while block kb is reduced); each
// lane dequantizes the B operands it feeds the matrix core (8 k of one
// weight row per 16-wide step) from the stage into registers, so the weights
// are dequantized exactly once per workgroup.  v_mfma_f32_32x32x16_f16, fp32
// accumulation.
__global__ __launch_bounds__(PF_THREADS) void k_prefill_q4k(const uint8_t *__restrict__ W,
                                                            const _Float16 *__restrict__ Xh,
                                                            float *__restrict__ Y, int T, int K,
                                                            int N, int mtiles, int ntiles)
{
    __shared__ __attribute__((aligned(16))) uint8_t As0[PF_A_STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t As1[PF_A_STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t Bs0[PF_B_STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t Bs1[PF_B_STAGE];

    // XCD-aware tile order: consecutive workgroups of one XCD walk the M
    // tiles of one N band, so the band's weight bytes are shared in its L2.
    const int bid = blockIdx.x;
    const int nxcd = 8;
    const int per_xcd = (mtiles * ntiles + nxcd - 1) / nxcd;
    const int lin = (bid % nxcd) * per_xcd + bid / nxcd;
    if (lin >= mtiles * ntiles)
        return; // whole workgroup
    const int mt = lin % mtiles, nt = lin / mtiles;
    const int m0 = mt * PF_BM, n0 = nt * PF_BN;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rh = wave & 1, j = wave >> 1;
    const int h = lane >> 5, li = lane & 31;
    const int nblk = K / 256;
    const size_t row_bytes = (size_t)nblk * 144;
    const int brow = 64 * rh + li; // this lane's first weight row inside the tile

    float16v acc[2][2];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[u][t][r] = 0.0f;

    PfRegs R;
    pf_load(Xh, W, m0, n0, T, N, K, row_bytes, 0, tid, R);
    pf_store(As0, Bs0, tid, R);
    __syncthreads();

    // two block columns per trip: stage 0 then stage 1
    for (int kb = 0; kb < nblk; kb += 2) {
        const bool more1 = kb + 1 < nblk, more2 = kb + 2 < nblk; // workgroup-uniform
        if (more1)
            pf_load(Xh, W, m0, n0, T, N, K, row_bytes, kb + 1, tid, R);
        pf_pair(As0, Bs0 + brow * 144, Bs0 + (brow + 32) * 144, j, h, li, acc);
        if (!more1)
            break;
        asm volatile("" ::: "memory"); // the stores below stay after the reduction
        pf_store(As1, Bs1, tid, R);
        __syncthreads(); // stage 1 holds block kb + 1; stage 0 is free
        if (more2)
            pf_load(Xh, W, m0, n0, T, N, K, row_bytes, kb + 2, tid, R);
        pf_pair(As1, Bs1 + brow * 144, Bs1 + (brow + 32) * 144, j, h, li, acc);
        if (!more2)
            break;
        asm volatile("" ::: "memory");
        pf_store(As0, Bs0, tid, R);
        __syncthreads(); // stage 0 holds block kb + 2; stage 1 is free
    }
    __syncthreads(); // every wave is done with the stages
    // pairs 1..3 hand their sums to pair 0 through LDS (the stages are free):
    // 2 x 2 x 16 floats per lane = 16 KB per (pair, row half); pairs 1 and 2
    // use the two activation stages (32 KB each), pair 3 the two weight
    // stages (18 KB each)
    auto slot_of = [&](int pj, int hh) -> float * {
        if (pj == 1)
            return reinterpret_cast<float *>(As0) + hh * 4096;
        if (pj == 2)
            return reinterpret_cast<float *>(As1) + hh * 4096;
        return reinterpret_cast<float *>(hh ? Bs1 : Bs0);
    };
    if (j != 0) {
        float *dst = slot_of(j, rh);
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    dst[((u * 2 + t) * 16 + r) * 64 + lane] = acc[u][t][r];
    }
    __syncthreads();
    if (j != 0)
        return;
    // store: D[m][n], lane l, reg r: n = l % 32, m = 8*(r/4) + 4*(l/32) + r%4
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int nn = n0 + brow + 32 * u;
        if (nn >= N)
            continue;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
                const int idx = ((u * 2 + t) * 16 + r) * 64 + lane;
                const float v = acc[u][t][r] + slot_of(1, rh)[idx] + slot_of(2, rh)[idx] +
                                slot_of(3, rh)[idx];
                if (m < T)
                    Y[(size_t)m * N + nn] = v;
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
    hipLaunchKernelGGL(k_prefill_q4k, dim3(per_xcd * 8), dim3(PF_THREADS), 0, s, (const uint8_t *)w,
                       (const _Float16 *)xh, Y, T, inner, outer, mtiles, ntiles);
    return hipGetLastError();
}

} // namespace ihip
