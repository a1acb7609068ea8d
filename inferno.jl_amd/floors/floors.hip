// floors.hip -- measurement kernels for bench.py (not part of the product ABI).
//
// They give the two floors a single decode-GEMV launch cannot beat on this
// device, measured the same way as the GEMV itself (HIP graph, back to back,
// weight copies rotated through HBM):
//   ifl_empty: a launch that does nothing, at a given grid and block size --
//              the per-launch cost of dispatch, wave launch and completion;
//   ifl_read:  a launch that reads n bytes with fully coalesced 16-byte loads
//              (each workgroup one contiguous slice, every load issued before
//              the first is used) and discards them -- the time to stream the
//              weight bytes alone.
// Built into inferno.jl_amd/lib/libinferno_floors.so; only bench.py loads it.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

__global__ void k_floor_empty() {}

// Every thread loads LPT 16-byte vectors of its workgroup's slice (a stride of
// the workgroup size apart, so each load instruction of a wave covers 1 KB of
// consecutive bytes) and folds them; the store is taken only when the fold
// equals `key` (never, for the keys bench.py passes), so the loads are live.
template <int LPT>
__global__ __launch_bounds__(1024) void k_floor_read(const uint4 *__restrict__ w, uint64_t n16,
                                                     uint32_t key, uint32_t *out)
{
    const uint64_t per_wg = (n16 + gridDim.x - 1) / gridDim.x;
    const uint64_t base = (uint64_t)blockIdx.x * per_wg;
    uint4 v[LPT];
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
        const uint64_t k = base + (uint64_t)i * blockDim.x + threadIdx.x;
        v[i] = (k < base + per_wg && k < n16) ? w[k] : make_uint4(0, 0, 0, 0);
    }
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < LPT; ++i)
        acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    if (acc == key)
        out[0] = acc;
}

} // namespace

extern "C" {

int ifl_empty(int grid, int block, void *stream)
{
    hipLaunchKernelGGL(k_floor_empty, dim3(grid), dim3(block), 0, (hipStream_t)stream);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// n: bytes to read (a multiple of 16); the grid's workgroups of `block`
// threads (64..1024) split them into contiguous slices of at most 32 loads
// per thread.
int ifl_read(const void *w, uint64_t n, uint32_t key, uint32_t *out, int grid, int block, void *stream)
{
    if (n % 16 || grid < 1 || block < 64 || block > 1024 || block % 64)
        return -1;
    const uint64_t n16 = n / 16;
    const uint64_t per_thread = (n16 + (uint64_t)grid * block - 1) / ((uint64_t)grid * block);
    const hipStream_t s = (hipStream_t)stream;
#define IFL_R(L)                                                                                   \
    if (per_thread <= L) {                                                                         \
        hipLaunchKernelGGL(k_floor_read<L>, dim3(grid), dim3(block), 0, s, (const uint4 *)w, n16, key, out); \
        return hipGetLastError() == hipSuccess ? 0 : -1;                                           \
    }
    IFL_R(1) IFL_R(2) IFL_R(4) IFL_R(5) IFL_R(8) IFL_R(9) IFL_R(16) IFL_R(32)
#undef IFL_R
    return -1;
}

} // extern "C"
