// api.hip -- the C ABI (include/inferno_hip.h): argument checks, the device
// weight cache, host<->device staging for the host-pointer entry points,
// and dispatch to the gfx950 kernels.
//
// Host-pointer entry points mirror the reference's synchronous C functions
// (src/kernels/quant_kernels.c:602-697 behind src/QuantizedKernels.jl:84-148
// of Inferno.jl).  Unlike the reference they report failures through a
// status code and ihip_last_error() instead of returning void.
#include "inferno_hip.h"
#include "kq_common.h"
#include "kq_launch.h"
#include "kq_sdig_plan.h"

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

using namespace ihip;

namespace {

thread_local std::string t_err;

int fail(int code, const char *fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    t_err = buf;
    return code;
}

#define HIPCHK(expr)                                                                          \
    do {                                                                                      \
        hipError_t e_ = (expr);                                                               \
        if (e_ != hipSuccess)                                                                 \
            return fail(IHIP_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(e_));          \
    } while (0)

#define RET_IF(expr)                                                                          \
    do {                                                                                      \
        int rc_ = (expr);                                                                     \
        if (rc_ != IHIP_OK)                                                                   \
            return rc_;                                                                       \
    } while (0)

struct Weight {
    void *dev = nullptr;
    size_t bytes = 0;
    int type = 0, inner = 0, outer = 0;
    const void *host = nullptr;
    uint64_t fp = 0; // content fingerprint of a weight cached by host address
};

// Sampled content fingerprint of a host buffer: its size and 64 windows of 16
// bytes at evenly spaced offsets (the first and the last 16 bytes included),
// mixed by a 64-bit multiply / xor-shift hash.  About 1 KB is read whatever
// the size, so it is checked on every host-pointer call.
constexpr int kFpWindows = 64;
constexpr int kMaxGroup = 64; // weights in one group upload

uint64_t fp_mix(uint64_t h, uint64_t v)
{
    h ^= v + 0x9e3779b97f4a7c15ull + (h << 6) + (h >> 2);
    h *= 0xff51afd7ed558ccdull;
    return h ^ (h >> 33);
}

uint64_t fingerprint(const void *p, size_t n)
{
    const uint8_t *b = (const uint8_t *)p;
    uint64_t h = fp_mix(0x243f6a8885a308d3ull, (uint64_t)n);
    if (n == 0)
        return h;
    const size_t span = n > 16 ? n - 16 : 0;
    for (int i = 0; i < kFpWindows; ++i) {
        const size_t off = span * (size_t)i / (kFpWindows - 1);
        uint64_t w[2] = {0, 0};
        memcpy(w, b + off, n < 16 ? n : 16);
        h = fp_mix(fp_mix(h, w[0]), w[1]);
    }
    return h;
}

struct DevBuf {
    void *p = nullptr;
    size_t cap = 0;
    void *hp = nullptr; // pinned host staging of the same buffer (hipHostMalloc, mapped)
    void *hdp = nullptr; // the staging's device-side address (hipHostGetDevicePointer)
    size_t hcap = 0;
};

// Host copies that wait for the library stream: y, h, logits ... come back
// through a buffer's pinned staging and are copied to the caller's memory
// once the stream has drained (finish_locked).
struct PendingOut {
    void *dst;
    const void *src;
    size_t bytes;
};

struct Ctx {
    std::recursive_mutex mu;
    bool ready = false;
    int device = -1;
    hipStream_t stream = nullptr;
    std::unordered_map<uint64_t, Weight> by_handle;
    std::unordered_map<const void *, uint64_t> by_host;
    uint64_t next_handle = 1;
    DevBuf x, y, h, t, src, nrm; // staging and scratch, grown on demand
    std::vector<PendingOut> pending; // host copies after the next stream drain
    void *argmax_ws = nullptr; // IHIP_ARGMAX_WS_BYTES, left zeroed by the kernels
    int32_t *d_token = nullptr;
    uint32_t *d_flags = nullptr;
};

Ctx &ctx()
{
    static Ctx c;
    return c;
}

// Scratch of the allocation-free lm_head entry point: the argmax partials
// (one 16-byte partial per workgroup, at most kArgMaxParts of them).  Every
// device the library runs on holds its own copy for the life of the process;
// the kernels write every partial they read, so nothing needs clearing.  In
// host code `scratch` only names the symbol: kernels get the device address
// resolved by hipGetSymbolAddress, kept per device in scratch_dev.
static __device__ __align__(256) uint8_t scratch[IHIP_ARGMAX_WS_BYTES];
constexpr int kMaxDevices = 64;
void *scratch_dev[kMaxDevices]; // device address of `scratch`, per device (nullptr: not resolved yet)

// The current device's copy of `scratch` (resolved on the first call on that
// device, with it current; the library mutex is held).
int scratch_for_current_device(void **p)
{
    int dev = -1;
    HIPCHK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices)
        return fail(IHIP_ERR_INVALID, "device %d is beyond the %d the library tracks", dev, kMaxDevices);
    if (!scratch_dev[dev]) {
        void *q = nullptr;
        HIPCHK(hipGetSymbolAddress(&q, HIP_SYMBOL(scratch)));
        if (!q)
            return fail(IHIP_ERR_HIP, "no device address for the scratch array");
        scratch_dev[dev] = q;
    }
    *p = scratch_dev[dev];
    return IHIP_OK;
}

bool disabled()
{
    const char *e = getenv("IHIP_DISABLE");
    return e && e[0] && strcmp(e, "0") != 0;
}

bool known_type(int t) { return block_elems(t) != 0; }

size_t weight_bytes(int type, int inner, int outer)
{
    return (size_t)outer * (size_t)(inner / block_elems(type)) * (size_t)block_bytes(type);
}

int check_shape(int type, int inner, int outer)
{
    if (!known_type(type))
        return fail(IHIP_ERR_INVALID, "unknown ggml type %d", type);
    if (inner <= 0 || outer <= 0)
        return fail(IHIP_ERR_INVALID, "inner=%d outer=%d must be positive", inner, outer);
    if (inner % block_elems(type))
        return fail(IHIP_ERR_INVALID, "inner=%d is not a multiple of %d for type %d", inner,
                    block_elems(type), type);
    return IHIP_OK;
}

bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// Whether [a, a + an) and [b, b + bn) share a byte.  A kernel that reads one
// buffer in every workgroup while it writes the other races on any overlap.
bool overlap(const void *a, size_t an, const void *b, size_t bn)
{
    const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    return an && bn && x < y + bn && y < x + an;
}

// Grow a host-path staging buffer.  Only the host-pointer entry points use
// these buffers, on the library stream; work still queued there (an earlier
// call that failed half-way) finishes before the old buffer is freed.
int ensure(DevBuf &b, size_t need)
{
    if (b.cap >= need)
        return IHIP_OK;
    if (b.p) {
        HIPCHK(hipStreamSynchronize(ctx().stream));
        HIPCHK(hipFree(b.p));
    }
    b.p = nullptr;
    b.cap = 0;
    const size_t cap = need < 4096 ? 4096 : need;
    HIPCHK(hipMalloc(&b.p, cap));
    b.cap = cap;
    return IHIP_OK;
}

int init_locked(int device)
{
    Ctx &c = ctx();
    if (disabled())
        return fail(IHIP_ERR_DISABLED, "IHIP_DISABLE is set");
    if (c.ready) {
        if (device == c.device)
            return IHIP_OK;
        return fail(IHIP_ERR_INVALID, "already initialised on device %d", c.device);
    }
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || n <= device)
        return fail(IHIP_ERR_NO_DEVICE, "no HIP device %d (count %d)", device, n);
    hipDeviceProp_t prop;
    HIPCHK(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(IHIP_ERR_NO_DEVICE, "device %d is %s; this library is built for gfx950",
                    device, prop.gcnArchName);
    HIPCHK(hipSetDevice(device));
    void *sp = nullptr;
    RET_IF(scratch_for_current_device(&sp)); // set-up of the allocation-free entry point
    HIPCHK(hipStreamCreateWithFlags(&c.stream, hipStreamNonBlocking));
    HIPCHK(hipMalloc(&c.argmax_ws, IHIP_ARGMAX_WS_BYTES + 64));
    HIPCHK(hipMemset(c.argmax_ws, 0, IHIP_ARGMAX_WS_BYTES + 64));
    c.d_token = (int32_t *)((char *)c.argmax_ws + IHIP_ARGMAX_WS_BYTES);
    c.d_flags = (uint32_t *)((char *)c.argmax_ws + IHIP_ARGMAX_WS_BYTES + 32);
    c.device = device;
    c.ready = true;
    return IHIP_OK;
}

int ready_locked()
{
    Ctx &c = ctx();
    c.pending.clear(); // a host call that failed half-way leaves no copies behind
    if (disabled())
        return fail(IHIP_ERR_DISABLED, "IHIP_DISABLE is set");
    if (!c.ready)
        return init_locked(0);
    HIPCHK(hipSetDevice(c.device));
    return IHIP_OK;
}

int release_handle_locked(uint64_t h)
{
    Ctx &c = ctx();
    auto it = c.by_handle.find(h);
    if (it == c.by_handle.end())
        return fail(IHIP_ERR_INVALID, "unknown weight handle %llu", (unsigned long long)h);
    if (it->second.host) {
        auto hi = c.by_host.find(it->second.host);
        if (hi != c.by_host.end() && hi->second == h)
            c.by_host.erase(hi);
    }
    HIPCHK(hipFree(it->second.dev));
    c.by_handle.erase(it);
    return IHIP_OK;
}

int upload_locked(const void *host, size_t bytes, int type, int inner, int outer,
                  bool cache_by_host, uint64_t *handle)
{
    Ctx &c = ctx();
    Weight w;
    w.bytes = bytes;
    w.type = type;
    w.inner = inner;
    w.outer = outer;
    w.host = cache_by_host ? host : nullptr;
    w.fp = cache_by_host ? fingerprint(host, bytes) : 0;
    HIPCHK(hipMalloc(&w.dev, bytes));
    hipError_t e = hipMemcpy(w.dev, host, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(w.dev);
        return fail(IHIP_ERR_HIP, "weight upload failed: %s", hipGetErrorString(e));
    }
    const uint64_t h = c.next_handle++;
    c.by_handle[h] = w;
    if (cache_by_host)
        c.by_host[host] = h;
    *handle = h;
    return IHIP_OK;
}

// Several weights of one type and row length uploaded back to back as one
// registered weight of sum(outers) rows (member i's bytes at its rows'
// offset): one GEMV over it computes every member's outputs.  bytes[i], when
// given, is what member i's source holds.
int upload_group_locked(const void *const *hosts, const size_t *bytes, const int *outers, int n,
                        int type, int inner, uint64_t *handle)
{
    Ctx &c = ctx();
    if (!hosts || !outers || !handle)
        return fail(IHIP_ERR_INVALID, "null pointer");
    if (n <= 0 || n > kMaxGroup)
        return fail(IHIP_ERR_INVALID, "a group holds 1 to %d weights, not %d", kMaxGroup, n);
    int64_t total = 0;
    for (int i = 0; i < n; ++i) {
        if (!hosts[i])
            return fail(IHIP_ERR_INVALID, "null pointer (member %d)", i);
        RET_IF(check_shape(type, inner, outers[i]));
        if (bytes && bytes[i] < weight_bytes(type, inner, outers[i]))
            return fail(IHIP_ERR_INVALID, "member %d: %zu bytes < %zu needed for %dx%d type %d", i,
                        bytes[i], weight_bytes(type, inner, outers[i]), outers[i], inner, type);
        total += outers[i];
    }
    if (total > INT32_MAX)
        return fail(IHIP_ERR_INVALID, "a group's rows must stay below 2^31");
    Weight w;
    w.bytes = weight_bytes(type, inner, (int)total);
    w.type = type;
    w.inner = inner;
    w.outer = (int)total;
    w.host = nullptr;
    w.fp = 0;
    HIPCHK(hipMalloc(&w.dev, w.bytes));
    size_t off = 0;
    for (int i = 0; i < n; ++i) {
        const size_t b = weight_bytes(type, inner, outers[i]);
        const hipError_t e = hipMemcpy(static_cast<uint8_t *>(w.dev) + off, hosts[i], b,
                                       hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            (void)hipFree(w.dev);
            return fail(IHIP_ERR_HIP, "weight upload failed: %s", hipGetErrorString(e));
        }
        off += b;
    }
    const uint64_t h = c.next_handle++;
    c.by_handle[h] = w;
    *handle = h;
    return IHIP_OK;
}

// Device copy of a host weight, uploaded on first sight and cached by its
// host address (weights are immutable after load in the reference).  The
// entry is reused only while the shape, type and sampled content fingerprint
// still match: a buffer freed and its address reused for other bytes, or a
// weight rewritten in place, is uploaded again.
int resolve_locked(const void *host, int type, int inner, int outer, const void **dev)
{
    Ctx &c = ctx();
    const size_t bytes = weight_bytes(type, inner, outer);
    auto hi = c.by_host.find(host);
    if (hi != c.by_host.end()) {
        const Weight &w = c.by_handle[hi->second];
        if (w.bytes == bytes && w.type == type && w.inner == inner && w.outer == outer &&
            w.fp == fingerprint(host, bytes)) {
            *dev = w.dev;
            return IHIP_OK;
        }
        // same address, new shape or new bytes: drop the stale copy (after any
        // queued host-path work that reads it) and upload again
        HIPCHK(hipStreamSynchronize(c.stream));
        RET_IF(release_handle_locked(hi->second));
    }
    uint64_t h = 0;
    RET_IF(upload_locked(host, bytes, type, inner, outer, true, &h));
    *dev = c.by_handle[h].dev;
    return IHIP_OK;
}

// Fast kernels need 16-byte aligned weights and x.  Rows of any whole number
// of blocks qualify: the streamed Q6_K / Q8_0 / IQ4_NL kernel copies rows
// that are not 16-byte multiples from the unit below each segment (which may
// read up to 14 bytes past the weight's last byte, inside its 16-byte unit).
bool fast_ok(int, const void *w, const float *x, int)
{
    return al16(w) && al16(x);
}

// resid != nullptr: out = epi_apply(resid, W x, epi) row by row: the residual
// add (resid may be out) or the SwiGLU against the gate row in out.
int gemv_dev_locked(int type, const void *w, const float *x, float *out, int inner, int outer,
                    hipStream_t s, const float *resid = nullptr, int epi = kEpiAdd)
{
    RET_IF(check_shape(type, inner, outer));
    if (!w || !x || !out)
        return fail(IHIP_ERR_INVALID, "null pointer");
    // every workgroup reads all of x while rows of out are written
    if (overlap(x, 4 * (size_t)inner, out, 4 * (size_t)outer))
        return fail(IHIP_ERR_INVALID, "x overlaps out");
    hipError_t e = fast_ok(type, w, x, inner)
                       ? launch_gemv(type, w, x, out, inner, outer, s, resid, epi)
                       : launch_gemv_generic(type, w, x, out, inner, outer, s, resid, epi);
    if (e != hipSuccess)
        return fail(IHIP_ERR_HIP, "gemv launch failed: %s", hipGetErrorString(e));
    return IHIP_OK;
}

bool gate_up_fused(int gt, const void *wg, int ut, const void *wu, const float *x, int hidden,
                   const float *norm_w)
{
    return gate_up_fusable(gt, ut) && fast_ok(gt, wg, x, hidden) && al16(wu) &&
           (!norm_w || al16(norm_w));
}

// h = silu(Wg n) .* (Wu n) with n = x, or n = rmsnorm(x) .* norm_w when norm_w
// is given.  A matching Q4_K/Q5_K pair runs as one fused pass (the norm folded
// in).  Any other pair writes g into h, and the up GEMV's epilogue turns h
// into silu(h) * u in place; a norm then goes first into xn (hidden floats
// of caller scratch).  No library buffer is touched.
int gate_up_dev_locked(int gt, const void *wg, int ut, const void *wu, const float *x, float *h,
                       int hidden, int inter, hipStream_t s, const float *norm_w = nullptr,
                       float eps = 0.0f, float *xn = nullptr)
{
    RET_IF(check_shape(gt, hidden, inter));
    RET_IF(check_shape(ut, hidden, inter));
    if (!wg || !wu || !x || !h)
        return fail(IHIP_ERR_INVALID, "null pointer");
    if (overlap(x, 4 * (size_t)hidden, h, 4 * (size_t)inter))
        return fail(IHIP_ERR_INVALID, "x overlaps h");
    if (xn && (overlap(x, 4 * (size_t)hidden, xn, 4 * (size_t)hidden) ||
               overlap(h, 4 * (size_t)inter, xn, 4 * (size_t)hidden)))
        return fail(IHIP_ERR_INVALID, "the norm scratch overlaps x or h");
    if (gate_up_fused(gt, wg, ut, wu, x, hidden, norm_w)) {
        hipError_t e = launch_gate_up_swiglu(gt, wg, wu, x, h, hidden, inter, s, norm_w, eps);
        if (e != hipSuccess)
            return fail(IHIP_ERR_HIP, "gate/up launch failed: %s", hipGetErrorString(e));
        return IHIP_OK;
    }
    if (norm_w) {
        if (!xn)
            return fail(IHIP_ERR_INVALID, "the norm of an unfused gate/up pair needs scratch");
        hipError_t e = launch_rmsnorm(x, norm_w, eps, xn, hidden, s);
        if (e != hipSuccess)
            return fail(IHIP_ERR_HIP, "rmsnorm launch failed: %s", hipGetErrorString(e));
        x = xn;
    }
    RET_IF(gemv_dev_locked(gt, wg, x, h, hidden, inter, s));
    return gemv_dev_locked(ut, wu, x, h, hidden, inter, s, h, kEpiSwiglu);
}

// Whether the lm_head runs with the argmax fused into its GEMV (no logits
// buffer needed).
bool lm_head_fused(int type, const void *w, const float *x, int hidden, int vocab)
{
    return (type == kQ6_K || type == kQ8_0) && fast_ok(type, w, x, hidden) && lm_head_fusable(type, hidden);
}

int lm_head_parts(int type, const void *w, const float *x, int hidden, int vocab)
{
    return lm_head_argmax_parts(type, hidden, vocab, lm_head_fused(type, w, x, hidden, vocab));
}

int lm_head_dev_locked(int type, const void *w, const float *x, float *logits, int32_t *token,
                       uint32_t *flags, int hidden, int vocab, void *ws, hipStream_t s)
{
    RET_IF(check_shape(type, hidden, vocab));
    if (!w || !x || !token || !flags || !ws)
        return fail(IHIP_ERR_INVALID, "null pointer");
    if (logits && overlap(x, 4 * (size_t)hidden, logits, 4 * (size_t)vocab))
        return fail(IHIP_ERR_INVALID, "x overlaps logits");
    if (lm_head_fused(type, w, x, hidden, vocab)) {
        hipError_t e = launch_lm_head_argmax(type, w, x, logits, token, flags, hidden, vocab, ws, s);
        if (e != hipSuccess)
            return fail(IHIP_ERR_HIP, "lm_head launch failed: %s", hipGetErrorString(e));
        return IHIP_OK;
    }
    if (!logits)
        return fail(IHIP_ERR_INVALID,
                    "this lm_head (type %d, %d x %d) runs the GEMV and the argmax separately: "
                    "pass a logits buffer (ihip_lm_head_fused tells)", type, vocab, hidden);
    RET_IF(gemv_dev_locked(type, w, x, logits, hidden, vocab, s));
    hipError_t e = launch_argmax(logits, vocab, token, flags, ws, s);
    if (e != hipSuccess)
        return fail(IHIP_ERR_HIP, "argmax launch failed: %s", hipGetErrorString(e));
    return IHIP_OK;
}

// Transfers up to this size go through a buffer's pinned host staging (a
// host memcpy plus a DMA copy: a pageable copy of a few KB costs several
// times more); larger ones are copied from the caller's memory directly.
constexpr size_t kStageMax = 1u << 20;

int finish_locked();

int ensure_pinned(DevBuf &b, size_t need)
{
    if (b.hcap >= need)
        return IHIP_OK;
    if (b.hp) {
        // outputs already staged (possibly in this buffer) are delivered first
        RET_IF(finish_locked());
        HIPCHK(hipHostFree(b.hp));
        b.hp = nullptr;
        b.hcap = 0;
    }
    size_t cap = 4096;
    while (cap < need)
        cap *= 2;
    HIPCHK(hipHostMalloc(&b.hp, cap, hipHostMallocMapped));
    b.hcap = cap;
    b.hdp = nullptr;
    void *d = nullptr;
    if (hipHostGetDevicePointer(&d, b.hp, 0) == hipSuccess)
        b.hdp = d; // else: outputs come back through a DMA copy
    else
        (void)hipGetLastError();
    return IHIP_OK;
}

int copy_in(DevBuf &b, const void *host, size_t bytes)
{
    RET_IF(ensure(b, bytes));
    if (bytes <= kStageMax) {
        // the staging is reused: an earlier copy from it has completed, because
        // every host entry point drains the stream before it returns
        RET_IF(ensure_pinned(b, bytes));
        memcpy(b.hp, host, bytes);
        HIPCHK(hipMemcpyAsync(b.p, b.hp, bytes, hipMemcpyHostToDevice, ctx().stream));
    } else {
        HIPCHK(hipMemcpyAsync(b.p, host, bytes, hipMemcpyHostToDevice, ctx().stream));
    }
    return IHIP_OK;
}

// bytes of b (device) -> host, complete after finish_locked().  `off` is a
// byte offset into b.
int copy_out(DevBuf &b, void *host, size_t bytes, size_t off = 0)
{
    const uint8_t *dev = (const uint8_t *)b.p + off;
    if (bytes <= kStageMax) {
        RET_IF(ensure_pinned(b, off + bytes));
        uint8_t *stage = (uint8_t *)b.hp + off;
        HIPCHK(hipMemcpyAsync(stage, dev, bytes, hipMemcpyDeviceToHost, ctx().stream));
        ctx().pending.push_back({host, stage, bytes});
    } else {
        HIPCHK(hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, ctx().stream));
    }
    return IHIP_OK;
}

// Drain the library stream, then deliver the staged outputs.
int finish_locked()
{
    Ctx &c = ctx();
    const hipError_t e = hipStreamSynchronize(c.stream);
    if (e != hipSuccess) {
        c.pending.clear();
        return fail(IHIP_ERR_HIP, "%s", hipGetErrorString(e));
    }
    for (const PendingOut &o : c.pending)
        memcpy(o.dst, o.src, o.bytes);
    c.pending.clear();
    return IHIP_OK;
}

int host_gemv(int type, const uint8_t *w, const float *x, float *out, int inner, int outer)
{
    Ctx &c = ctx();
    std::lock_guard<std::recursive_mutex> lk(c.mu);
    RET_IF(ready_locked());
    RET_IF(check_shape(type, inner, outer));
    if (!w || !x || !out)
        return fail(IHIP_ERR_INVALID, "null pointer");
    const void *dw = nullptr;
    RET_IF(resolve_locked(w, type, inner, outer, &dw));
    RET_IF(copy_in(c.x, x, sizeof(float) * (size_t)inner));
    const size_t ybytes = sizeof(float) * (size_t)outer;
    if (ybytes <= kStageMax) {
        // the kernel stores y straight into the mapped pinned staging: no
        // device-to-host copy behind it
        RET_IF(ensure_pinned(c.y, ybytes));
        if (c.y.hdp) {
            RET_IF(gemv_dev_locked(type, dw, (const float *)c.x.p, (float *)c.y.hdp, inner, outer,
                                   c.stream));
            c.pending.push_back({out, c.y.hp, ybytes});
            return finish_locked();
        }
    }
    RET_IF(ensure(c.y, ybytes));
    RET_IF(gemv_dev_locked(type, dw, (const float *)c.x.p, (float *)c.y.p, inner, outer, c.stream));
    RET_IF(copy_out(c.y, out, ybytes));
    return finish_locked();
}

bool q8k_type(int t) { return t == kQ4_K || t == kQ5_K || t == kQ6_K; }

size_t q8k_bytes(int64_t k) { return (size_t)(k / 256) * IHIP_Q8_K_BYTES; }

// The int8-activation entry points: x re-quantized to Q8_K, integer dots
// (the reference C numerics, quant_kernels.c:166-194, 204-521, 602-650).
int host_gemv_q8k(int type, const uint8_t *w, const float *x, float *out, void *q8_buf,
                  int inner, int outer)
{
    Ctx &c = ctx();
    std::lock_guard<std::recursive_mutex> lk(c.mu);
    RET_IF(ready_locked());
    RET_IF(check_shape(type, inner, outer));
    if (!w || !x || !out)
        return fail(IHIP_ERR_INVALID, "null pointer");
    const void *dw = nullptr;
    RET_IF(resolve_locked(w, type, inner, outer, &dw));
    RET_IF(copy_in(c.x, x, sizeof(float) * (size_t)inner));
    RET_IF(ensure(c.t, q8k_bytes(inner)));
    RET_IF(ensure(c.y, sizeof(float) * (size_t)outer));
    // one launch quantizes x and runs the GEMV where the kernel takes the shape
    hipError_t e = launch_gemv_q8k_x(type, dw, (const float *)c.x.p, q8_buf ? c.t.p : nullptr, c.t.p,
                                     (float *)c.y.p, inner, outer, c.stream);
    if (e != hipSuccess)
        return fail(IHIP_ERR_HIP, "q8k gemv launch failed: %s", hipGetErrorString(e));
    RET_IF(copy_out(c.y, out, sizeof(float) * (size_t)outer));
    if (q8_buf)
        RET_IF(copy_out(c.t, q8_buf, q8k_bytes(inner)));
    return finish_locked();
}

int host_vec_dot_q8k(int type, const void *x, const void *y, int nb, float *s)
{
    Ctx &c = ctx();
    std::lock_guard<std::recursive_mutex> lk(c.mu);
    RET_IF(ready_locked());
    if (!x || !y || !s)
        return fail(IHIP_ERR_INVALID, "null pointer");
    if (nb <= 0)
        return fail(IHIP_ERR_INVALID, "nb=%d must be positive", nb);
    // a row is not a registered weight: staged, not cached
    RET_IF(copy_in(c.src, x, (size_t)nb * block_bytes(type)));
    RET_IF(copy_in(c.t, y, (size_t)nb * IHIP_Q8_K_BYTES));
    RET_IF(ensure(c.y, sizeof(float)));
    hipError_t e = launch_gemv_q8k(type, c.src.p, c.t.p, (float *)c.y.p, nb * 256, 1, c.stream);
    if (e != hipSuccess)
        return fail(IHIP_ERR_HIP, "q8k dot launch failed: %s", hipGetErrorString(e));
    RET_IF(copy_out(c.y, s, sizeof(float)));
    return finish_locked();
}

} // namespace

// Hooks for gguf.hip (same library): report an error through
// ihip_last_error, and upload GGML blocks into the registry.
int ihip_fail_msg(int code, const char *msg) { return fail(code, "%s", msg); }

int ihip_register_device_copy(const void *host, size_t bytes, int type, int inner, int outer,
                              uint64_t *handle)
{
    Ctx &c = ctx();
    std::lock_guard<std::recursive_mutex> lk(c.mu);
    RET_IF(ready_locked());
    RET_IF(check_shape(type, inner, outer));
    if (bytes < weight_bytes(type, inner, outer))
        return fail(IHIP_ERR_INVALID, "%zu bytes < %zu needed for %dx%d type %d", bytes,
                    weight_bytes(type, inner, outer), outer, inner, type);
    return upload_locked(host, weight_bytes(type, inner, outer), type, inner, outer, false, handle);
}

int ihip_register_device_group(const void *const *hosts, const size_t *bytes, const int *outers,
                               int n, int type, int inner, uint64_t *handle)
{
    std::lock_guard<std::recursive_mutex> lk(ctx().mu);
    RET_IF(ready_locked());
    return upload_group_locked(hosts, bytes, outers, n, type, inner, handle);
}

extern "C" {

const char *ihip_last_error(void) { return t_err.c_str(); }

int ihip_version(void) { return 10000; }

int ihip_available(void)
{
    if (disabled())
        return 0;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
        return 0;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, 0) != hipSuccess)
        return 0;
    return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

int ihip_init(int device)
{
    std::lock_guard<std::recursive_mutex> lk(ctx().mu);
    return init_locked(device);
}

int ihip_shutdown(void)
{
    Ctx &c = ctx();
    std::lock_guard<std::recursive_mutex> lk(c.mu);
    if (!c.ready)
        return IHIP_OK;
    (void)hipSetDevice(c.device);
    (void)hipStreamSynchronize(c.stream);
    for (auto &kv : c.by_handle)
        (void)hipFree(kv.second.dev);
    c.by_handle.clear();
    c.by_host.clear();
    for (DevBuf *b : {&c.x, &c.y, &c.h, &c.t, &c.src, &c.nrm}) {
        if (b->p)
            (void)hipFree(b->p);
        if (b->hp)
            (void)hipHostFree(b->hp);
        b->p = nullptr;
        b->cap = 0;
        b->hp = nullptr;
        b->hdp = nullptr;
        b->hcap = 0;
    }
    c.pending.clear();
    (void)hipFree(c.argmax_ws);
    c.argmax_ws = nullptr;
    (void)hipStreamDestroy(c.stream);
    c.stream = nullptr;
    c.ready = false;
    c.device = -1;
    return IHIP_OK;
}

// inter + hidden for every pair: a Q4_K/Q5_K pair whose pointers rule the
// fused pass out (alignment) takes the unfused path, which needs room for the
// normed input after h.
size_t ihip_ffn_block_scratch_floats(int, int, int hidden, int inter)
{
    if (hidden <= 0 || inter <= 0)
        return 0;
    return (size_t)inter + (size_t)hidden;
}

int ihip_lm_head_fused(int ggml_type, const void *w, const float *x, int hidden, int vocab)
{
    if (!known_type(ggml_type) || hidden <= 0 || vocab <= 0 || hidden % block_elems(ggml_type))
        return 0;
    return lm_head_fused(ggml_type, w, x, hidden, vocab) ? 1 : 0;
}

int ihip_weight_register(const void *host, size_t bytes, int ggml_type, int inner, int outer,
                         uint64_t *handle)
{
    Ctx &c = ctx();
    std::lock_guard<std::recursive_mutex> lk(c.mu);
    RET_IF(ready_locked());
    RET_IF(check_shape(ggml_type, inner, outer));
    if (!host || !handle)
        return fail(IHIP_ERR_INVALID, "null pointer");
    if (bytes < weight_bytes(ggml_type, inner, outer))
        return fail(IHIP_ERR_INVALID, "%zu bytes < %zu needed for %dx%d type %d", bytes,
                    weight_bytes(ggml_type, inner, outer), outer, inner, ggml_type);
    return upload_locked(host, weight_bytes(ggml_type, inner, outer), ggml_type, inner, outer,
                         false, handle);
}

int ihip_weight_register_group(const void *const *hosts, const int *outers, int n, int ggml_type,
                               int inner, uint64_t *handle)
{
    std::lock_guard<std::recursive_mutex> lk(ctx().mu);
    RET_IF(ready_locked());
    return upload_group_locked(hosts, nullptr, outers, n, ggml_type, inner, handle);
}

size_t ihip_weight_bytes(int ggml_type, int inner, int outer)
{
    if (!known_type(ggml_type) || inner <= 0 || outer < 0 || inner % block_elems(ggml_type))
        return 0;
    return weight_bytes(ggml_type, inner, outer);
}

int ihip_weight_release(uint64_t handle)
{
    std::lock_guard<std::recursive_mutex> lk(ctx().mu);
    return release_handle_locked(handle);
}

int ihip_weight_forget(const void *host)
{
    Ctx &c = ctx();
    std::lock_guard<std::recursive_mutex> lk(c.mu);
    auto it = c.by_host.find(host);
    if (it == c.by_host.end())
        return IHIP_OK;
    return release_handle_locked(it->second);
}

int ihip_weight_fingerprint(const void *host, size_t bytes, uint64_t *fp)
{
    if (!fp || (!host && bytes))
        return fail(IHIP_ERR_INVALID, "null pointer");
    *fp = fingerprint(host, bytes);
    return IHIP_OK;
}

int ihip_weight_device_ptr(uint64_t handle, const void **dev)
{
    Ctx &c = ctx();
    std::lock_guard<std::recursive_mutex> lk(c.mu);
    auto it = c.by_handle.find(handle);
    if (it == c.by_handle.end() || !dev)
        return fail(IHIP_ERR_INVALID, "unknown weight handle %llu", (unsigned long long)handle);
    *dev = it->second.dev;
    return IHIP_OK;
}

int ihip_q4_k_gemv(const uint8_t *weight, const float *x, float *out, void *q8_buf_unused,
                   int inner_dim, int outer_dim)
{
    (void)q8_buf_unused;
    return host_gemv(kQ4_K, weight, x, out, inner_dim, outer_dim);
}

int ihip_q5_k_gemv(const uint8_t *weight, const float *x, float *out, void *q8_buf_unused,
                   int inner_dim, int outer_dim)
{
    (void)q8_buf_unused;
    return host_gemv(kQ5_K, weight, x, out, inner_dim, outer_dim);
}

int ihip_q6_k_gemv(const uint8_t *weight, const float *x, float *out, void *q8_buf_unused,
                   int inner_dim, int outer_dim)
{
    (void)q8_buf_unused;
    return host_gemv(kQ6_K, weight, x, out, inner_dim, outer_dim);
}

int ihip_q8_0_gemv(const uint8_t *weight, const float *x, float *out, int inner_dim,
                   int outer_dim)
{
    return host_gemv(kQ8_0, weight, x, out, inner_dim, outer_dim);
}

int ihip_iq4_nl_gemv(const uint8_t *weight, const float *x, float *out, int inner_dim,
                     int outer_dim)
{
    return host_gemv(kIQ4_NL, weight, x, out, inner_dim, outer_dim);
}

int ihip_quantize_row_q8_k(const float *x, void *y, int64_t k)
{
    Ctx &c = ctx();
    std::lock_guard<std::recursive_mutex> lk(c.mu);
    RET_IF(ready_locked());
    if (!x || !y)
        return fail(IHIP_ERR_INVALID, "null pointer");
    if (k <= 0 || k % 256)
        return fail(IHIP_ERR_INVALID, "k=%lld is not a positive multiple of 256", (long long)k);
    RET_IF(copy_in(c.x, x, sizeof(float) * (size_t)k));
    RET_IF(ensure(c.t, q8k_bytes(k)));
    hipError_t e = launch_quantize_q8k((const float *)c.x.p, c.t.p, k, c.stream);
    if (e != hipSuccess)
        return fail(IHIP_ERR_HIP, "quantize launch failed: %s", hipGetErrorString(e));
    RET_IF(copy_out(c.t, y, q8k_bytes(k)));
    return finish_locked();
}

int ihip_vec_dot_q4_k_q8_k(const void *x, const void *y, int nb, float *s)
{
    return host_vec_dot_q8k(kQ4_K, x, y, nb, s);
}

int ihip_vec_dot_q5_k_q8_k(const void *x, const void *y, int nb, float *s)
{
    return host_vec_dot_q8k(kQ5_K, x, y, nb, s);
}

int ihip_vec_dot_q6_k_q8_k(const void *x, const void *y, int nb, float *s)
{
    return host_vec_dot_q8k(kQ6_K, x, y, nb, s);
}

int ihip_q4_k_gemv_q8k(const uint8_t *weight, const float *x, float *out, void *q8_buf,
                       int inner_dim, int outer_dim)
{
    return host_gemv_q8k(kQ4_K, weight, x, out, q8_buf, inner_dim, outer_dim);
}

int ihip_q5_k_gemv_q8k(const uint8_t *weight, const float *x, float *out, void *q8_buf,
                       int inner_dim, int outer_dim)
{
    return host_gemv_q8k(kQ5_K, weight, x, out, q8_buf, inner_dim, outer_dim);
}

int ihip_q6_k_gemv_q8k(const uint8_t *weight, const float *x, float *out, void *q8_buf,
                       int inner_dim, int outer_dim)
{
    return host_gemv_q8k(kQ6_K, weight, x, out, q8_buf, inner_dim, outer_dim);
}

int ihip_dequantize(int ggml_type, const uint8_t *src, float *dst, int64_t n)
{
    Ctx &c = ctx();
    std::lock_guard<std::recursive_mutex> lk(c.mu);
    RET_IF(ready_locked());
    if (!known_type(ggml_type))
        return fail(IHIP_ERR_INVALID, "unknown ggml type %d", ggml_type);
    if (n < 0 || n % block_elems(ggml_type))
        return fail(IHIP_ERR_INVALID, "n=%lld is not a multiple of %d", (long long)n,
                    block_elems(ggml_type));
    if (n == 0)
        return IHIP_OK;
    if (!src || !dst)
        return fail(IHIP_ERR_INVALID, "null pointer");
    const size_t in_bytes = (size_t)(n / block_elems(ggml_type)) * block_bytes(ggml_type);
    RET_IF(copy_in(c.src, src, in_bytes));
    RET_IF(ensure(c.y, sizeof(float) * (size_t)n));
    hipError_t e = launch_dequant(ggml_type, c.src.p, (float *)c.y.p, n, true, c.stream);
    if (e != hipSuccess)
        return fail(IHIP_ERR_HIP, "dequant launch failed: %s", hipGetErrorString(e));
    RET_IF(copy_out(c.y, dst, sizeof(float) * (size_t)n));
    return finish_locked();
}

int ihip_ffn_swiglu(int gate_type, const uint8_t *wg, int up_type, const uint8_t *wu,
                    int down_type, const uint8_t *wd, const float *x, float *h, float *y,
                    int hidden, int inter)
{
    Ctx &c = ctx();
    std::lock_guard<std::recursive_mutex> lk(c.mu);
    RET_IF(ready_locked());
    RET_IF(check_shape(gate_type, hidden, inter));
    RET_IF(check_shape(up_type, hidden, inter));
    RET_IF(check_shape(down_type, inter, hidden));
    if (!wg || !wu || !wd || !x || !y)
        return fail(IHIP_ERR_INVALID, "null pointer");
    const void *dg, *du, *dd;
    RET_IF(resolve_locked(wg, gate_type, hidden, inter, &dg));
    RET_IF(resolve_locked(wu, up_type, hidden, inter, &du));
    RET_IF(resolve_locked(wd, down_type, inter, hidden, &dd));
    RET_IF(copy_in(c.x, x, sizeof(float) * (size_t)hidden));
    RET_IF(ensure(c.h, sizeof(float) * (size_t)inter));
    RET_IF(ensure(c.y, sizeof(float) * (size_t)hidden));
    RET_IF(gate_up_dev_locked(gate_type, dg, up_type, du, (const float *)c.x.p, (float *)c.h.p,
                              hidden, inter, c.stream));
    RET_IF(gemv_dev_locked(down_type, dd, (const float *)c.h.p, (float *)c.y.p, inter, hidden,
                           c.stream));
    if (h)
        RET_IF(copy_out(c.h, h, sizeof(float) * (size_t)inter));
    RET_IF(copy_out(c.y, y, sizeof(float) * (size_t)hidden));
    return finish_locked();
}

int ihip_ffn_block(int gate_type, const uint8_t *wg, int up_type, const uint8_t *wu,
                   int down_type, const uint8_t *wd, const float *norm_w, float eps, float *x,
                   int hidden, int inter)
{
    Ctx &c = ctx();
    std::lock_guard<std::recursive_mutex> lk(c.mu);
    RET_IF(ready_locked());
    RET_IF(check_shape(gate_type, hidden, inter));
    RET_IF(check_shape(up_type, hidden, inter));
    RET_IF(check_shape(down_type, inter, hidden));
    if (!wg || !wu || !wd || !norm_w || !x)
        return fail(IHIP_ERR_INVALID, "null pointer");
    const void *dg, *du, *dd;
    RET_IF(resolve_locked(wg, gate_type, hidden, inter, &dg));
    RET_IF(resolve_locked(wu, up_type, hidden, inter, &du));
    RET_IF(resolve_locked(wd, down_type, inter, hidden, &dd));
    RET_IF(copy_in(c.x, x, sizeof(float) * (size_t)hidden));
    RET_IF(copy_in(c.src, norm_w, sizeof(float) * (size_t)hidden));
    RET_IF(ensure(c.h, sizeof(float) * (size_t)inter));
    RET_IF(ensure(c.nrm, sizeof(float) * (size_t)hidden));
    RET_IF(gate_up_dev_locked(gate_type, dg, up_type, du, (const float *)c.x.p, (float *)c.h.p,
                              hidden, inter, c.stream, (const float *)c.src.p, eps,
                              (float *)c.nrm.p));
    RET_IF(gemv_dev_locked(down_type, dd, (const float *)c.h.p, (float *)c.x.p, inter, hidden,
                           c.stream, (const float *)c.x.p));
    RET_IF(copy_out(c.x, x, sizeof(float) * (size_t)hidden));
    return finish_locked();
}

int ihip_lm_head_argmax(int ggml_type, const uint8_t *w, const float *x, float *logits,
                        int32_t *token, int hidden, int vocab)
{
    Ctx &c = ctx();
    std::lock_guard<std::recursive_mutex> lk(c.mu);
    RET_IF(ready_locked());
    RET_IF(check_shape(ggml_type, hidden, vocab));
    if (!w || !x || !token)
        return fail(IHIP_ERR_INVALID, "null pointer");
    const void *dw;
    RET_IF(resolve_locked(w, ggml_type, hidden, vocab, &dw));
    RET_IF(copy_in(c.x, x, sizeof(float) * (size_t)hidden));
    // logits on the device: wanted by the caller, or needed because the
    // argmax runs as a second kernel over them (not fused into the GEMV)
    float *dlog = nullptr;
    if (logits || !lm_head_fused(ggml_type, dw, (const float *)c.x.p, hidden, vocab)) {
        RET_IF(ensure(c.y, sizeof(float) * (size_t)vocab));
        dlog = (float *)c.y.p;
    }
    RET_IF(lm_head_dev_locked(ggml_type, dw, (const float *)c.x.p, dlog, c.d_token, c.d_flags,
                              hidden, vocab, c.argmax_ws, c.stream));
    int32_t tok = 0;
    uint32_t fl = 0;
    HIPCHK(hipMemcpyAsync(&tok, c.d_token, 4, hipMemcpyDeviceToHost, c.stream));
    HIPCHK(hipMemcpyAsync(&fl, c.d_flags, 4, hipMemcpyDeviceToHost, c.stream));
    if (logits) {
        if (dlog == (float *)c.y.p)
            RET_IF(copy_out(c.y, logits, sizeof(float) * (size_t)vocab));
        else
            HIPCHK(hipMemcpyAsync(logits, dlog, sizeof(float) * (size_t)vocab, hipMemcpyDeviceToHost,
                                  c.stream));
    }
    RET_IF(finish_locked());
    if (fl & IHIP_FLAG_NAN)
        return fail(IHIP_ERR_NONFINITE, "logits must not contain NaN");
    if (fl & IHIP_FLAG_POSINF)
        return fail(IHIP_ERR_NONFINITE, "logits must not contain +Inf");
    *token = tok;
    return IHIP_OK;
}

int ihip_prefill_q4_k(const uint8_t *w, const float *X, float *Y, int T, int inner, int outer)
{
    Ctx &c = ctx();
    std::lock_guard<std::recursive_mutex> lk(c.mu);
    RET_IF(ready_locked());
    RET_IF(check_shape(kQ4_K, inner, outer));
    if (T <= 0)
        return fail(IHIP_ERR_INVALID, "T=%d must be positive", T);
    if (!prefill_fits(T, inner, outer))
        return fail(IHIP_ERR_INVALID, "prefill operands must stay below 4 GiB (T*inner*2 and W bytes) and T*outer below 2^31");
    if (!w || !X || !Y)
        return fail(IHIP_ERR_INVALID, "null pointer");
    const void *dw;
    RET_IF(resolve_locked(w, kQ4_K, inner, outer, &dw));
    RET_IF(copy_in(c.x, X, sizeof(float) * (size_t)T * inner));
    RET_IF(ensure(c.h, prefill_scratch_bytes(T, inner)));
    RET_IF(ensure(c.y, sizeof(float) * (size_t)T * outer));
    hipError_t e = launch_prefill_q4k(dw, (const float *)c.x.p, c.h.p, (float *)c.y.p, T, inner,
                                      outer, c.stream);
    if (e != hipSuccess)
        return fail(IHIP_ERR_HIP, "prefill launch failed: %s", hipGetErrorString(e));
    RET_IF(copy_out(c.y, Y, sizeof(float) * (size_t)T * outer));
    return finish_locked();
}

// ---- device-pointer entry points ----------------------------------------

int ihip_gemv_dev(int ggml_type, const void *w, const float *x, float *out, int inner, int outer,
                  ihip_stream stream)
{
    std::lock_guard<std::recursive_mutex> lk(ctx().mu);
    if (disabled())
        return fail(IHIP_ERR_DISABLED, "IHIP_DISABLE is set");
    return gemv_dev_locked(ggml_type, w, x, out, inner, outer, (hipStream_t)stream);
}

int ihip_gemv_add_dev(int ggml_type, const void *w, const float *x, const float *resid, float *out,
                      int inner, int outer, ihip_stream stream)
{
    std::lock_guard<std::recursive_mutex> lk(ctx().mu);
    if (disabled())
        return fail(IHIP_ERR_DISABLED, "IHIP_DISABLE is set");
    if (!resid)
        return fail(IHIP_ERR_INVALID, "null pointer");
    // row r reads resid[r] and writes out[r]: in place is fine, a shifted overlap races
    // (x against out is checked with every GEMV)
    if (out && outer > 0 && resid != out && overlap(resid, 4 * (size_t)outer, out, 4 * (size_t)outer))
        return fail(IHIP_ERR_INVALID, "resid overlaps out without being out");
    return gemv_dev_locked(ggml_type, w, x, out, inner, outer, (hipStream_t)stream, resid, kEpiAdd);
}

int ihip_gemv_norm_dev(int ggml_type, const void *w, const float *norm_w, float eps, const float *x,
                       float *xn, float *out, int inner, int outer, ihip_stream stream)
{
    std::lock_guard<std::recursive_mutex> lk(ctx().mu);
    if (disabled())
        return fail(IHIP_ERR_DISABLED, "IHIP_DISABLE is set");
    RET_IF(check_shape(ggml_type, inner, outer));
    if (!w || !norm_w || !x || !out)
        return fail(IHIP_ERR_INVALID, "null pointer");
    if (overlap(x, 4 * (size_t)inner, out, 4 * (size_t)outer))
        return fail(IHIP_ERR_INVALID, "x overlaps out");
    if (gemv_norm_fusable(ggml_type, inner, outer) && fast_ok(ggml_type, w, x, inner) && al16(norm_w)) {
        hipError_t e = launch_gemv_norm(ggml_type, w, x, norm_w, eps, out, inner, outer, (hipStream_t)stream);
        if (e != hipSuccess)
            return fail(IHIP_ERR_HIP, "gemv launch failed: %s", hipGetErrorString(e));
        return IHIP_OK;
    }
    // the norm first, into the caller's scratch, then the plain GEMV
    if (!xn)
        return fail(IHIP_ERR_INVALID, "this GEMV (type %d, %d x %d) cannot fold the norm: pass xn",
                    ggml_type, outer, inner);
    if (overlap(xn, 4 * (size_t)inner, out, 4 * (size_t)outer))
        return fail(IHIP_ERR_INVALID, "xn overlaps out");
    hipError_t e = launch_rmsnorm(x, norm_w, eps, xn, inner, (hipStream_t)stream);
    if (e != hipSuccess)
        return fail(IHIP_ERR_HIP, "rmsnorm launch failed: %s", hipGetErrorString(e));
    return gemv_dev_locked(ggml_type, w, xn, out, inner, outer, (hipStream_t)stream);
}

int ihip_dequantize_dev(int ggml_type, const void *src, float *dst, int64_t n, ihip_stream stream)
{
    std::lock_guard<std::recursive_mutex> lk(ctx().mu);
    if (disabled())
        return fail(IHIP_ERR_DISABLED, "IHIP_DISABLE is set");
    if (!known_type(ggml_type))
        return fail(IHIP_ERR_INVALID, "unknown ggml type %d", ggml_type);
    if (n < 0 || n % block_elems(ggml_type))
        return fail(IHIP_ERR_INVALID, "n=%lld is not a multiple of %d", (long long)n,
                    block_elems(ggml_type));
    if (n == 0)
        return IHIP_OK;
    if (!src || !dst)
        return fail(IHIP_ERR_INVALID, "null pointer");
    if (overlap(src, (size_t)(n / block_elems(ggml_type)) * (size_t)block_bytes(ggml_type), dst,
                4 * (size_t)n))
        return fail(IHIP_ERR_INVALID, "src overlaps dst");
    hipError_t e = launch_dequant(ggml_type, src, dst, n, al16(src) && al16(dst), (hipStream_t)stream);
    if (e != hipSuccess)
        return fail(IHIP_ERR_HIP, "dequant launch failed: %s", hipGetErrorString(e));
    return IHIP_OK;
}

int ihip_gate_up_swiglu_dev(int gate_type, const void *wg, int up_type, const void *wu,
                            const float *x, float *h, int hidden, int inter, ihip_stream stream)
{
    std::lock_guard<std::recursive_mutex> lk(ctx().mu);
    if (disabled())
        return fail(IHIP_ERR_DISABLED, "IHIP_DISABLE is set");
    return gate_up_dev_locked(gate_type, wg, up_type, wu, x, h, hidden, inter, (hipStream_t)stream);
}

int ihip_ffn_swiglu_dev(int gate_type, const void *wg, int up_type, const void *wu,
                        int down_type, const void *wd, const float *x, float *h, float *y,
                        int hidden, int inter, ihip_stream stream)
{
    std::lock_guard<std::recursive_mutex> lk(ctx().mu);
    if (disabled())
        return fail(IHIP_ERR_DISABLED, "IHIP_DISABLE is set");
    RET_IF(check_shape(down_type, inter, hidden));
    if (!wd || !y)
        return fail(IHIP_ERR_INVALID, "null pointer");
    RET_IF(gate_up_dev_locked(gate_type, wg, up_type, wu, x, h, hidden, inter, (hipStream_t)stream));
    return gemv_dev_locked(down_type, wd, h, y, inter, hidden, (hipStream_t)stream);
}

int ihip_lm_head_argmax_dev(int ggml_type, const void *w, const float *x, float *logits,
                            int32_t *token, uint32_t *flags, int hidden, int vocab, void *workspace,
                            ihip_stream stream)
{
    std::lock_guard<std::recursive_mutex> lk(ctx().mu);
    if (disabled())
        return fail(IHIP_ERR_DISABLED, "IHIP_DISABLE is set");
    return lm_head_dev_locked(ggml_type, w, x, logits, token, flags, hidden, vocab, workspace,
                              (hipStream_t)stream);
}

int ihip_lm_head_argmax_noalloc_dev(int ggml_type, const void *w, const float *x, float *logits,
                                    int32_t *token, uint32_t *flags, int hidden, int vocab,
                                    ihip_stream stream)
{
    std::lock_guard<std::recursive_mutex> lk(ctx().mu);
    if (disabled())
        return fail(IHIP_ERR_DISABLED, "IHIP_DISABLE is set");
    RET_IF(check_shape(ggml_type, hidden, vocab));
    const int nparts = lm_head_parts(ggml_type, w, x, hidden, vocab);
    if (nparts > kArgMaxParts)
        return fail(IHIP_ERR_INVALID, "this lm_head needs %d argmax partials; the scratch holds %d",
                    nparts, kArgMaxParts);
    void *ws = nullptr;
    RET_IF(scratch_for_current_device(&ws));
    return lm_head_dev_locked(ggml_type, w, x, logits, token, flags, hidden, vocab, ws,
                              (hipStream_t)stream);
}

int ihip_argmax_dev(const float *logits, int64_t n, int32_t *token, uint32_t *flags,
                    void *workspace, ihip_stream stream)
{
    std::lock_guard<std::recursive_mutex> lk(ctx().mu);
    if (disabled())
        return fail(IHIP_ERR_DISABLED, "IHIP_DISABLE is set");
    if (n == 0)
        return fail(IHIP_ERR_EMPTY, "logits must not be empty");
    if (n < 0 || n >= 0xffffffffll)
        return fail(IHIP_ERR_INVALID, "n=%lld out of range", (long long)n);
    if (!logits || !token || !flags || !workspace)
        return fail(IHIP_ERR_INVALID, "null pointer");
    hipError_t e = launch_argmax(logits, n, token, flags, workspace, (hipStream_t)stream);
    if (e != hipSuccess)
        return fail(IHIP_ERR_HIP, "argmax launch failed: %s", hipGetErrorString(e));
    return IHIP_OK;
}

int ihip_fused_mlp_gate_mul_dev(float *gate, const float *up, int64_t n, ihip_stream stream)
{
    if (disabled())
        return fail(IHIP_ERR_DISABLED, "IHIP_DISABLE is set");
    if (n < 0)
        return fail(IHIP_ERR_INVALID, "n < 0");
    if (n == 0)
        return IHIP_OK;
    if (!gate || !up)
        return fail(IHIP_ERR_INVALID, "null pointer");
    hipError_t e = launch_mlp_gate_mul(gate, up, n, (hipStream_t)stream);
    if (e != hipSuccess)
        return fail(IHIP_ERR_HIP, "launch failed: %s", hipGetErrorString(e));
    return IHIP_OK;
}

int ihip_fused_silu_gate_mul_dev(float *out, const float *x, const float *gate, int64_t n,
                                 ihip_stream stream)
{
    if (disabled())
        return fail(IHIP_ERR_DISABLED, "IHIP_DISABLE is set");
    if (n < 0)
        return fail(IHIP_ERR_INVALID, "n < 0");
    if (n == 0)
        return IHIP_OK;
    if (!out || !x || !gate)
        return fail(IHIP_ERR_INVALID, "null pointer");
    hipError_t e = launch_silu_gate_mul(out, x, gate, n, (hipStream_t)stream);
    if (e != hipSuccess)
        return fail(IHIP_ERR_HIP, "launch failed: %s", hipGetErrorString(e));
    return IHIP_OK;
}

size_t ihip_prefill_scratch_bytes(int T, int inner)
{
    if (T <= 0 || inner <= 0)
        return 0;
    return prefill_scratch_bytes(T, inner);
}

int ihip_prefill_q4_k_dev(const void *w, const float *X, void *xh, float *Y, int T, int inner,
                          int outer, ihip_stream stream)
{
    std::lock_guard<std::recursive_mutex> lk(ctx().mu);
    if (disabled())
        return fail(IHIP_ERR_DISABLED, "IHIP_DISABLE is set");
    RET_IF(check_shape(kQ4_K, inner, outer));
    if (T <= 0)
        return fail(IHIP_ERR_INVALID, "T=%d must be positive", T);
    if (!prefill_fits(T, inner, outer))
        return fail(IHIP_ERR_INVALID, "prefill operands must stay below 4 GiB (T*inner*2 and W bytes) and T*outer below 2^31");
    if (!w || !X || !xh || !Y)
        return fail(IHIP_ERR_INVALID, "null pointer");
    if (!al16(w) || !al16(X) || !al16(xh) || !al16(Y))
        return fail(IHIP_ERR_INVALID, "prefill pointers must be 16-byte aligned");
    {
        const size_t xb = 4 * (size_t)T * (size_t)inner, yb = 4 * (size_t)T * (size_t)outer;
        const size_t sb = prefill_scratch_bytes(T, inner);
        if (overlap(X, xb, Y, yb) || overlap(xh, sb, X, xb) || overlap(xh, sb, Y, yb))
            return fail(IHIP_ERR_INVALID, "X, xh and Y must not overlap");
    }
    hipError_t e = launch_prefill_q4k(w, X, xh, Y, T, inner, outer, (hipStream_t)stream);
    if (e != hipSuccess)
        return fail(IHIP_ERR_HIP, "prefill launch failed: %s", hipGetErrorString(e));
    return IHIP_OK;
}

int ihip_prefill_convert_dev(const float *X, void *xh, int T, int inner, ihip_stream stream)
{
    std::lock_guard<std::recursive_mutex> lk(ctx().mu);
    if (disabled())
        return fail(IHIP_ERR_DISABLED, "IHIP_DISABLE is set");
    RET_IF(check_shape(kQ4_K, inner, 1));
    if (T <= 0)
        return fail(IHIP_ERR_INVALID, "T=%d must be positive", T);
    if (inner <= kPrefillF32MaxK)
        return fail(IHIP_ERR_INVALID, "rows of at most %d columns are multiplied on fp32 operands "
                    "straight from X: call ihip_prefill_q4_k_dev", kPrefillF32MaxK);
    if (!prefill_fits(T, inner, 1))
        return fail(IHIP_ERR_INVALID, "T*inner*2 must stay below 4 GiB");
    if (!X || !xh)
        return fail(IHIP_ERR_INVALID, "null pointer");
    if (!al16(X) || !al16(xh))
        return fail(IHIP_ERR_INVALID, "prefill pointers must be 16-byte aligned");
    if (overlap(X, 4 * (size_t)T * (size_t)inner, xh, prefill_scratch_bytes(T, inner)))
        return fail(IHIP_ERR_INVALID, "X and xh must not overlap");
    hipError_t e = launch_prefill_convert(X, xh, T, inner, (hipStream_t)stream);
    if (e != hipSuccess)
        return fail(IHIP_ERR_HIP, "prefill conversion launch failed: %s", hipGetErrorString(e));
    return IHIP_OK;
}

int ihip_prefill_q4_k_xh_dev(const void *w, void *xh, float *Y, int T, int inner, int outer,
                             ihip_stream stream)
{
    std::lock_guard<std::recursive_mutex> lk(ctx().mu);
    if (disabled())
        return fail(IHIP_ERR_DISABLED, "IHIP_DISABLE is set");
    RET_IF(check_shape(kQ4_K, inner, outer));
    if (T <= 0)
        return fail(IHIP_ERR_INVALID, "T=%d must be positive", T);
    if (inner <= kPrefillF32MaxK)
        return fail(IHIP_ERR_INVALID, "rows of at most %d columns are multiplied on fp32 operands "
                    "straight from X: call ihip_prefill_q4_k_dev", kPrefillF32MaxK);
    if (!prefill_fits(T, inner, outer))
        return fail(IHIP_ERR_INVALID, "prefill operands must stay below 4 GiB (T*inner*2 and W bytes) and T*outer below 2^31");
    if (!w || !xh || !Y)
        return fail(IHIP_ERR_INVALID, "null pointer");
    if (!al16(w) || !al16(xh) || !al16(Y))
        return fail(IHIP_ERR_INVALID, "prefill pointers must be 16-byte aligned");
    if (overlap(xh, prefill_scratch_bytes(T, inner), Y, 4 * (size_t)T * (size_t)outer))
        return fail(IHIP_ERR_INVALID, "xh and Y must not overlap");
    hipError_t e = launch_prefill_gemm(w, xh, Y, T, inner, outer, (hipStream_t)stream);
    if (e != hipSuccess)
        return fail(IHIP_ERR_HIP, "prefill launch failed: %s", hipGetErrorString(e));
    return IHIP_OK;
}

int ihip_prefill_q4_k_f32_dev(const void *w, const float *X, float *Y, int T, int inner,
                              int outer, ihip_stream stream)
{
    std::lock_guard<std::recursive_mutex> lk(ctx().mu);
    if (disabled())
        return fail(IHIP_ERR_DISABLED, "IHIP_DISABLE is set");
    RET_IF(check_shape(kQ4_K, inner, outer));
    if (T <= 0)
        return fail(IHIP_ERR_INVALID, "T=%d must be positive", T);
    if ((int64_t)T * outer > (int64_t)INT32_MAX)
        return fail(IHIP_ERR_INVALID, "T*outer must stay below 2^31");
    if (!w || !X || !Y)
        return fail(IHIP_ERR_INVALID, "null pointer");
    if (!al16(w) || !al16(X) || !al16(Y))
        return fail(IHIP_ERR_INVALID, "prefill pointers must be 16-byte aligned");
    if (overlap(X, 4 * (size_t)T * (size_t)inner, Y, 4 * (size_t)T * (size_t)outer))
        return fail(IHIP_ERR_INVALID, "X and Y must not overlap");
    hipError_t e = launch_prefill_q4k_f32(w, X, Y, T, inner, outer, (hipStream_t)stream);
    if (e != hipSuccess)
        return fail(IHIP_ERR_HIP, "prefill launch failed: %s", hipGetErrorString(e));
    return IHIP_OK;
}

int ihip_quantize_row_q8_k_dev(const float *x, void *y, int64_t k, ihip_stream stream)
{
    std::lock_guard<std::recursive_mutex> lk(ctx().mu);
    if (disabled())
        return fail(IHIP_ERR_DISABLED, "IHIP_DISABLE is set");
    if (!x || !y)
        return fail(IHIP_ERR_INVALID, "null pointer");
    if (k <= 0 || k % 256)
        return fail(IHIP_ERR_INVALID, "k=%lld is not a positive multiple of 256", (long long)k);
    if (((uintptr_t)x & 3u) || ((uintptr_t)y & 3u))
        return fail(IHIP_ERR_INVALID, "x and y must be 4-byte aligned");
    hipError_t e = launch_quantize_q8k(x, y, k, (hipStream_t)stream);
    if (e != hipSuccess)
        return fail(IHIP_ERR_HIP, "quantize launch failed: %s", hipGetErrorString(e));
    return IHIP_OK;
}

int ihip_gemv_q8k_dev(int ggml_type, const void *w, const void *q8, float *out, int inner,
                      int outer, ihip_stream stream)
{
    std::lock_guard<std::recursive_mutex> lk(ctx().mu);
    if (disabled())
        return fail(IHIP_ERR_DISABLED, "IHIP_DISABLE is set");
    RET_IF(check_shape(ggml_type, inner, outer));
    if (!q8k_type(ggml_type))
        return fail(IHIP_ERR_INVALID, "the Q8_K path takes Q4_K, Q5_K or Q6_K, not type %d",
                    ggml_type);
    if (!w || !q8 || !out)
        return fail(IHIP_ERR_INVALID, "null pointer");
    const uintptr_t wa = ggml_type == kQ6_K ? 1u : 15u;
    if (((uintptr_t)w & wa) || ((uintptr_t)q8 & 3u) || ((uintptr_t)out & 3u))
        return fail(IHIP_ERR_INVALID, "w must be %d-byte aligned, q8 and out 4-byte aligned",
                    (int)wa + 1);
    hipError_t e = launch_gemv_q8k(ggml_type, w, q8, out, inner, outer, (hipStream_t)stream);
    if (e != hipSuccess)
        return fail(IHIP_ERR_HIP, "q8k gemv launch failed: %s", hipGetErrorString(e));
    return IHIP_OK;
}

int ihip_gemv_q8k_x_dev(int ggml_type, const void *w, const float *x, float *out, void *q8,
                        int inner, int outer, ihip_stream stream)
{
    std::lock_guard<std::recursive_mutex> lk(ctx().mu);
    if (disabled())
        return fail(IHIP_ERR_DISABLED, "IHIP_DISABLE is set");
    RET_IF(check_shape(ggml_type, inner, outer));
    if (!q8k_type(ggml_type))
        return fail(IHIP_ERR_INVALID, "the Q8_K path takes Q4_K, Q5_K or Q6_K, not type %d",
                    ggml_type);
    if (!w || !x || !out)
        return fail(IHIP_ERR_INVALID, "null pointer");
    const uintptr_t wa = ggml_type == kQ6_K ? 1u : 15u;
    if (((uintptr_t)w & wa) || ((uintptr_t)x & 3u) || ((uintptr_t)q8 & 3u) || ((uintptr_t)out & 3u))
        return fail(IHIP_ERR_INVALID, "w must be %d-byte aligned, x, q8 and out 4-byte aligned",
                    (int)wa + 1);
    const bool one_launch = (ggml_type == kQ4_K || ggml_type == kQ5_K) && inner <= 32768 &&
                            ((uintptr_t)x & 15u) == 0;
    if (!one_launch && !q8)
        return fail(IHIP_ERR_INVALID, "this shape or type quantizes x into q8 first: pass q8 "
                                      "(inner/256 Q8_K blocks)");
    hipError_t e = launch_gemv_q8k_x(ggml_type, w, x, q8, nullptr, out, inner, outer, (hipStream_t)stream);
    if (e != hipSuccess)
        return fail(IHIP_ERR_HIP, "q8k gemv launch failed: %s", hipGetErrorString(e));
    return IHIP_OK;
}

int ihip_rmsnorm_dev(const float *x, const float *w, float eps, float *out, int n,
                     ihip_stream stream)
{
    std::lock_guard<std::recursive_mutex> lk(ctx().mu);
    if (disabled())
        return fail(IHIP_ERR_DISABLED, "IHIP_DISABLE is set");
    if (!x || !w || !out)
        return fail(IHIP_ERR_INVALID, "null pointer");
    if (n <= 0)
        return fail(IHIP_ERR_INVALID, "n=%d must be positive", n);
    hipError_t e = launch_rmsnorm(x, w, eps, out, n, (hipStream_t)stream);
    if (e != hipSuccess)
        return fail(IHIP_ERR_HIP, "rmsnorm launch failed: %s", hipGetErrorString(e));
    return IHIP_OK;
}

int ihip_ffn_block_dev(int gate_type, const void *wg, int up_type, const void *wu, int down_type,
                       const void *wd, const float *norm_w, float eps, float *x, float *h,
                       int hidden, int inter, ihip_stream stream)
{
    std::lock_guard<std::recursive_mutex> lk(ctx().mu);
    if (disabled())
        return fail(IHIP_ERR_DISABLED, "IHIP_DISABLE is set");
    RET_IF(check_shape(down_type, inter, hidden));
    if (!wd || !norm_w || !x || !h)
        return fail(IHIP_ERR_INVALID, "null pointer");
    // h holds inter + hidden floats (ihip_ffn_block_scratch_floats): the
    // unfused pass puts the normed input after h
    float *xn = gate_up_fused(gate_type, wg, up_type, wu, x, hidden, norm_w) ? nullptr : h + inter;
    RET_IF(gate_up_dev_locked(gate_type, wg, up_type, wu, x, h, hidden, inter, (hipStream_t)stream,
                              norm_w, eps, xn));
    return gemv_dev_locked(down_type, wd, h, x, inter, hidden, (hipStream_t)stream, x);
}

int ihip_lm_head_argmax_norm_dev(int ggml_type, const void *w, const float *norm_w, float eps,
                                 const float *x, float *xn, float *logits, int32_t *token,
                                 uint32_t *flags, int hidden, int vocab, void *workspace,
                                 ihip_stream stream)
{
    std::lock_guard<std::recursive_mutex> lk(ctx().mu);
    if (disabled())
        return fail(IHIP_ERR_DISABLED, "IHIP_DISABLE is set");
    if (!norm_w || !x || !xn)
        return fail(IHIP_ERR_INVALID, "null pointer");
    RET_IF(check_shape(ggml_type, hidden, vocab));
    hipError_t e = launch_rmsnorm(x, norm_w, eps, xn, hidden, (hipStream_t)stream);
    if (e != hipSuccess)
        return fail(IHIP_ERR_HIP, "rmsnorm launch failed: %s", hipGetErrorString(e));
    return lm_head_dev_locked(ggml_type, w, xn, logits, token, flags, hidden, vocab, workspace,
                              (hipStream_t)stream);
}

} // extern "C"
