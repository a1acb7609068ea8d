// kq_sdig_plan.h -- launch plan and index arithmetic of the streamed digit
// GEMV (k_gemv_sdig, kq_gemv.hip): Q6_K / Q8_0 / IQ4_NL rows, the lm_head with
// the fused argmax, the FFN down projection.
//
// The kernel forms every global address, LDS offset, wait count and row index
// through these functions, and the host-side bounds check
// (tests/native/sdig_check.hip) enumerates the same functions over every
// workgroup, wave, item and lane of a launch, so the check runs the very
// arithmetic the kernel runs.
//
// Geometry.  K is cut into segments of 2048 columns (8 Q6_K blocks of 210 B,
// 64 Q8_0 blocks of 34 B, 64 IQ4_NL blocks of 18 B; the last may be shorter).
// A wave's time per row segment is its instruction count whatever the number
// of active lanes, so a short last segment is not worth evening out.  A
// workgroup of NW waves walks chunks of `rpc` rows grid-stride.  Wave w owns
// segment w % nseg and, when there are more waves than segments, every
// (NW / nseg)-th row of a chunk; its rows of all its chunks are numbered
// items k = 0, 1, ... and stream through a private D-slot LDS ring (slot
// k % D) by direct-to-LDS copies of 64 lanes x 16 bytes.
//
// Rows need not be 16-byte multiples (Q6_K rows of any block count, Q8_0 and
// IQ4_NL rows of any multiple of 32 columns): a row segment is copied from the
// 16-byte unit at or below its first byte, so it sits in its slot at a byte
// phase of 0..14 (even: every block size is even), which the dot adds to its
// offsets.  The copies read whole aligned units: the matrix's last unit may
// reach up to 14 bytes past W's last byte, inside the 16-byte unit (and so the
// page) that holds that byte; those bytes are never used.
#pragma once

#include "kq_common.h"

#include <stddef.h>
#include <stdint.h>

namespace ihip {

constexpr int kSdigMaxRows = 64;    // rows per chunk (part[] in LDS holds one chunk)
constexpr int kSdigMaxSeg = 16;     // segments per row: one wave each in a 16-wave workgroup
constexpr int kArgMaxParts = 16384; // argmax partials: IHIP_ARGMAX_WS_BYTES / 16
constexpr int kDigQuads = 10;       // staged digits per lane: 10 x 16 bytes

__host__ __device__ constexpr int sd_min(int a, int b) { return a < b ? a : b; }
__host__ __device__ constexpr int sd_max(int a, int b) { return a > b ? a : b; }

// blocks and bytes per 2048-column segment
__host__ __device__ constexpr int sdig_seg_blocks(int fmt) { return fmt == kQ6_K ? 8 : 64; }
__host__ __device__ constexpr int sdig_seg_bytes(int fmt)
{
    return sdig_seg_blocks(fmt) * block_bytes(fmt);
}
// copy instructions per row segment (each moves 1 KB) and the ring slot size
__host__ __device__ constexpr int sdig_ipr(int fmt) { return (sdig_seg_bytes(fmt) / 16 + 63) / 64; }
__host__ __device__ constexpr int sdig_slot(int fmt) { return sdig_ipr(fmt) * 1024; }
// segments whose digits can be staged in LDS for the segment's other waves
__host__ __device__ constexpr int sdig_share_cap(int nw) { return nw == 12 ? 6 : nw == 8 ? 2 : 0; }

// LDS of a workgroup of NW waves with D ring slots: the ring, the staged
// digits, the chunk partial sums (one column per wave) and 2 KB for the rest;
// it must fit the 160 KB of a CU.
__host__ __device__ constexpr int sdig_lds(int fmt, int nw, int d)
{
    return nw * d * sdig_slot(fmt) + sdig_share_cap(nw) * kDigQuads * 1024 + kSdigMaxRows * nw * 4 + 2048;
}
__host__ __device__ constexpr bool sdig_fits(int fmt, int nw, int d) { return sdig_lds(fmt, nw, d) <= 160 * 1024; }

__host__ __device__ inline int sdig_nseg(int fmt, int nblk)
{
    return (nblk + sdig_seg_blocks(fmt) - 1) / sdig_seg_blocks(fmt);
}

// One wave's share of a launch.
struct SdigWave {
    int nseg;        // segments per row (<= NW, host-checked)
    int wps;         // waves per segment
    int sg, rl;      // this wave's segment and its rank among the segment's waves
    bool worker;     // waves past nseg * wps only join the barriers
    bool share;      // the segment's digits are staged in LDS (workgroup-uniform)
    bool producer;   // this wave loads x and forms the digits
    int nchunks;     // chunks of the whole matrix
    int seg_blocks;  // blocks of this wave's segment
    int seg_len;     // bytes of this wave's segment
    int x0;          // first column (element of x) of this wave's segment
    uint32_t my_ring;// LDS byte offset of this wave's ring within the ring array
    int m;           // rows per full chunk
    int my_chunks;   // chunks of this workgroup
    int nitems;      // rows (items) of this wave over all its chunks
    int mm;          // max(m, 1)
    size_t row_bytes;
};

__host__ __device__ inline SdigWave sdig_wave(int fmt, int NW, int D, int SHC, int outer, int nblk,
                                              int rpc, int bid, int grid, int w)
{
    SdigWave g;
    const int bb = block_bytes(fmt);
    g.row_bytes = (size_t)nblk * bb;
    g.nseg = sdig_nseg(fmt, nblk);
    g.wps = NW / g.nseg;
    g.sg = w % g.nseg;
    g.rl = w / g.nseg;
    g.worker = g.rl < g.wps;
    g.share = SHC > 0 && g.nseg <= SHC && g.wps >= 2;
    g.producer = !g.share || g.rl == 0;
    g.nchunks = (outer + rpc - 1) / rpc;
    g.seg_blocks = sd_min(sdig_seg_blocks(fmt), nblk - g.sg * sdig_seg_blocks(fmt));
    g.seg_len = g.seg_blocks * bb;
    g.x0 = g.sg * sdig_seg_blocks(fmt) * block_elems(fmt);
    g.my_ring = (uint32_t)(w * D * sdig_slot(fmt));
    g.m = g.worker ? (rpc - g.rl + g.wps - 1) / g.wps : 0;
    g.my_chunks = bid < g.nchunks ? (g.nchunks - 1 - bid) / grid + 1 : 0;
    g.nitems = g.my_chunks * g.m;
    if (g.worker && g.my_chunks > 0 && bid + (g.my_chunks - 1) * grid == g.nchunks - 1) {
        const int last = outer - (g.nchunks - 1) * rpc; // rows of the last chunk
        g.nitems = (g.my_chunks - 1) * g.m + sd_max(0, (last - g.rl + g.wps - 1) / g.wps);
    }
    g.mm = sd_max(g.m, 1);
    return g;
}

// Global row of item k (clamped: always a row of W).  int operands throughout
// (an unsigned operand would send min to its double overload in device code).
__host__ __device__ inline int sdig_item_row(const SdigWave &g, int k, int bid, int grid, int rpc,
                                             int outer)
{
    const int ci = k / g.mm, rr = k - ci * g.mm;
    return sd_min((bid + ci * grid) * rpc + g.rl + rr * g.wps, outer - 1);
}

// Byte offset in W of this wave's segment of `row`.
__host__ __device__ inline size_t sdig_seg_off(const SdigWave &g, int fmt, int row)
{
    return (size_t)g.sg * (size_t)sdig_seg_bytes(fmt) + (size_t)row * g.row_bytes;
}
// Byte offset in W of the row segment copied for item k: items past the
// wave's last re-copy its last item's row into a slot no remaining item uses.
__host__ __device__ inline size_t sdig_copy_row(const SdigWave &g, int fmt, int k, int bid, int grid,
                                                int rpc, int outer)
{
    const int kk = sd_max(0, sd_min(k, g.nitems - 1));
    return sdig_seg_off(g, fmt, sdig_item_row(g, kk, bid, grid, rpc, outer));
}
// Whether rows of nblk blocks leave segments off 16-byte boundaries.
__host__ __device__ constexpr bool sdig_phased(int fmt, int nblk) { return (nblk * block_bytes(fmt)) % 16 != 0; }
// Where a segment at byte offset `off` of W lands in its slot (0..15; even),
// and the 16-byte units its copies cover, from the unit at off - phase.
__host__ __device__ inline uint32_t sdig_phase(size_t off) { return (uint32_t)(off & 15u); }
__host__ __device__ inline int sdig_units(const SdigWave &g, uint32_t phase)
{
    return ((int)phase + g.seg_len + 15) >> 4;
}
// Byte offset, from the segment's first unit, of lane `lane`'s 16 bytes in
// copy i: every copy runs with all 64 lanes on (lanes past the segment
// re-read its last unit into the slot's tail), so the copies in flight are a
// compile-time count.
__host__ __device__ inline uint32_t sdig_copy_lane(int units, int i, int lane)
{
    return 16u * (uint32_t)sd_min(64 * i + lane, units - 1);
}
// LDS byte offset (within the ring array) where copy i of item k lands; lane
// l's 16 bytes go to this + 16 l.
__host__ __device__ inline uint32_t sdig_copy_dst(const SdigWave &g, int fmt, int D, int k, int i)
{
    return g.my_ring + (uint32_t)((k % D) * sdig_slot(fmt)) + 1024u * (uint32_t)i;
}
// Items whose copies may still be in flight when item k is read: those issued
// after it (k + 1 .. max(D, nitems) - 1, at most D - 1).  The wait is
// vmcnt(ipr x this); younger loads and stores only lengthen it.
__host__ __device__ inline int sdig_wait_items(const SdigWave &g, int D, int k)
{
    return sd_min(D - 1, sd_max(D, g.nitems) - 1 - k);
}

// A producer lane's x slice: float offset of its first element within the
// segment, and whether the lane covers a block of the segment (an inactive
// lane loads the segment's first values and zeroes them).
//   Q6_K: block bs = lane >> 3, half n = (lane >> 2) & 1, positions
//         l0 = 8 (lane & 3) .. +7, groups g at +32 g (elements 128n + 32g + l0 + i);
//   Q8_0 / IQ4_NL: block lane, 32 consecutive values.
__host__ __device__ inline int sdig_x_lane(int fmt, int lane, int seg_blocks, bool &active)
{
    if (fmt == kQ6_K) {
        const int bs = lane >> 3, n = (lane >> 2) & 1, l0 = 8 * (lane & 3);
        active = bs < seg_blocks;
        return active ? 256 * bs + 128 * n + l0 : 0;
    }
    active = lane < seg_blocks;
    return active ? 32 * lane : 0;
}
// Byte offset of the lane's load t (0..7, 16 bytes each) from its first element.
__host__ __device__ constexpr int sdig_x_load_byte(int fmt, int t)
{
    return fmt == kQ6_K ? 128 * (t >> 1) + 16 * (t & 1) : 16 * t;
}

// ---- lane geometry of the ring reads --------------------------------------
// A lane's place in a Q6_K segment: the dword-aligned LDS offsets (within a
// ring slot) of its ql, qh and scale bytes and of d, and the byte phase they
// share (210-byte blocks leave odd blocks 2 bytes past a dword boundary).
// The dot reads 3 dwords at a, at a + 32, at h and at s, and 2 bytes at d.
// Computed once, so a row costs one address add per array.
struct Q6DigLane {
    uint32_t a, h, s, d, sh;
    int c; // which 16 of the lane's 32 elements' scale: l0 >> 4
};

// The same lane's offsets for a segment at byte phase ph (even, 0..14) of its
// slot: the byte positions move by ph, so the dword-aligned offsets move by
// ph rounded down to 4 (plus 4 when the 2-byte phases add up to 4) and the
// byte phase of the reads becomes (sh + ph) mod 4.
__host__ __device__ inline Q6DigLane q6_dig_lane_at(Q6DigLane L, uint32_t ph)
{
    const uint32_t t = L.sh + (ph & 3u);
    const uint32_t o = (ph & ~3u) + (t & 4u);
    L.a += o;
    L.h += o;
    L.s += o;
    L.d += ph;
    L.sh = t & 3u;
    return L;
}

__host__ __device__ inline Q6DigLane q6_dig_lane(int lane)
{
    const uint32_t bs = lane >> 3, n = (lane >> 2) & 1, l0 = 8 * (lane & 3);
    const uint32_t bo = 210u * bs;
    Q6DigLane L;
    L.a = (bo + 64 * n + l0) & ~3u;
    L.h = (bo + 128 + 32 * n + l0) & ~3u;
    L.s = (bo + 192 + 8 * n) & ~3u;
    L.d = bo + 208;
    L.sh = bo & 3u;
    L.c = (int)(l0 >> 4);
    return L;
}

// Q8_0 / IQ4_NL: lane = block of the segment.  The dot reads d (2 bytes at the
// block's offset) and sdig_blk_dwords dwords from the dword below offset + 2.
__host__ __device__ constexpr uint32_t sdig_blk_off(int fmt, int lane)
{
    return (uint32_t)block_bytes(fmt) * (uint32_t)lane;
}
__host__ __device__ constexpr int sdig_blk_dwords(int fmt) { return fmt == kQ8_0 ? 9 : 5; }

// Chunk ci of a workgroup: first row, rows, and this wave's rows in it.
struct SdigChunk {
    int row0, nrows, mine;
};
__host__ __device__ inline SdigChunk sdig_chunk(const SdigWave &g, int ci, int bid, int grid, int rpc,
                                                int outer)
{
    SdigChunk c;
    c.row0 = (bid + ci * grid) * rpc;
    c.nrows = sd_min(rpc, outer - c.row0);
    c.mine = g.worker ? sd_max(0, sd_min(g.m, (c.nrows - g.rl + g.wps - 1) / g.wps)) : 0;
    return c;
}
// Row (within the chunk) of the wave's rr-th row of a chunk.
__host__ __device__ inline int sdig_chunk_row(const SdigWave &g, int rr) { return g.rl + rr * g.wps; }

// ---- host: the launch plan ------------------------------------------------
struct SdigPlan {
    int nseg, nw, d, rpc, grid;
};

// Waves per workgroup, rows per chunk and workgroups per CU by segment count,
// measured on MI355X (us per GEMV in sweeps of HBM-resident copies; the
// previous plan in parentheses where it differed):
//   1 segment     8 waves, 2 per CU (LDS), 32 rows for the 151936 x 2048
//                 Q6_K lm_head (53-55 us), by size for plain rows (sdig_plan).
//                 Rows finish inside their wave.
//   2..6          12 waves, 16 rows, 1 per CU (all of 113-137 KB of LDS a CU
//                 holds; 4 per CU queued three more in rounds: 12288 x 4096
//                 Q6_K 11.2 us against 15.6): 4096 x 4096 Q8_0 6.47, Q6_K 6.48,
//                 IQ4_NL 6.23 (8 waves: 6.95+); 4096 x 6144 Q6_K 8.17;
//                 4096 x 8192 Q8_0 9.67 (16.0); 4096 x 10240 Q8_0 12.70
//                 (18.7); 4096 x 12288 Q6_K 12.3-12.4 (6 waves: 14.3).
//                 Two or more waves per segment share its staged digits.
//   7..8          16 waves, 16 rows, 2 per CU: 4096 x 14336 Q6_K 15.1-15.5
//                 (18.2), IQ4_NL 16.1-16.3 (19.8); 4096 x 16384 Q6_K 15.7
//                 (18.9).  Q8_0, whose 16-wave workgroup takes 104 KB of
//                 LDS: 8 waves, 16 rows, 4 per CU (4096 x 16384 17.0; 21.8).
//   9..12         12 waves, 16 rows, 1 per CU: 4096 x 24576 Q6_K 20.6 (16
//                 waves 21.3), 4096 x 20480 Q8_0 21.9 (23.0).
//   13..16        16 waves, 16 rows, 1 per CU: 8192 x 28672 Q6_K 42.6 (2 per
//                 CU 46.5), 4096 x 32768 Q8_0 30.7.
// Rows of several segments meet in LDS once per chunk; at 4096 rows the
// sweeps' best chunk was 16 rows throughout (4 and 8 lost 0.5-7 us, 32 up to
// 10 us).  Other row counts: sdig_plan.
inline int sdig_waves(int fmt, int nseg)
{
    return nseg == 1 ? 8 : nseg <= 6 ? 12 : nseg <= 8 ? (fmt == kQ8_0 ? 8 : 16) : nseg <= 12 ? 12 : 16;
}
inline int sdig_rows(int nseg) { return nseg == 1 ? 32 : 16; }
inline int sdig_wg_per_cu(int fmt, int nseg)
{
    return nseg == 1 ? 3 : nseg <= 6 ? 1 : nseg <= 8 ? (fmt == kQ8_0 ? 4 : 2) : 1;
}

// Whether the streamed kernel takes rows of nblk blocks: 1..16 segments.
inline bool sdig_rows_ok(int fmt, int nblk)
{
    const int nseg = (nblk + sdig_seg_blocks(fmt) - 1) / sdig_seg_blocks(fmt);
    return nblk > 0 && nseg >= 1 && nseg <= kSdigMaxSeg;
}

// The launch: waves, ring depth (slots per wave), rows per chunk and grid.
// With the fused argmax every workgroup leaves one partial, so the grid stays
// within kArgMaxParts whatever the device's CU count.
inline SdigPlan sdig_plan(int fmt, int nblk, int outer, bool argmax, int ncu)
{
    SdigPlan p;
    p.nseg = sdig_nseg(fmt, nblk);
    p.nw = sdig_waves(fmt, p.nseg);
    p.d = 2;
    p.rpc = sd_min(sdig_rows(p.nseg), kSdigMaxRows);
    const int ncu1 = sd_max(1, ncu);
    int per_cu = sdig_wg_per_cu(fmt, p.nseg);
    // One-segment rows: the staged digits put a workgroup at 56-72 KB of LDS,
    // two per CU.  With the argmax (the lm_head) 32 rows per chunk (151936 x
    // 2048 Q6_K 53.3-54.6 us against 55.3-57.2 with one x load per wave and
    // three workgroups per CU); plain, rows per chunk by matrix size (151936 x
    // 2048 52.1 us against 61.0 with 3 per CU and 32 rows; 4096 x 2048 Q8_0
    // 4.72 against 6.30; 2048 x 2048 Q6_K with 8-row chunks 4.39 against 6.12).
    if (p.nseg == 1) {
        per_cu = 2;
        if (!argmax)
            p.rpc = outer >= 64 * ncu1 ? 32 : outer >= 16 * ncu1 ? 16 : 8;
        // a third ring slot per wave where two workgroups still fit a CU
        // (Q6_K / IQ4_NL: 2 x 71 KB; Q8_0's 3 KB slots would not): 151936 x
        // 2048 Q6_K 49.4 us against 52.1 with two slots (four: 58.1, one
        // workgroup per CU)
        if (per_cu * sdig_lds(fmt, p.nw, 3) <= 160 * 1024)
            p.d = 3;
    }
    // Two-segment rows of more chunks than one 12-wave workgroup per CU holds
    // at once: 8-wave workgroups, two per CU, keep 16 waves working on a CU
    // instead of 12 (12288 x 4096 Q6_K 10.75 us against 11.2; 9728 x 2560
    // 10.96 against 11.6).
    if (p.nseg == 2 && (outer + p.rpc - 1) / p.rpc > ncu1) {
        p.nw = 8;
        per_cu = 2;
    }
    // Two-segment rows of fewer 16-row chunks than CUs: 8-row chunks on
    // 8-wave workgroups, two per CU, so no CU idles (2048 x 4096 Q6_K 5.5 us
    // against 6.2, IQ4_NL 4.9 against 5.8; at 4096 rows, one 16-row chunk per
    // CU, the 12-wave plan stays: 6.3 us against 7.1 with 8-row chunks and
    // 7.4 with 16 waves).
    if (p.nseg == 2 && (outer + 15) / 16 < ncu1) {
        p.nw = 8;
        per_cu = 2;
        p.rpc = 8;
    }
    const int resident = ncu1 * per_cu;
    // rows of the busiest resident slot with r rows per chunk
    auto busiest = [&](int r) { return ((outer + r - 1) / r + resident - 1) / resident * r; };
    // 12 or 16 waves: 8-row chunks where 16-row chunks spill past one round
    // of resident workgroups unevenly (5120 x 17408 Q6_K: 320 chunks of 16 on
    // 256 workgroups, 29.0 us with 8-row chunks against 36.8)
    if (p.nw >= 12 && p.nseg > 1 && (outer + 15) / 16 > resident && busiest(8) < busiest(16))
        p.rpc = 8;
    int grid = sd_max(1, sd_min((outer + p.rpc - 1) / p.rpc, ncu1 * per_cu));
    if (argmax)
        grid = sd_min(grid, kArgMaxParts);
    p.grid = grid;
    return p;
}

} // namespace ihip
