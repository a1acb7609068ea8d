// sdig_check.hip -- host-side bounds and coverage check of the streamed digit
// GEMV launch (k_gemv_sdig in inferno.jl_amd/csrc/kq_gemv.hip).
//
// Test infrastructure, run on the CPU only: it launches nothing.  It includes
// the header the kernel forms its indices with (kq_sdig_plan.h) and walks one
// launch exactly as the kernel does -- every workgroup, wave, item, copy and
// lane -- asserting that
//   * every global byte read (x loads, row copies) and written (y, argmax
//     partials) lies inside its buffer -- the row copies, which read whole
//     aligned 16-byte units, inside W or the 16-byte unit holding W's last
//     byte -- and every copy covers its row segment;
//   * shapes the host sends to the unphased kernel have every segment on a
//     16-byte boundary;
//   * every direct-to-LDS copy lands inside the wave's own ring, and every
//     ring read of the dot lies inside the slot;
//   * the explicit vmcnt wait before reading item k never allows more copies
//     in flight than were issued after item k's (so the wait covers k), and
//     its count fits the instruction's field;
//   * the staged-digit slots, the chunk partial-sum rows and the argmax
//     partial index are inside their arrays;
//   * every wave of a workgroup executes the same number of barriers;
//   * every row (and, with several segments, every row segment) is produced
//     exactly once, and each wave reads exactly the items it issued.
//
// Built by inferno_hip.build as tests/native/_build/libsdig_check.so; called
// from tests/test_sdig_plan.py through ctypes.
#include "kq_sdig_plan.h"

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <vector>

using namespace ihip;

namespace {

struct Report {
    char *msg;
    int cap;
    long long errors = 0;
    void fail(const char *fmt, ...)
    {
        if (errors++ == 0 && msg && cap > 0) {
            va_list ap;
            va_start(ap, fmt);
            vsnprintf(msg, (size_t)cap, fmt, ap);
            va_end(ap);
        }
    }
};

} // namespace

// Returns the number of violations (0: the launch is clean); msg receives the
// first.  stats[0..7]: grid, waves, ring depth, rows per chunk, segments,
// copies checked, rows produced, highest W byte read + 1.
extern "C" long long sdig_check(int fmt, int inner, int outer, int argmax, int ncu, char *msg,
                                int cap, long long *stats)
{
    Report R{msg, cap};
    if (msg && cap > 0)
        msg[0] = 0;
    if (fmt != kQ6_K && fmt != kQ8_0 && fmt != kIQ4_NL) {
        R.fail("format %d is not streamed", fmt);
        return R.errors;
    }
    if (inner <= 0 || outer <= 0 || inner % block_elems(fmt)) {
        R.fail("bad shape %d x %d", outer, inner);
        return R.errors;
    }
    const int nblk = inner / block_elems(fmt);
    if (!sdig_rows_ok(fmt, nblk)) {
        R.fail("the host does not take %d blocks to this kernel", nblk);
        return R.errors;
    }
    const SdigPlan p = sdig_plan(fmt, nblk, outer, argmax != 0, ncu);
    const int NW = p.nw, D = p.d, rpc = p.rpc, grid = p.grid;
    const int IPR = sdig_ipr(fmt), SLOT = sdig_slot(fmt), bb = block_bytes(fmt);
    const int SHC = sdig_share_cap(NW);
    const size_t row_bytes = (size_t)nblk * bb, w_bytes = (size_t)outer * row_bytes;
    const size_t w_units_end = (w_bytes + 15) & ~(size_t)15; // end of the unit holding W's last byte
    const int ring_bytes = NW * D * SLOT;

    // the instantiations the launcher can dispatch, and their LDS
    if (!((NW == 8 || NW == 12 || NW == 16) && (D == 2 || (D == 3 && NW == 8))))
        R.fail("plan picked %d waves x depth %d, which is not instantiated", NW, D);
    if (!sdig_fits(fmt, NW, D))
        R.fail("%d waves x depth %d do not fit the LDS", NW, D);
    if (p.nseg > NW)
        R.fail("%d segments > %d waves", p.nseg, NW);
    if (rpc < 1 || rpc > kSdigMaxRows)
        R.fail("rows per chunk %d outside 1..%d", rpc, kSdigMaxRows);
    if (grid < 1)
        R.fail("empty grid");
    if (argmax && grid > kArgMaxParts)
        R.fail("grid %d > %d argmax partials", grid, kArgMaxParts);
    if (SLOT < sdig_seg_bytes(fmt) + 16)
        R.fail("slot %d < segment %d + 16", SLOT, sdig_seg_bytes(fmt));
    const bool phased = sdig_phased(fmt, nblk);
    // the segments tile the row: contiguous, non-empty, at most 2048 columns
    {
        int next = 0;
        for (int s = 0; s < p.nseg; ++s) {
            const SdigWave g = sdig_wave(fmt, NW, D, 0, outer, nblk, rpc, 0, grid, s);
            if (g.sg != s || g.x0 != next * block_elems(fmt) || g.seg_blocks < 1 ||
                g.seg_blocks > sdig_seg_blocks(fmt))
                R.fail("segment %d: first block %d, %d blocks (expected first block %d)", s,
                       g.x0 / block_elems(fmt), g.seg_blocks, next);
            next += g.seg_blocks;
        }
        if (next != nblk)
            R.fail("segments cover %d of %d blocks", next, nblk);
    }
    if (R.errors)
        return R.errors;

    long long copies = 0;
    size_t w_hi = 0;
    std::vector<unsigned char> seen_row((size_t)outer, 0);
    std::vector<unsigned char> seen_seg((size_t)outer * p.nseg, 0);

    for (int bid = 0; bid < grid && R.errors < 20; ++bid) {
        int barriers0 = -1;
        for (int w = 0; w < NW; ++w) {
            const SdigWave g = sdig_wave(fmt, NW, D, SHC, outer, nblk, rpc, bid, grid, w);
            // x loads
            if (g.producer) {
                for (int lane = 0; lane < 64; ++lane) {
                    bool act = false;
                    const int base = g.x0 + sdig_x_lane(fmt, lane, g.seg_blocks, act);
                    for (int t = 0; t < 8; ++t) {
                        const long long f0 = base + sdig_x_load_byte(fmt, t) / 4;
                        if (f0 < 0 || f0 + 4 > inner)
                            R.fail("wg %d wave %d lane %d: x load %d reads floats [%lld, %lld) of %d",
                                   bid, w, lane, t, f0, f0 + 4, inner);
                    }
                }
            }
            if (g.share && g.sg >= SHC)
                R.fail("wg %d wave %d: staged digits of segment %d >= %d slots", bid, w, g.sg, SHC);
            // copies: items [0, max(D, nitems)) are issued (the prologue issues D)
            const int nissue = sd_max(D, g.nitems);
            for (int k = 0; k < nissue; ++k) {
                const size_t off = sdig_copy_row(g, fmt, k, bid, grid, rpc, outer);
                const uint32_t ph = sdig_phase(off);
                const int units = sdig_units(g, ph);
                if (!phased && ph)
                    R.fail("wg %d wave %d item %d: segment at phase %u in the unphased kernel", bid, w, k, ph);
                if (ph & 1)
                    R.fail("odd phase %u", ph);
                if (16 * units < (int)ph + g.seg_len || units > 64 * IPR)
                    R.fail("wg %d wave %d item %d: %d units for a %d-byte segment at phase %u (%d copies)",
                           bid, w, k, units, g.seg_len, ph, IPR);
                const size_t row = off - ph; // the first unit
                for (int i = 0; i < IPR; ++i) {
                    const uint32_t dst = sdig_copy_dst(g, fmt, D, k, i);
                    if (dst < g.my_ring || dst + 1024u > g.my_ring + (uint32_t)(D * SLOT) ||
                        dst + 1024u > (uint32_t)ring_bytes)
                        R.fail("wg %d wave %d item %d copy %d: LDS [%u, %u) outside the wave's ring "
                               "[%u, %u)", bid, w, k, i, dst, dst + 1024u, g.my_ring,
                               g.my_ring + (uint32_t)(D * SLOT));
                    for (int lane = 0; lane < 64; ++lane) {
                        const size_t src = row + sdig_copy_lane(units, i, lane);
                        ++copies;
                        if (src % 16 || src + 16 > w_units_end)
                            R.fail("wg %d wave %d item %d copy %d lane %d: W bytes [%zu, %zu) of %zu",
                                   bid, w, k, i, lane, src, src + 16, w_bytes);
                        // inside the units that hold this wave's segment of one row
                        if (src < row || src + 16 > row + 16 * (size_t)units)
                            R.fail("wg %d wave %d item %d copy %d lane %d: bytes [%zu, %zu) outside "
                                   "the segment's units [%zu, %zu)", bid, w, k, i, lane, src, src + 16,
                                   row, row + 16 * (size_t)units);
                        if (src + 16 > w_hi)
                            w_hi = src + 16;
                    }
                }
            }
            // ring reads of the dot (relative to a slot), at every phase the
            // kernel can meet: the bytes it uses lie inside the block at that
            // phase, and every read stays inside the slot
            for (uint32_t ph = 0; ph < (phased ? 16u : 1u); ph += 2) {
                for (int lane = 0; lane < 64; ++lane) {
                    uint32_t hi = 0;
                    if (fmt == kQ6_K) {
                        if ((lane >> 3) >= g.seg_blocks)
                            continue;
                        const Q6DigLane L0 = q6_dig_lane(lane);
                        const Q6DigLane L = phased ? q6_dig_lane_at(L0, ph) : L0;
                        const uint32_t bs = lane >> 3, n = (lane >> 2) & 1, l0 = 8 * (lane & 3);
                        const uint32_t blk = ph + 210u * bs; // the block's first byte in the slot
                        // the 8 bytes each read uses, and d
                        if (L.a + L.sh != blk + 64 * n + l0 || L.h + L.sh != blk + 128 + 32 * n + l0 ||
                            L.s + L.sh != blk + 192 + 8 * n || L.d != blk + 208 || L.sh > 2 || L.a % 4 ||
                            L.h % 4 || L.s % 4)
                            R.fail("phase %u lane %d: Q6_K offsets a %u h %u s %u d %u sh %u for block at %u",
                                   ph, lane, L.a, L.h, L.s, L.d, L.sh, blk);
                        const uint32_t ends[] = {L.a + 12, L.a + 32 + 12, L.h + 12, L.s + 12, L.d + 2};
                        for (uint32_t e : ends)
                            hi = e > hi ? e : hi;
                    } else {
                        if (lane >= g.seg_blocks)
                            continue;
                        const uint32_t o = sdig_blk_off(fmt, lane) + ph;
                        hi = ((o + 2) & ~3u) + 4u * (uint32_t)sdig_blk_dwords(fmt);
                        hi = o + 2 > hi ? o + 2 : hi;
                    }
                    if (hi > (uint32_t)SLOT)
                        R.fail("wave %d lane %d phase %u: the dot reads up to byte %u of a %d-byte slot", w,
                               lane, ph, hi, SLOT);
                    if (hi > (uint32_t)(IPR * 1024))
                        R.fail("lane %d reads past the copied bytes of a slot", lane);
                }
            }
            // the item walk: waits, rows, partial sums
            int k = 0, barriers = g.share ? 1 : 0;
            for (int ci = 0; ci < g.my_chunks; ++ci) {
                const SdigChunk c = sdig_chunk(g, ci, bid, grid, rpc, outer);
                if (c.row0 < 0 || c.row0 >= outer || c.nrows < 1)
                    R.fail("wg %d chunk %d: rows [%d, +%d) of %d", bid, ci, c.row0, c.nrows, outer);
                for (int rr = 0; rr < c.mine; ++rr, ++k) {
                    // issued before item k is read: [0, D) and j + D for j < k with j + D < nitems
                    const int last_issued = sd_max(D - 1, sd_min(k - 1 + D, g.nitems - 1));
                    const int wi = sdig_wait_items(g, D, k);
                    if (wi < 0 || wi > last_issued - k)
                        R.fail("wg %d wave %d item %d: waits for %d younger items, %d issued", bid,
                               w, k, wi, last_issued - k);
                    if (IPR * wi > 31)
                        R.fail("vmcnt(%d) does not fit the wait", IPR * wi);
                    const int lr = sdig_chunk_row(g, rr);
                    const int row = c.row0 + lr;
                    if (lr < 0 || lr >= c.nrows || row >= outer)
                        R.fail("wg %d wave %d chunk %d: row %d of %d", bid, w, ci, lr, c.nrows);
                    // the row whose copy item k read
                    if (sdig_item_row(g, k, bid, grid, rpc, outer) != row)
                        R.fail("wg %d wave %d item %d: read row %d, copied row %d", bid, w, k, row,
                               sdig_item_row(g, k, bid, grid, rpc, outer));
                    // the phase the dot adds is the phase the copy left
                    if (sdig_phase(sdig_seg_off(g, fmt, row)) !=
                        sdig_phase(sdig_copy_row(g, fmt, k, bid, grid, rpc, outer)))
                        R.fail("wg %d wave %d item %d: dot phase differs from the copy's", bid, w, k);
                    if (p.nseg == 1) {
                        if (row >= 0 && row < outer)
                            seen_row[(size_t)row]++;
                    } else {
                        if (lr >= kSdigMaxRows || g.sg >= NW)
                            R.fail("part[%d][%d] outside [%d][%d]", lr, g.sg, kSdigMaxRows, NW);
                        if (row >= 0 && row < outer)
                            seen_seg[(size_t)row * p.nseg + g.sg]++;
                    }
                }
                if (p.nseg > 1) {
                    barriers += 2;
                    if (w == 0) // the epilogue threads of this chunk
                        for (int i = 0; i < c.nrows; ++i) {
                            if (c.row0 + i >= outer)
                                R.fail("epilogue row %d >= %d", c.row0 + i, outer);
                            else
                                seen_row[(size_t)(c.row0 + i)]++;
                        }
                }
            }
            if (k != g.nitems)
                R.fail("wg %d wave %d reads %d items but issued for %d", bid, w, k, g.nitems);
            if (argmax) {
                barriers += 1;
                if (bid >= kArgMaxParts)
                    R.fail("parts[%d] outside %d", bid, kArgMaxParts);
            }
            if (barriers0 < 0)
                barriers0 = barriers;
            else if (barriers != barriers0)
                R.fail("wg %d: wave %d reaches %d barriers, wave 0 %d", bid, w, barriers, barriers0);
        }
    }
    for (int r = 0; r < outer && R.errors < 20; ++r) {
        if (seen_row[(size_t)r] != 1)
            R.fail("row %d produced %d times", r, (int)seen_row[(size_t)r]);
        if (p.nseg > 1)
            for (int s = 0; s < p.nseg; ++s)
                if (seen_seg[(size_t)r * p.nseg + s] != 1)
                    R.fail("row %d segment %d summed %d times", r, s,
                           (int)seen_seg[(size_t)r * p.nseg + s]);
    }
    if (stats) {
        stats[0] = grid;
        stats[1] = NW;
        stats[2] = D;
        stats[3] = rpc;
        stats[4] = p.nseg;
        stats[5] = copies;
        stats[6] = outer;
        stats[7] = (long long)w_hi;
    }
    return R.errors;
}
