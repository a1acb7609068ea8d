// prefill_check.hip -- host-side check of the prefill GEMM's split over K
// (k_prefill_q4k and k_prefill_splits_sum in inferno.jl_amd/csrc/kq_prefill.hip).
//
// Test infrastructure, run on the CPU only: it launches nothing.  It includes
// the header the launcher and the kernel take the plan from (kq_launch.h:
// prefill_splits, prefill_grid, prefill_lin, prefill_split_of and the scratch
// layout) and walks one launch, workgroup by workgroup, asserting that
//   * the grid's workgroups map one to one onto (split, tile) pairs, the rest
//     exit;
//   * every split has at least one block column and its columns lie inside
//     the row, and every (tile, block column) is reduced by exactly one
//     workgroup, so the planes summed hold each column once;
//   * the activation and weight bytes a split's copies reach (the last block
//     column's 512 bytes of the last token row, 144 bytes of the last weight
//     row) lie inside Xh and W;
//   * the partial planes the splits past the first write (T x outer floats
//     each) lie inside the scratch, after the fp16 activations and the
//     per-token scales, and the summing launch reads only those planes.
//
// Built by inferno_hip.build into tests/native/_build/libsdig_check.so;
// called from tests/test_prefill_plan.py through ctypes.
#include "kq_launch.h"

#include <cstdarg>
#include <cstdio>
#include <vector>

using namespace ihip;

namespace {

struct PReport {
    char *msg;
    int cap;
    long long n = 0;
    void fail(const char *fmt, ...)
    {
        if (n++ == 0 && msg && cap > 0) {
            va_list ap;
            va_start(ap, fmt);
            vsnprintf(msg, (size_t)cap, fmt, ap);
            va_end(ap);
        }
    }
};

} // namespace

// Returns the number of violations (0: the launch is sound); msg receives
// the first.  stats[0] = nsplit, stats[1] = grid, stats[2] = partial floats
// written, stats[3] = the scratch's partial capacity in floats.
extern "C" long long prefill_check(int T, int inner, int outer, int ncu, char *msg, int cap,
                                   long long *stats)
{
    PReport r{msg, cap};
    if (T <= 0 || inner <= 0 || inner % 256 || outer <= 0) {
        r.fail("bad shape");
        return r.n;
    }
    const int nblk = inner / 256;
    const int mtiles = (T + kPrefillBM - 1) / kPrefillBM, ntiles = (outer + kPrefillBN - 1) / kPrefillBN;
    const int tiles = mtiles * ntiles;
    const int nsplit = prefill_splits(T, inner, outer, ncu);
    const int grid = prefill_grid(tiles, nsplit);
    if (nsplit < 1 || nsplit > nblk)
        r.fail("nsplit %d outside 1..%d", nsplit, nblk);
    if (nsplit > 1 && tiles * nsplit > kPrefillMaxTiles)
        r.fail("%d tiles x %d splits past the %d partial tiles", tiles, nsplit, kPrefillMaxTiles);

    const size_t xh_bytes = (size_t)2 * T * inner, w_bytes = (size_t)outer * nblk * 144;
    const size_t plane = (size_t)T * outer;
    const size_t part_cap = prefill_part_floats(T);
    if (prefill_scale_offset(T, inner) < xh_bytes)
        r.fail("scales overlap the activations");
    if (prefill_part_offset(T, inner) < prefill_scale_offset(T, inner) + 4 * (size_t)T ||
        prefill_part_offset(T, inner) % 16)
        r.fail("partial planes overlap the scales or are not 16-byte aligned");
    if (prefill_scratch_bytes(T, inner) != prefill_part_offset(T, inner) + 4 * part_cap)
        r.fail("scratch size is not the partial planes' end");

    std::vector<int> seen_lin((size_t)tiles * nsplit, 0);
    std::vector<int> cover((size_t)tiles * nblk, 0);
    size_t part_written = 0;
    for (int bid = 0; bid < grid; ++bid) {
        const int lin = prefill_lin(bid, tiles, nsplit);
        if (lin < 0) {
            r.fail("workgroup %d: negative place %d", bid, lin);
            continue;
        }
        if (lin >= tiles * nsplit)
            continue; // exits before any access
        seen_lin[lin]++;
        const PrefillSplit s = prefill_split_of(lin, mtiles, ntiles, nblk, nsplit);
        if (s.sp < 0 || s.sp >= nsplit || s.mt < 0 || s.mt >= mtiles || s.nt < 0 || s.nt >= ntiles) {
            r.fail("workgroup %d: split %d tile (%d, %d) outside the launch", bid, s.sp, s.mt, s.nt);
            continue;
        }
        if (s.nk < 1 || s.kb0 < 0 || s.kb0 + s.nk > nblk) {
            r.fail("workgroup %d: columns %d + %d outside 0..%d", bid, s.kb0, s.nk, nblk);
            continue;
        }
        for (int kb = s.kb0; kb < s.kb0 + s.nk; ++kb)
            cover[(size_t)(s.nt * mtiles + s.mt) * nblk + kb]++;
        // the farthest bytes the copies reach: token rows and weight rows
        // past T or outer re-read the last one
        const size_t last_x = ((size_t)(T - 1) * inner + (size_t)(s.kb0 + s.nk) * 256) * 2;
        const size_t last_w = (size_t)(outer - 1) * nblk * 144 + (size_t)(s.kb0 + s.nk) * 144;
        if (last_x > xh_bytes)
            r.fail("workgroup %d: activation copies reach byte %zu of %zu", bid, last_x, xh_bytes);
        if (last_w > w_bytes)
            r.fail("workgroup %d: weight copies reach byte %zu of %zu", bid, last_w, w_bytes);
        if (s.sp > 0) {
            const size_t end = (size_t)s.sp * plane; // plane sp - 1 ends here
            if (end > part_cap)
                r.fail("workgroup %d: partial plane %d ends at float %zu of %zu", bid, s.sp - 1, end, part_cap);
            if (end > part_written)
                part_written = end;
        }
    }
    for (size_t i = 0; i < seen_lin.size(); ++i)
        if (seen_lin[i] != 1)
            r.fail("place %zu taken by %d workgroups", i, seen_lin[i]);
    for (size_t i = 0; i < cover.size(); ++i)
        if (cover[i] != 1)
            r.fail("tile %zu column %zu reduced %d times", i / nblk, i % nblk, cover[i]);
    // the summing launch reads planes 0 .. nsplit - 2
    if (nsplit > 1 && (size_t)(nsplit - 1) * plane != part_written)
        r.fail("summed planes %d x %zu floats, written %zu", nsplit - 1, plane, part_written);
    if (stats) {
        stats[0] = nsplit;
        stats[1] = grid;
        stats[2] = (long long)part_written;
        stats[3] = (long long)part_cap;
    }
    return r.n;
}
