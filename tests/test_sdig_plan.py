"""CPU check of the streamed digit GEMV's launch arithmetic (no GPU).

k_gemv_sdig (Q6_K / Q8_0 / IQ4_NL GEMV, the lm_head with the fused argmax,
the FFN down projection) forms every address, LDS offset, wait count and row
index through inferno.jl_amd/csrc/kq_sdig_plan.h.  tests/native/sdig_check.hip
includes the same header and walks a whole launch -- every workgroup, wave,
item, copy and lane -- asserting that global reads and writes stay inside W,
x, y and the argmax partials, copies land in the wave's own LDS ring, ring
reads stay inside a slot, each vmcnt wait covers the item it guards, every
wave meets the same barriers and every row is produced exactly once.

The launches checked are the ones the GPU tests and the benchmark make, the
151936 x 2048 plain Q6_K GEMV, rows of every segment count the kernel takes
(1..16), and CU counts that push the grid to its limits.
"""
import ctypes as C
from pathlib import Path

import pytest

from inferno_hip import synth

LIB = Path(__file__).resolve().parent / "native" / "_build" / "libsdig_check.so"
Q6_K, Q8_0, IQ4_NL = synth.Q6_K, synth.Q8_0, synth.IQ4_NL


@pytest.fixture(scope="module")
def chk():
    if not LIB.exists():
        from inferno_hip import build
        build.build_checks()
    L = C.CDLL(str(LIB))
    L.sdig_check.argtypes = [C.c_int] * 5 + [C.c_char_p, C.c_int, C.POINTER(C.c_longlong)]
    L.sdig_check.restype = C.c_longlong

    def run(t, inner, outer, argmax=False, ncu=256):
        msg = C.create_string_buffer(512)
        st = (C.c_longlong * 8)()
        n = L.sdig_check(t, inner, outer, int(argmax), ncu, msg, 512, st)
        return n, msg.value.decode(), list(st)
    return run


# (type, outer, inner) the GPU tests run through the streamed kernel
STREAM_SHAPES = ((Q6_K, 1029, 12288), (Q6_K, 77, 6144), (Q6_K, 300, 24576), (Q6_K, 33, 10240),
                 (Q6_K, 65, 16384), (Q8_0, 1031, 4096), (Q8_0, 45, 2304), (Q8_0, 19, 256),
                 (IQ4_NL, 517, 4608), (Q8_0, 300, 14336), (Q8_0, 129, 18688), (Q6_K, 40, 32768),
                 (IQ4_NL, 70, 30720), (Q6_K, 1031, 20480), (Q8_0, 300, 18432), (Q6_K, 515, 4096),
                 (Q8_0, 1030, 2048), (IQ4_NL, 777, 1024), (Q6_K, 1029, 14336), (IQ4_NL, 260, 16384))
DEFAULT_SHAPES = ((Q6_K, 4096, 12288), (Q6_K, 300, 2048), (Q8_0, 4096, 4096), (Q8_0, 11, 2304),
                  (IQ4_NL, 2048, 1024), (IQ4_NL, 1000, 4096), (IQ4_NL, 13, 2304),
                  (Q6_K, 4096, 4096), (IQ4_NL, 4096, 4096), (Q6_K, 512, 2048), (Q8_0, 256, 4096),
                  (Q6_K, 1, 2048), (Q8_0, 1, 256), (Q6_K, 65, 16384), (Q8_0, 8191, 14336))
# lm_head shapes of the GPU tests (vocab, hidden) with the fused argmax
ARGMAX_SHAPES = ((Q6_K, 1000, 2048), (Q8_0, 32000, 2048), (Q6_K, 4099, 8192), (Q8_0, 3001, 20480))


def _ok(res, what):
    n, msg, st = res
    assert n == 0, f"{what}: {n} violations, first: {msg}"
    return st


@pytest.mark.parametrize("argmax", [False, True])
def test_lm_head_shape_151936x2048(chk, argmax):
    """The Q6_K lm_head shape, plain GEMV and fused argmax, default launch:
    8 waves, three ring slots, 32 rows per chunk, 512 workgroups (the ring
    and the staged digits leave LDS for two per CU)."""
    st = _ok(chk(Q6_K, 2048, 151936, argmax), "Q6_K 151936x2048")
    grid, nw, d, rpc, nseg, copies, rows, w_hi = st
    assert (grid, nw, d, rpc, nseg) == (512, 8, 3, 32, 1)
    assert rows == 151936 and w_hi == 151936 * 8 * 210  # reads reach the last byte, no further
    assert copies == 151936 * 2 * 64  # every wave has >= 2 rows: one pair of 64-lane copies per row


@pytest.mark.parametrize("t,outer,inner", DEFAULT_SHAPES)
def test_default_launches(chk, t, outer, inner):
    for argmax in (False, True):
        _ok(chk(t, inner, outer, argmax), f"type {t} {outer}x{inner} argmax={argmax}")


@pytest.mark.parametrize("t,outer,inner", STREAM_SHAPES)
def test_gpu_test_launches(chk, t, outer, inner):
    for argmax in (False, True):
        _ok(chk(t, inner, outer, argmax), f"type {t} {outer}x{inner} argmax={argmax}")


@pytest.mark.parametrize("t,vocab,hidden", ARGMAX_SHAPES)
def test_fused_argmax_launches(chk, t, vocab, hidden):
    _ok(chk(t, hidden, vocab, True), f"type {t} vocab {vocab} hidden {hidden}")


@pytest.mark.parametrize("t", [Q6_K, Q8_0, IQ4_NL])
def test_every_segment_count(chk, t):
    """Rows of 1..16 segments (full and partial last segments): 8 waves for
    one segment, 12 for 2..6 and 9..12, 16 for 7..8 (Q8_0: 8) and 13..16; three
    ring slots for one segment where two workgroups still fit a CU (not Q8_0's
    3 KB slots), else two; 16 rows per chunk (at 4096 rows)."""
    unit = 2048 if t == Q6_K else 256  # the host's row-alignment unit
    for nseg in range(1, 17):
        for inner in {2048 * nseg, 2048 * nseg - (2048 - unit)}:
            st = _ok(chk(t, inner, 4096, False), f"type {t} inner {inner}")
            want = (8 if nseg == 1 else 12 if nseg <= 6 else (8 if t == Q8_0 else 16) if nseg <= 8
                    else 12 if nseg <= 12 else 16)
            depth = 3 if nseg == 1 and t != Q8_0 else 2
            assert (st[1], st[2], st[4]) == (want, depth, nseg), (inner, st)
            assert st[3] == 16, (inner, st)  # one segment: 16 rows per chunk at 4096 plain rows
    n, msg, _ = chk(t, 2048 * 16 + unit, 7)
    assert n > 0 and "does not take" in msg  # 17 segments: the byte-granular kernel's
    for nseg in range(1, 17):  # ragged row counts
        _ok(chk(t, 2048 * nseg - (2048 - unit), 1037, False), f"type {t} {nseg} segments, 1037 rows")


def test_plans_past_one_round_of_workgroups(chk):
    """Rows per chunk and waves where the chunks outnumber the workgroups a
    device holds at once: 5120 rows of 9 Q6_K segments (320 chunks of 16 on
    256 one-per-CU workgroups) take 8-row chunks, 4096 rows (256 chunks) keep
    16; two-segment rows of more than 256 chunks take two 8-wave workgroups per
    CU (grid, waves, rows per chunk)."""
    assert _ok(chk(Q6_K, 17408, 5120), "5120x17408")[3] == 8
    assert _ok(chk(Q6_K, 16384, 4096), "4096x16384")[3] == 16
    assert _ok(chk(Q6_K, 9728, 1037), "1037x9728")[3] == 16
    assert _ok(chk(Q8_0, 4096, 4096), "Q8_0 4096x4096")[:4] == [256, 12, 2, 16]
    assert _ok(chk(Q6_K, 4096, 4097), "4097x4096")[:4] == [257, 8, 2, 16]
    assert _ok(chk(Q6_K, 2560, 9728), "9728x2560")[:4] == [512, 8, 2, 16]
    assert _ok(chk(Q6_K, 2560, 151936), "151936x2560")[:4] == [512, 8, 2, 16]
    assert _ok(chk(Q6_K, 2560, 151936, True), "151936x2560 argmax")[:4] == [512, 8, 2, 16]


def test_argmax_grid_stays_within_the_partials(chk):
    """One partial per workgroup: whatever the CU count, the fused-argmax grid
    is at most 16384 workgroups (the 256 KiB workspace)."""
    for ncu in (256, 304, 1024, 4096, 5000, 20000):
        st = _ok(chk(Q6_K, 2048, 1_000_003, True, ncu=ncu), f"ncu {ncu}")
        assert st[0] == min(16384, 2 * ncu)
        st = _ok(chk(Q8_0, 8192, 600_000, True, ncu=ncu), f"ncu {ncu}")
        assert st[0] == min(16384, ncu)
        st = _ok(chk(Q8_0, 20480, 600_000, True, ncu=ncu), f"ncu {ncu}")
        assert st[0] == min(16384, ncu)


def test_small_and_odd_devices(chk):
    for ncu in (1, 7, 80):
        for t, outer, inner in ((Q6_K, 4096, 12288), (Q6_K, 151936, 2048), (Q8_0, 1031, 4096),
                                (Q8_0, 129, 18688)):
            _ok(chk(t, inner, outer, False, ncu=ncu), f"ncu {ncu} type {t} {outer}x{inner}")


# rows that are not 16-byte multiples: segments at byte phases 2..14
PHASED_SHAPES = ((Q6_K, 7, 768), (Q6_K, 1029, 9728), (Q6_K, 300, 2560), (Q6_K, 5, 256),
                 (Q6_K, 77, 17408), (Q6_K, 33, 2304), (Q8_0, 13, 896), (Q8_0, 31, 480),
                 (Q8_0, 1000, 2336), (IQ4_NL, 9, 2336), (IQ4_NL, 517, 4640), (Q6_K, 1031, 32512),
                 (Q8_0, 3, 32), (IQ4_NL, 1, 32))


@pytest.mark.parametrize("t,outer,inner", PHASED_SHAPES)
def test_phased_launches(chk, t, outer, inner):
    """Rows of any whole number of blocks: every copy starts on a 16-byte unit
    at or below its segment, covers it, and reads nothing past the 16-byte unit
    holding W's last byte; the dot's offsets at each phase land on the block."""
    bb = {Q6_K: 210, Q8_0: 34, IQ4_NL: 18}[t]
    nblk = inner // (256 if t == Q6_K else 32)
    assert (nblk * bb) % 16, "an aligned shape"
    for argmax in (False, True):
        st = _ok(chk(t, inner, outer, argmax), f"type {t} {outer}x{inner} argmax={argmax}")
        w_bytes = outer * nblk * bb
        assert w_bytes <= st[7] <= -(-w_bytes // 16) * 16, (w_bytes, st[7])


def test_phased_full_lm_head(chk):
    """The Q6_K lm_head of a 2560-wide model (151936 x 2560, 10 blocks a row)."""
    for argmax in (False, True):
        _ok(chk(Q6_K, 2560, 151936, argmax), f"151936x2560 argmax={argmax}")


def test_checker_flags_shapes_the_host_never_sends(chk):
    n, msg, _ = chk(Q6_K, 2048 * 17, 7)  # 17 segments: more than the kernel takes
    assert n > 0
    n, msg, _ = chk(Q8_0, 100, 7)  # not a whole number of blocks
    assert n > 0 and "bad shape" in msg
