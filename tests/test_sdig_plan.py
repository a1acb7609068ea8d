"""CPU check of the streamed digit GEMV's launch arithmetic (no GPU).

k_gemv_sdig (Q6_K / Q8_0 / IQ4_NL GEMV, the lm_head with the fused argmax,
the FFN down projection) forms every address, LDS offset, wait count and row
index through inferno.jl_amd/csrc/kq_sdig_plan.h.  tests/native/sdig_check.hip
includes the same header and walks a whole launch -- every workgroup, wave,
item, copy and lane -- asserting that global reads and writes stay inside W,
x, y and the argmax partials, copies land in the wave's own LDS ring, ring
reads stay inside a slot, each vmcnt wait covers the item it guards, every
wave meets the same barriers and every row is produced exactly once.

The launches checked are the ones the GPU tests and the benchmark make (with
every tuning-knob combination they set), the 151936 x 2048 plain Q6_K GEMV,
and knob values and CU counts that push the grid to its limits.
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
    L.sdig_check.argtypes = [C.c_int] * 9 + [C.c_char_p, C.c_int, C.POINTER(C.c_longlong)]
    L.sdig_check.restype = C.c_longlong

    def run(t, inner, outer, argmax=False, rows=0, depth=0, wg=0, waves=0, ncu=256):
        msg = C.create_string_buffer(512)
        st = (C.c_longlong * 8)()
        n = L.sdig_check(t, inner, outer, int(argmax), rows, depth, wg, waves, ncu, msg, 512, st)
        return n, msg.value.decode(), list(st)
    return run


# (type, outer, inner) the GPU tests run through the streamed kernel
STREAM_SHAPES = ((Q6_K, 1029, 12288), (Q6_K, 77, 6144), (Q6_K, 300, 24576), (Q6_K, 33, 10240),
                 (Q8_0, 1031, 4096), (Q8_0, 45, 2304), (Q8_0, 19, 256), (IQ4_NL, 517, 4608))
DEFAULT_SHAPES = ((Q6_K, 4096, 12288), (Q6_K, 300, 2048), (Q8_0, 4096, 4096), (Q8_0, 11, 2304),
                  (IQ4_NL, 2048, 1024), (IQ4_NL, 1000, 4096), (IQ4_NL, 13, 2304),
                  (Q6_K, 4096, 4096), (IQ4_NL, 4096, 4096), (Q6_K, 512, 2048), (Q8_0, 256, 4096),
                  (Q6_K, 1, 2048), (Q8_0, 1, 256), (Q6_K, 65, 16384), (Q8_0, 8191, 14336))
# sdig knob sets of the GPU tests: (depth, rows, workgroups per CU, waves)
KNOBS = ((2, 0, 0, 0), (4, 1, 1, 8), (8, 7, 2, 16), (2, 64, 1, 12), (4, 33, 3, 6), (2, 5, 2, 16),
         (6, 16, 2, 12))


def _streamed(t, inner):
    """Rows the host gives this kernel: 1..8 segments of 2048 columns."""
    return -(-inner // 2048) <= 8


def _ok(res, what):
    n, msg, st = res
    assert n == 0, f"{what}: {n} violations, first: {msg}"
    return st


@pytest.mark.parametrize("argmax", [False, True])
def test_lm_head_shape_151936x2048(chk, argmax):
    """The Q6_K lm_head shape, plain GEMV and fused argmax, default launch:
    8 waves, two ring slots, 32 rows per chunk, 768 workgroups."""
    st = _ok(chk(Q6_K, 2048, 151936, argmax), "Q6_K 151936x2048")
    grid, nw, d, rpc, nseg, copies, rows, w_hi = st
    assert (grid, nw, d, rpc, nseg) == (768, 8, 2, 32, 1)
    assert rows == 151936 and w_hi == 151936 * 8 * 210  # reads reach the last byte, no further
    assert copies == 151936 * 2 * 64  # every wave has >= 2 rows: one pair of 64-lane copies per row


def test_lm_head_knob_sets(chk):
    for argmax in (False, True):
        for t, vocab in ((Q6_K, 151936), (Q6_K, 1000), (Q8_0, 32000)):
            for kn in ({}, {"wg": 1, "rows": 7}):
                _ok(chk(t, 2048, vocab, argmax, **kn), f"type {t} vocab {vocab} {kn} argmax={argmax}")


@pytest.mark.parametrize("t,outer,inner", DEFAULT_SHAPES)
def test_default_launches(chk, t, outer, inner):
    for argmax in (False, True):
        _ok(chk(t, inner, outer, argmax), f"type {t} {outer}x{inner} argmax={argmax}")


@pytest.mark.parametrize("knobs", KNOBS)
def test_tuned_launches(chk, knobs):
    depth, rows, wg, waves = knobs
    for t, outer, inner in STREAM_SHAPES + DEFAULT_SHAPES[:4]:
        if not _streamed(t, inner):
            continue  # 12 segments: the fp32 streamed kernel takes these rows
        for argmax in (False, True):
            _ok(chk(t, inner, outer, argmax, rows=rows, depth=depth, wg=wg, waves=waves),
                f"type {t} {outer}x{inner} knobs {knobs} argmax={argmax}")


def test_argmax_grid_stays_within_the_partials(chk):
    """One partial per workgroup: whatever the knobs and the CU count, the
    fused-argmax grid is at most 16384 workgroups (the 256 KiB workspace)."""
    for ncu in (256, 304, 1024):
        st = _ok(chk(Q6_K, 2048, 1_000_003, True, rows=1, wg=64, ncu=ncu), f"ncu {ncu}")
        assert st[0] == 16384
        st = _ok(chk(Q8_0, 2048, 600_000, True, rows=1, wg=1000, ncu=ncu), f"ncu {ncu}")
        assert st[0] <= 16384


def test_small_and_odd_devices(chk):
    for ncu in (1, 7, 80):
        for t, outer, inner in ((Q6_K, 4096, 12288), (Q6_K, 151936, 2048), (Q8_0, 1031, 4096)):
            _ok(chk(t, inner, outer, False, ncu=ncu), f"ncu {ncu} type {t} {outer}x{inner}")


def test_checker_flags_shapes_the_host_never_sends(chk):
    # 3 Q6_K blocks (630 bytes) or 15 Q8_0 blocks are not whole 16-byte units:
    # the host routes them to the byte-granular kernel, and the check says why
    n, msg, _ = chk(Q6_K, 768, 7)
    assert n > 0 and "16-byte" in msg
    n, msg, _ = chk(Q8_0, 480, 7)
    assert n > 0 and "16-byte" in msg
    n, msg, _ = chk(Q6_K, 2048 * 9, 7)  # nine segments: more than the kernel takes
    assert n > 0
