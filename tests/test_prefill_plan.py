"""CPU check of the prefill GEMM's split over K (no GPU).

A weight of few rows leaves most CUs without a 64-token x 128-row tile, so
the launcher shares each tile's block columns out over several workgroups
(the splits) and a second launch adds their partial sums.  The plan comes
from inferno.jl_amd/csrc/kq_launch.h; tests/native/prefill_check.hip walks a
whole launch with the same functions and checks that every (tile, block
column) is reduced exactly once, that the copies stay inside the operands and
that the partial planes fit the caller's scratch (ihip_prefill_scratch_bytes
does not depend on the number of weight rows).
"""
import ctypes as C
from pathlib import Path

import pytest

LIB = Path(__file__).resolve().parent / "native" / "_build" / "libsdig_check.so"


@pytest.fixture(scope="module")
def chk():
    from inferno_hip import build
    build.build_checks()  # the checker follows the header it includes
    L = C.CDLL(str(LIB))
    L.prefill_check.argtypes = [C.c_int] * 4 + [C.c_char_p, C.c_int, C.POINTER(C.c_longlong)]
    L.prefill_check.restype = C.c_longlong

    def run(T, inner, outer, ncu=256):
        msg = C.create_string_buffer(512)
        st = (C.c_longlong * 4)()
        n = L.prefill_check(T, inner, outer, ncu, msg, 512, st)
        assert n == 0, f"T={T} {outer}x{inner} ncu={ncu}: {n} violations, first: {msg.value.decode()}"
        return list(st)
    return run


# (T, outer, inner) of the GPU tests and the benchmark
GPU_SHAPES = ((512, 4096, 4096), (70, 300, 2048), (1, 128, 256), (33, 129, 1792), (5, 64, 512),
              (40, 200, 768), (64, 256, 1024), (512, 512, 4096), (100, 384, 4096),
              (17, 1000, 2816), (7, 129, 2048), (48, 320, 2048), (8, 128, 1024),
              (9, 300, 14336), (3, 130, 8448), (582, 1758, 768), (100, 300, 2560), (66, 130, 768))


@pytest.mark.parametrize("T,outer,inner", GPU_SHAPES)
def test_gpu_test_launches(chk, T, outer, inner):
    chk(T, inner, outer)


def test_which_launches_split(chk):
    # the full-size workload keeps one workgroup per tile; narrow weights split
    assert chk(512, 4096, 4096)[0] == 1
    assert chk(512, 4096, 512)[0] == 8
    assert chk(64, 4096, 4096)[0] == 8
    assert chk(512, 4096, 2048)[0] == 2
    assert chk(17, 2816, 1000)[0] == 5      # 11 block columns: uneven splits
    assert chk(512, 1024, 1024)[0] == 1     # 4 block columns: not split
    assert chk(512, 4096, 512, ncu=32)[0] == 1  # a small device has no idle CUs


@pytest.mark.parametrize("ncu", [1, 32, 80, 256, 304, 1024])
def test_sweep(chk, ncu):
    for T in (1, 7, 64, 65, 100, 512, 2048):
        for outer in (1, 64, 129, 512, 1000, 4096, 14336):
            for inner in (256, 1792, 2048, 2816, 4096, 8192, 16384):
                chk(T, inner, outer, ncu)
