"""The host-side GGUF parser (inferno.jl_amd/csrc/gguf.hip, plain C++) under
AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU.

The parser reads untrusted files, so it is compiled with the sanitizers into a
small driver (tests/native/gguf_asan_main.cpp) and run over the well-formed
files and refusal cases of tests/test_gguf.py plus seeded mutations of a good
file (truncations at every section boundary, byte flips in the header, the
key/value and tensor-info sections, oversized counts and lengths).  Every file
must be accepted or refused cleanly: a sanitizer report fails the test.
"""
import os
import shutil
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

from inferno_hip import synth

from test_gguf import ALL_KVS, ARR, STR, U8, U32, gguf_bytes, sample_tensors

ROOT = Path(__file__).resolve().parents[1]
GXX = shutil.which("g++")


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    if GXX is None:
        pytest.skip("no g++")
    d = tmp_path_factory.mktemp("gguf_asan")
    src = d / "gguf_reader.cpp"      # the reader's source, compiled as C++
    shutil.copyfile(ROOT / "inferno.jl_amd" / "csrc" / "gguf.hip", src)
    exe = d / "gguf_asan"
    flags = ["-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
             "-fsanitize=address,undefined", "-fno-sanitize-recover=all"]
    cmd = [GXX, *flags, "-I", str(ROOT / "include"), "-o", str(exe), str(src),
           str(ROOT / "tests" / "native" / "gguf_asan_main.cpp")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    return exe


def _run(exe, files):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:exitcode=86",
               UBSAN_OPTIONS="print_stacktrace=1:exitcode=87")
    env.pop("LD_PRELOAD", None)
    r = subprocess.run([str(exe), *map(str, files)], capture_output=True, text=True, env=env,
                       errors="replace")
    assert r.returncode == 0 and "Sanitizer" not in r.stderr, r.stderr[-6000:]
    return r.stdout


def _files(tmp_path):
    rng = synth.rng_for(0xA5A)
    tensors = sample_tensors(rng)
    good, data_offset, _ = gguf_bytes(ALL_KVS + [("general.alignment", U32, 64)], tensors, 64)
    blobs = {"good": good, "v2": gguf_bytes(ALL_KVS[:4], tensors[:2], version=2)[0],
             "empty": b"", "magic_only": b"GGUF",
             "v1": gguf_bytes(ALL_KVS, tensors, version=1)[0],
             "huge_count": b"GGUF" + struct.pack("<IQQ", 3, 2 ** 62, 2 ** 62),
             "huge_string": b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 2 ** 63) + b"k",
             "huge_array": b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k"
                           + struct.pack("<IIQ", ARR, U8, 2 ** 62),
             "deep_nesting": b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k"
                             + struct.pack("<I", ARR) + struct.pack("<IQ", ARR, 1) * 10000,
             "rank5": gguf_bytes([], [("w", (1, 1, 1, 1, 32), 0, b"\0" * 128)])[0],
             "bad_type": gguf_bytes([], [("w", (64,), 99, b"\0" * 64)])[0],
             "past_end": good[:-1],
             "huge_offset": gguf_bytes([], [("w", (32,), 0, b"\0" * 128)])[0]}
    # truncate at many points, including every section boundary
    cuts = sorted(set(list(range(0, 64)) + list(range(64, data_offset + 64, 7)) + [len(good) - 16]))
    for c in cuts:
        blobs[f"cut{c}"] = good[:c]
    # seeded byte flips in the header / key-values / tensor infos
    r = np.random.default_rng(7)
    for i in range(300):
        b = bytearray(good)
        for _ in range(int(r.integers(1, 4))):
            pos = int(r.integers(0, data_offset))
            b[pos] = int(r.integers(0, 256))
        blobs[f"flip{i}"] = bytes(b)
    # tensor offset pointing far past the end
    ho = bytearray(blobs["huge_offset"])
    # header 24 bytes, then name length 8, "w", ndim 4, one dim 8, type 4: the offset
    idx = 24 + 8 + 1 + 4 + 8 + 4
    assert ho[idx:idx + 8] == struct.pack("<Q", 0)
    ho[idx:idx + 8] = struct.pack("<Q", 2 ** 40)
    blobs["huge_offset"] = bytes(ho)
    paths = []
    for k, v in blobs.items():
        p = tmp_path / f"{k}.gguf"
        p.write_bytes(v)
        paths.append(p)
    return paths


def test_gguf_reader_under_address_sanitizer(driver, tmp_path):
    paths = _files(tmp_path)
    out = _run(driver, paths)
    last = out.strip().splitlines()[-1]
    acc, ref = int(last.split()[1]), int(last.split()[3])
    assert acc + ref == len(paths)
    assert "good.gguf: accepted" in out and "v2.gguf: accepted" in out
    for bad in ("empty", "magic_only", "v1", "huge_count", "huge_string", "huge_array", "rank5",
                "past_end", "huge_offset"):
        assert f"{bad}.gguf: refused" in out, bad


def test_the_sanitizer_is_live(driver):
    env = dict(os.environ, ASAN_OPTIONS="exitcode=86")
    env.pop("LD_PRELOAD", None)
    r = subprocess.run([str(driver), "--self-check"], capture_output=True, text=True, env=env,
                       errors="replace")
    assert r.returncode == 86 and "heap-buffer-overflow" in r.stderr
