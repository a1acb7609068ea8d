"""The C-ABI library loads, exports every symbol include/inferno_hip.h
declares, and behaves sanely without a GPU (CPU only: no compute calls)."""
import os
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "inferno_hip.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ihip_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_drop_in_surface():
    syms = declared_symbols()
    for s in ("ihip_q4_k_gemv", "ihip_q5_k_gemv", "ihip_q6_k_gemv", "ihip_q8_0_gemv",
              "ihip_dequantize", "ihip_ffn_swiglu", "ihip_lm_head_argmax", "ihip_prefill_q4_k",
              "ihip_gemv_dev", "ihip_argmax_dev", "ihip_fused_mlp_gate_mul_dev",
              "ihip_fused_silu_gate_mul_dev", "ihip_available", "ihip_last_error"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    from inferno_hip import _lib
    L = _lib.lib()
    missing = [s for s in declared_symbols() if not hasattr(L, s)]
    assert not missing, missing
    # and the ctypes table covers the header exactly
    assert sorted(_lib.SIGNATURES) == declared_symbols()


def test_library_is_gfx950_code():
    # the offload bundle inside the .so names its target triple
    blob = (ROOT / "inferno.jl_amd" / "lib" / "libinferno_hip.so").read_bytes()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob


def _run(code, env_extra=None):
    env = dict(os.environ)
    env.update(env_extra or {})
    env["HIP_VISIBLE_DEVICES"] = env.get("HIP_VISIBLE_DEVICES", "")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env,
                       cwd=str(ROOT))
    assert r.returncode == 0, r.stderr
    return r.stdout.strip()


PRE = ("import sys; sys.path[:0]=['inferno.jl_amd']\n"
       "import numpy as np\nfrom inferno_hip import _lib, QuantizedKernels as QK\n")


def test_disable_switch_reports_unavailable_and_raises():
    # mirrors INFERNO_NO_QUANT_KERNELS (src/QuantizedKernels.jl:26-32)
    out = _run(PRE + (
        "print(QK.quant_kernels_available())\n"
        "w=np.zeros(144,np.uint8); x=np.zeros(256,np.float32); o=np.zeros(1,np.float32)\n"
        "try:\n    QK.q4_k_gemv_(o,w,x,256,1); print('noraise')\n"
        "except _lib.IHIPError as e:\n    print(e.code)\n"), {"IHIP_DISABLE": "1"})
    assert out.splitlines() == ["False", str(_lib_code("IHIP_ERR_DISABLED"))]


def _lib_code(name):
    from inferno_hip import _lib
    return getattr(_lib, name)


def test_argument_errors_are_raised_before_any_device_work():
    from inferno_hip import QuantizedKernels as QK, _lib
    o = np.zeros(4, np.float32)
    x = np.zeros(256, np.float32)
    with pytest.raises(_lib.IHIPArgumentError):
        QK.q4_k_gemv_(o, np.zeros(10, np.uint8), x, 256, 4)      # too few weight bytes
    with pytest.raises(_lib.IHIPArgumentError):
        QK.q4_k_gemv_(o, np.zeros(4 * 144, np.uint8), x, 200, 4)  # inner not a multiple of 256
    with pytest.raises(_lib.IHIPArgumentError):
        QK.q8_0_gemv_(o, np.zeros(4 * 8 * 34, np.uint8), x.astype(np.float64), 256, 4)


def test_prefill_operands_past_32_bit_offsets_are_refused():
    """The prefill GEMM forms its operand addresses as 32-bit byte offsets from
    the start of Xh and W: shapes whose fp16 activations (T * inner * 2 bytes)
    or weights pass 4 GiB are refused before any device work."""
    import ctypes as C
    from inferno_hip import _lib
    L = _lib.lib()
    fake = C.c_void_p(1 << 20)  # 16-byte aligned, never dereferenced
    T = (1 << 31) // 4096 + 64  # 2 * T * 4096 > 2^32
    rc = L.ihip_prefill_q4_k_dev(fake, fake, fake, fake, T, 4096, 4096, None)
    assert rc == _lib.IHIP_ERR_INVALID
    assert b"4 GiB" in L.ihip_last_error()
    rows = (1 << 32) // (16 * 144) + 8  # weights of 4096 columns past 4 GiB
    rc = L.ihip_prefill_q4_k_dev(fake, fake, fake, fake, 512, 4096, rows, None)
    assert rc == _lib.IHIP_ERR_INVALID


def test_gemv_operands_that_race_are_refused():
    """Every workgroup of a device GEMV reads all of x while rows of out are
    written, so x overlapping out is refused, as is a residual that overlaps
    out without being out; checked before any device work (the pointers are
    never dereferenced, and every call here is refused before a launch)."""
    import ctypes as C
    from inferno_hip import _lib
    L = _lib.lib()
    w = C.c_void_p(1 << 20)
    base = 1 << 24
    x, out = C.c_void_p(base), C.c_void_p(base + 4 * 100)  # 256-float x covers out[0..155]
    assert L.ihip_gemv_dev(12, w, x, out, 256, 64, None) == _lib.IHIP_ERR_INVALID
    assert b"overlaps" in L.ihip_last_error()
    r = C.c_void_p(base + 4 * 1000)
    o = C.c_void_p(base + 4 * 1004)  # out shifted by 4 floats from resid
    assert L.ihip_gemv_add_dev(12, w, x, r, o, 256, 64, None) == _lib.IHIP_ERR_INVALID
    assert b"resid overlaps out" in L.ihip_last_error()
    h = C.c_void_p(base + 4 * 100)  # 64 floats inside x's 256
    assert L.ihip_gate_up_swiglu_dev(12, w, 12, w, x, h, 256, 64, None) == _lib.IHIP_ERR_INVALID
    assert b"x overlaps h" in L.ihip_last_error()
    assert L.ihip_dequantize_dev(12, x, C.c_void_p(base + 64), 256, None) == _lib.IHIP_ERR_INVALID
    assert b"src overlaps dst" in L.ihip_last_error()
    assert L.ihip_prefill_q4_k_f32_dev(w, x, C.c_void_p(base + 16), 2, 256, 64, None) == _lib.IHIP_ERR_INVALID
    assert b"must not overlap" in L.ihip_last_error()


def test_weight_bytes_follow_the_block_layouts():
    """ihip_weight_bytes (the offsets of a weight group's members) against the
    block sizes of the formats (src/QuantsCPU.jl:22-26); no device
    needed."""
    from inferno_hip import _lib, synth
    L = _lib.lib()
    for t in (synth.Q4_K, synth.Q5_K, synth.Q6_K, synth.Q8_0, synth.IQ4_NL):
        e, b = synth.BLOCK_ELEMS[t], synth.BLOCK_BYTES[t]
        for inner, outer in ((e, 1), (4096, 1024), (8 * e, 0), (12288, 4096)):
            assert L.ihip_weight_bytes(t, inner, outer) == outer * (inner // e) * b
        assert L.ihip_weight_bytes(t, e + 1, 4) == 0      # not a whole number of blocks
        assert L.ihip_weight_bytes(t, e, -1) == 0
    assert L.ihip_weight_bytes(99, 256, 4) == 0             # unknown type


def test_no_device_is_an_error_not_a_fallback():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from inferno_hip import QuantizedKernels as QK, _lib
    assert not QK.quant_kernels_available()
    o = np.zeros(1, np.float32)
    with pytest.raises(_lib.IHIPError):
        QK.q4_k_gemv_(o, np.zeros(144, np.uint8), np.zeros(256, np.float32), 256, 1)


# ---- the host-pointer weight cache's staleness guard ----------------------

def _fp(buf: np.ndarray) -> int:
    import ctypes as C
    from inferno_hip import _lib
    out = C.c_uint64(0)
    _lib.check(_lib.lib().ihip_weight_fingerprint(buf.ctypes.data, buf.nbytes, C.byref(out)))
    return out.value


def test_weight_fingerprint_sees_new_bytes_at_the_same_address():
    """The cache reuses a device copy only while the buffer's sampled
    fingerprint is unchanged: a rewrite in place, or other bytes at a reused
    address, changes it; identical bytes elsewhere do not."""
    from inferno_hip import synth
    rng = synth.rng_for(0xF1)
    w = synth.weight(rng, synth.Q4_K, 256, 4096)          # 589824 bytes
    f0 = _fp(w)
    assert _fp(w.copy()) == f0                             # same bytes, other address
    w2 = w.copy()
    w2[:] = synth.weight(rng, synth.Q4_K, 256, 4096)       # another weight, same shape
    assert _fp(w2) != f0
    # a one-byte change inside each sampled window (first, middle, last) is seen
    span = w.nbytes - 16
    for i in (0, 31, 63):
        v = w.copy()
        v[span * i // 63 + 7] ^= 0x40
        assert _fp(v) != f0, i
    # the size is part of it
    assert _fp(w[:-144]) != f0
    # tiny buffers (shorter than one window) work
    t = np.arange(5, dtype=np.uint8)
    assert _fp(t) != _fp(t[:4])


# ---- *_dev entry points use no library-owned device memory ----------------

def _functions(src: str):
    """name -> body of every top-level function definition in a C++ file."""
    out = {}
    for m in re.finditer(r"^[A-Za-z_][\w\s\*&:<>,]*?\b(\w+)\s*\(([^;{]*?)\)\s*\{", src, re.M):
        depth, i = 1, m.end()
        while depth and i < len(src):
            depth += {"{": 1, "}": -1}.get(src[i], 0)
            i += 1
        out[m.group(1)] = src[m.end():i]
    return out


def test_dev_entry_points_touch_no_library_buffers():
    """Scratch on a *_dev path is the caller's: no function reachable from an
    ihip_*_dev entry point reads or writes the library's staging buffers
    (Ctx::x, y, h, t, src, nrm) or its argmax workspace, so calls on different
    streams never share memory and nothing is freed under queued work."""
    src = (ROOT / "inferno.jl_amd" / "csrc" / "api.hip").read_text()
    fns = _functions(src)
    roots = [n for n in fns if n.startswith("ihip_") and n.endswith("_dev")]
    assert sorted(roots) == [s for s in declared_symbols() if s.endswith("_dev")]
    seen, todo = set(), list(roots)
    while todo:
        n = todo.pop()
        if n in seen:
            continue
        seen.add(n)
        for callee in re.findall(r"\b(\w+)\s*\(", fns[n]):
            if callee in fns and callee not in seen:
                todo.append(callee)
    bad = re.compile(r"(\bc\.|ctx\(\)\.)(x|y|h|t|src|nrm|argmax_ws|d_token|d_flags|stream)\b|\bensure\(|\bcopy_in\(")
    for n in sorted(seen):
        hits = bad.findall(fns[n])
        assert not hits, f"{n} (reachable from a *_dev entry point) uses library buffers: {hits}"
    assert "gate_up_dev_locked" in seen and "lm_head_dev_locked" in seen
