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


def test_no_device_is_an_error_not_a_fallback():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from inferno_hip import QuantizedKernels as QK, _lib
    assert not QK.quant_kernels_available()
    o = np.zeros(1, np.float32)
    with pytest.raises(_lib.IHIPError):
        QK.q4_k_gemv_(o, np.zeros(144, np.uint8), np.zeros(256, np.float32), 256, 1)
