"""The Julia drop-in (julia/InfernoHIP.jl) binds the library it claims to.

Julia is not installed here, so this is a text check: every
`ccall((:ihip_..., LIBIHIP), Ret, (T1, ..., Tn), args...)` in the file names
a symbol that include/inferno_hip.h declares, with as many argument types as
the declaration has parameters and as many arguments as types; and the
modules export the reference's function names (src/QuantizedKernels.jl:14-16,
src/FusedKernels.jl:14-16, src/Dequant.jl:5-6).
"""
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
JL = ROOT / "julia" / "InfernoHIP.jl"
HEADER = ROOT / "include" / "inferno_hip.h"


def header_arity():
    return {k: v[1] for k, v in header_decls().items()}


def header_decls():
    """ihip_* name -> (Julia return type, parameter count) from the header."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    jl = {"int": "Cint", "size_t": "Csize_t", "const char *": "Cstring"}
    out = {}
    for m in re.finditer(r"^([A-Za-z_][\w ]*?\s*\**)\s*\b(ihip_\w+)\s*\(([^;{]*?)\)\s*;", text, re.S | re.M):
        params = m.group(3).strip()
        ret = re.sub(r"\s+", " ", m.group(1).strip()).replace(" *", " *")
        out[m.group(2)] = (jl.get(ret, ret), 0 if params in ("", "void") else len(_split(params)))
    return out


def _split(s):
    """Top-level comma split (brackets and braces nest)."""
    parts, depth, cur = [], 0, ""
    for ch in s:
        if ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
        if ch == "," and depth == 0:
            parts.append(cur)
            cur = ""
        else:
            cur += ch
    if cur.strip():
        parts.append(cur)
    return [p.strip() for p in parts if p.strip()]


def _balanced(text, i):
    """text[i] == '(' -> index just past its matching ')'."""
    depth = 0
    for j in range(i, len(text)):
        if text[j] == "(":
            depth += 1
        elif text[j] == ")":
            depth -= 1
            if depth == 0:
                return j + 1
    raise AssertionError("unbalanced parentheses")


def ccalls(lib="LIBIHIP"):
    text = JL.read_text()
    out = []
    for m in re.finditer(r"ccall\(", text):
        end = _balanced(text, m.end() - 1)
        args = _split(text[m.end():end - 1])
        sym = re.fullmatch(r"\(:(\w+),\s*(\w+)\)", args[0])
        assert sym, args[0]
        types = args[2]
        assert types.startswith("(") and types.endswith(")"), types
        tlist = _split(types[1:-1])
        out.append((sym.group(1), sym.group(2), args[1], tlist, args[3:]))
    return out


def test_every_library_ccall_matches_the_header():
    decls = header_decls()
    calls = [c for c in ccalls() if c[1] == "LIBIHIP"]
    assert len(calls) >= 15
    for sym, _, ret, types, args in calls:
        assert sym in decls, f"{sym} is not declared in include/inferno_hip.h"
        want, n = decls[sym]
        assert len(types) == n, f"{sym}: {len(types)} argument types, header has {n}"
        assert len(args) == len(types), f"{sym}: {len(args)} arguments for {len(types)} types"
        assert ret == want, f"{sym} returns {ret}, the header says {want}"


def test_hip_runtime_calls_are_the_documented_ones():
    hip = {c[0] for c in ccalls() if c[1] == "LIBHIP"}
    assert hip <= {"hipMalloc", "hipFree", "hipMemcpy", "hipStreamSynchronize"}, hip


def test_modules_export_the_reference_names():
    text = JL.read_text()
    mods = {}
    for name in ("QuantizedKernels", "Dequant", "FusedKernels", "Device", "GGUF"):
        m = re.search(r"^module " + name + r"\n(.*?)^end # module " + name, text, re.S | re.M)
        assert m, name
        mods[name] = m.group(1)
    exports = {m: set(re.findall(r"(\w+!?)", " ".join(re.findall(r"^export (.*)$", body, re.M))))
               for m, body in mods.items()}
    assert {"quant_kernels_available", "q4_k_gemv!", "q5_k_gemv!", "q6_k_gemv!", "q8_0_gemv!",
            "quantize_q8_k!", "vec_dot_q4_k_q8_k", "vec_dot_q5_k_q8_k",
            "vec_dot_q6_k_q8_k"} <= exports["QuantizedKernels"]
    assert {"dequantize_q8_0", "dequantize_q4_k", "dequantize_q5_k",
            "dequantize_q6_k"} <= exports["Dequant"]
    assert {"fused_mlp_gate_mul!", "fused_silu_gate_mul!", "gpu_argmax!"} <= exports["FusedKernels"]
    # every exported name is defined in its module (a function or a const)
    for m, names in exports.items():
        for n in names:
            assert re.search(r"(function\s+|^)" + re.escape(n) + r"\s*\(", mods[m], re.M) or \
                re.search(r"^const\s+" + re.escape(n) + r"\s*=", mods[m], re.M), (m, n)
    # the opt-in C numerics reach the int8-activation entry points
    assert {"q4_k_gemv_q8k!", "q5_k_gemv_q8k!", "q6_k_gemv_q8k!", "EXACT_C_NUMERICS"} <= exports["QuantizedKernels"]


def test_julia_source_is_structurally_balanced():
    """No Julia parser here: check the block structure (every module/function/
    if/for/begin/let/struct closes) and bracket balance."""
    text = JL.read_text()
    code = re.sub(r'""".*?"""', '""', text, flags=re.S)
    code = re.sub(r'"(\\.|[^"\\])*"', '""', code)
    code = re.sub(r"#.*", "", code)
    for a, b in ("()", "[]", "{}"):
        assert code.count(a) == code.count(b), (a, b)
    opens = len(re.findall(r"^\s*(module|function|if|for|while|begin|let|struct|mutable struct)\b",
                           code, re.M))
    opens += len(re.findall(r"^\s*\w[^=\n]*=\s*(if|begin|let)\b", code, re.M))
    opens += len(re.findall(r"^\s*(?:\w+\.)?@\w+[^\n]*\bbegin\s*$", code, re.M))  # GC.@preserve x begin
    ends = len(re.findall(r"^\s*end\b", code, re.M))
    assert opens == ends, (opens, ends)
