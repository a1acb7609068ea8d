"""Write the golden vectors in tests/golden/ from the reference's own C path.

Runs the reference's src/kernels/quant_kernels.c, compiled from its source
file by oracle/Makefile into oracle/_ref/libquant_ref.so, on small seeded
inputs, and stores inputs and outputs as .npz (plain arrays, no pickles):

* ``gauss``   -- x ~ N(0,1): the reference int8-activation GEMV output
                 (q{4,5,6}_k_gemv) or fp32 q8_0_gemv output, plus the Q8_K
                 bytes quantize_row_q8_K makes from x;
* ``intx``    -- integer x in [-127,127] with |x|max = 127 in every
                 256-block, which makes the Q8_K step exact, so the output is
                 the dequantized dot product up to fp32 summation;
* ``onehot``  -- x = 127 at one column c, 0 elsewhere, for a set of columns:
                 output[r] = 127 * W[r, c] up to one fp32 rounding, which pins
                 where each element lives in the block.

Usage:  python tests/golden/make_golden.py      (needs oracle/_ref built)
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "inferno.jl_amd"))

import oracle  # noqa: E402
from inferno_hip import synth  # noqa: E402

SHAPES = {  # type -> (outer, inner)
    synth.Q4_K: (8, 512),
    synth.Q5_K: (8, 512),
    synth.Q6_K: (8, 512),
    synth.Q8_0: (8, 512),
}


def make(ggml_type: int, seed: int) -> dict:
    outer, inner = SHAPES[ggml_type]
    rng = synth.rng_for(seed)
    w = synth.weight(rng, ggml_type, outer, inner)
    # plant fp16 subnormal scales in the first blocks so the fixture covers them
    bb = synth.BLOCK_BYTES[ggml_type]
    sub = np.array([0x0001, 0x03FF, 0x0200, 0x8001], dtype=np.uint16).view(np.uint8)
    if ggml_type in (synth.Q4_K, synth.Q5_K):
        w[0:2] = sub[0:2]          # d of block 0
        w[bb + 2:bb + 4] = sub[2:4]  # dmin of block 1
        w[2 * bb:2 * bb + 2] = sub[4:6]
    elif ggml_type == synth.Q6_K:
        w[208:210] = sub[0:2]
        w[bb + 208:bb + 210] = sub[2:4]
    else:
        w[0:2] = sub[0:2]
        w[bb:bb + 2] = sub[2:4]
        w[2 * bb:2 * bb + 2] = sub[6:8]
    x = synth.activations(rng, inner)
    xi = rng.integers(-127, 128, size=inner).astype(np.float32)
    for b in range(inner // 256 if inner >= 256 else 1):
        xi[b * 256 + int(rng.integers(0, 256))] = 127.0
    cols = np.unique(np.concatenate([np.arange(0, 256), rng.integers(0, inner, 32)]))
    onehot_out = np.empty((len(cols), outer), dtype=np.float32)
    for i, c in enumerate(cols):
        e = np.zeros(inner, dtype=np.float32)
        e[c] = 127.0
        onehot_out[i] = oracle.ref_gemv(ggml_type, w, e, inner, outer)
    d = dict(
        ggml_type=np.int32(ggml_type), outer=np.int32(outer), inner=np.int32(inner),
        w=w, x=x, xi=xi, cols=cols.astype(np.int32),
        ref_gauss=oracle.ref_gemv(ggml_type, w, x, inner, outer),
        ref_intx=oracle.ref_gemv(ggml_type, w, xi, inner, outer),
        ref_onehot=onehot_out,
    )
    if ggml_type != synth.Q8_0:
        d["ref_q8k"] = oracle.ref_quantize_row_q8k(x)
    return d


def main() -> None:
    if oracle.ref_lib() is None:
        raise SystemExit("oracle/_ref/libquant_ref.so is not built (make -C oracle)")
    out = Path(__file__).resolve().parent
    for t, seed in ((synth.Q4_K, 0x40), (synth.Q5_K, 0x50), (synth.Q6_K, 0x60),
                    (synth.Q8_0, 0x80)):
        name = synth.TYPE_NAMES[t].lower()
        np.savez_compressed(out / f"ref_{name}.npz", **make(t, seed))
        print("wrote", out / f"ref_{name}.npz")


if __name__ == "__main__":
    main()
