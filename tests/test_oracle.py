"""Pins the CPU oracle (CPU only, no GPU).

Each check is chosen so that a plausible slip in the restatement (a wrong
element position, a swapped scale/min, a dropped high bit, a wrong fp16
conversion, a tie broken the wrong way) fails it:

* fp16 widening against numpy over all 65536 bit patterns;
* closed forms that the GGML block formats fix (Q8_0 identity, the 6-bit
  scale/min packing as a bijection, one Q5_K high bit per element, Q6_K
  scale slot = element // 16);
* the reference's own C kernels (src/kernels/quant_kernels.c compiled from
  source), through the committed golden vectors: one-hot x pins every element
  position, integer x pins the dot product, Gaussian x pins the int8 lane
  restatement bit for bit;
* the greedy-argmax cases of the reference's tests/unit/test_common_ops.jl.
"""
import numpy as np
import pytest

import oracle
from inferno_hip import synth

TYPES = [synth.Q4_K, synth.Q5_K, synth.Q6_K, synth.Q8_0]
NAMES = {t: synth.TYPE_NAMES[t].lower() for t in TYPES}


# ---------------------------------------------------------------- fp16 ----

def test_half_to_float_all_patterns():
    # Q8_0 blocks with q[0] = 1 dequantize to exactly d: convert every half.
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    blocks = np.zeros((65536, 34), dtype=np.uint8)
    blocks[:, 0:2] = h.view(np.uint8).reshape(-1, 2)
    blocks[:, 2] = 1
    y = oracle.dequant(synth.Q8_0, blocks.reshape(-1), 65536 * 32).reshape(65536, 32)
    got = y[:, 0]
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # q = 0 gives +0 or -0 by the sign of d; never NaN unless d is NaN/Inf
    assert np.all(y[~nan & np.isfinite(want), 1] == 0)


def test_float_to_half_rne_matches_numpy():
    rng = np.random.default_rng(5)
    edge = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 70000.0, 2.0**-24, 2.0**-25,
                     3 * 2.0**-26, 2.0**-14, 2.0**-14 * (1 - 2**-11), 1.0 + 2**-11,
                     1.0 + 3 * 2**-11, np.inf, -np.inf, 1e-30], dtype=np.float32)
    vals = np.concatenate([edge, rng.standard_normal(20000).astype(np.float32),
                           (rng.standard_normal(20000) * 1e-5).astype(np.float32),
                           (rng.standard_normal(5000) * 3e4).astype(np.float32)])
    got = np.array([oracle.float_to_half(float(v)) for v in vals], dtype=np.uint16)
    want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ------------------------------------------------------- closed forms ----

def test_q8_0_identity_and_subnormal_scale():
    q = np.arange(-127, 128, dtype=np.int16)
    q = np.resize(q, 32 * 8).astype(np.int8)
    blocks = np.zeros((8, 34), dtype=np.uint8)
    blocks[:4, 0:2] = np.array([0x3C00], np.uint16).view(np.uint8)   # d = 1
    blocks[4:, 0:2] = np.array([0x0001], np.uint16).view(np.uint8)   # d = 2^-24
    blocks[:, 2:] = q.view(np.uint8).reshape(8, 32)
    y = oracle.dequant(synth.Q8_0, blocks.reshape(-1), 256).reshape(8, 32)
    assert np.array_equal(y[:4], q.reshape(8, 32)[:4].astype(np.float32))
    assert np.array_equal(y[4:], q.reshape(8, 32)[4:].astype(np.float32) * np.float32(2.0**-24))


def pack_k_scales(sc, m):
    """GGML K-quant 12-byte packing of eight 6-bit scales and eight 6-bit mins:
    bytes 0-3 carry sc0-3 in their low 6 bits and the top 2 bits of sc4-7;
    bytes 4-7 carry m0-3 and the top 2 bits of m4-7; bytes 8-11 carry the low
    nibbles of sc4-7 (low half) and m4-7 (high half)."""
    s = np.zeros(12, dtype=np.uint8)
    for k in range(4):
        s[k] = (sc[k] & 63) | ((sc[4 + k] >> 4) << 6)
        s[4 + k] = (m[k] & 63) | ((m[4 + k] >> 4) << 6)
        s[8 + k] = (sc[4 + k] & 0xF) | ((m[4 + k] & 0xF) << 4)
    return s


@pytest.mark.parametrize("t", [synth.Q4_K, synth.Q5_K])
def test_k_scale_min_bijection(t):
    rng = np.random.default_rng(11)
    bb = synth.BLOCK_BYTES[t]
    n = 64
    scb = rng.integers(0, 256, size=(n, 12), dtype=np.uint8)
    one = np.array([0x3C00], np.uint16).view(np.uint8)
    # (a) d = 1, dmin = 0, every 4-bit quant = 1, high bits 0 -> y = sc
    a = np.zeros((n, bb), dtype=np.uint8)
    a[:, 0:2] = one
    a[:, 4:16] = scb
    a[:, bb - 128:] = 0x11
    ya = oracle.dequant(t, a.reshape(-1), n * 256).reshape(n, 8, 32)
    # (b) d = 0, dmin = 1, all quants 0 -> y = -m
    b = np.zeros((n, bb), dtype=np.uint8)
    b[:, 2:4] = one
    b[:, 4:16] = scb
    yb = oracle.dequant(t, b.reshape(-1), n * 256).reshape(n, 8, 32)
    for i in range(n):
        assert np.all(ya[i] == ya[i][:, :1]) and np.all(yb[i] == yb[i][:, :1])
        sc = ya[i][:, 0].astype(np.int64)
        m = (-yb[i][:, 0]).astype(np.int64)
        assert sc.min() >= 0 and sc.max() <= 63 and m.min() >= 0 and m.max() <= 63
        assert np.array_equal(pack_k_scales(sc, m), scb[i])


def test_q5_k_high_bit_positions():
    # one qh bit per block: bit b of qh[l] must add 16 to element 32*b + l only
    blocks = np.zeros((256, 176), dtype=np.uint8)
    blocks[:, 0:2] = np.array([0x3C00], np.uint16).view(np.uint8)
    blocks[:, 4:16] = pack_k_scales(np.ones(8, np.int64), np.zeros(8, np.int64))
    for e in range(256):
        b, l = divmod(e, 32)
        blocks[e, 16 + l] = 1 << b
    y = oracle.dequant(synth.Q5_K, blocks.reshape(-1), 256 * 256).reshape(256, 256)
    assert np.array_equal(y, 16 * np.eye(256, dtype=np.float32))


def test_q6_k_scale_slot_is_element_div_16():
    primes = np.array([2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, -2, -3, -5, -7, -11], np.int8)
    blk = np.zeros(210, dtype=np.uint8)
    blk[0:128] = 0x55          # low nibbles 5, high nibbles 5
    blk[128:192] = 0xAA        # every 2-bit pair = 2 -> q = 5 | 2<<4 = 37
    blk[192:208] = primes.view(np.uint8)
    blk[208:210] = np.array([0x3C00], np.uint16).view(np.uint8)
    y = oracle.dequant(synth.Q6_K, blk, 256)
    want = np.repeat(primes.astype(np.float32), 16) * (37 - 32)
    assert np.array_equal(y, want)


def test_gemv_f64_row_layout_matches_numpy():
    rng = synth.rng_for(3)
    for t in TYPES:
        outer, inner = 24, 1024
        w = synth.weight(rng, t, outer, inner)
        x = synth.activations(rng, inner)
        W = oracle.dequant(t, w, outer * inner).reshape(outer, inner).astype(np.float64)
        assert np.allclose(oracle.gemv_f64(t, w, x, inner, outer), W @ x, rtol=1e-12, atol=1e-12)
        nrm = oracle.row_norms(t, w, inner, outer)
        assert np.allclose(nrm, np.linalg.norm(W, axis=1), rtol=1e-12)
        # the Julia fallback's serial fp32 sum stays inside the parity bound
        s = oracle.gemv_f32_serial(t, w, x, inner, outer)
        assert np.all(np.abs(s - W @ x) <= oracle.tolerance(nrm, x))


@pytest.mark.parametrize("t", TYPES + [synth.IQ4_NL])
def test_gemv_f32_serial_bits(t):
    """src/ModelCPU.jl:290-306 fixes the bits of the fallback: `sum_val +=
    block_values[i] * x[col_idx]` rounds each product to fp32 and adds it to a
    single fp32 accumulator in column order (Julia does not contract `a += b*c`
    into an FMA).  numpy's accumulate over fp32-rounded products is that
    sequential sum; an fp64 accumulator, a fused multiply-add or a pairwise or
    lane-split sum each change the last bits of some rows."""
    rng = synth.rng_for(0x5E + t)
    outer, inner = 96, 4096 if t != synth.Q8_0 else 2048
    w = synth.weight(rng, t, outer, inner)
    x = synth.activations(rng, inner) * np.float32(rng.uniform(0.5, 8))
    W = oracle.dequant(t, w, outer * inner).reshape(outer, inner)
    prods = W * x[None, :]                              # fp32 products, each rounded once
    want = np.add.accumulate(prods, axis=1, dtype=np.float32)[:, -1]
    got = oracle.gemv_f32_serial(t, w, x, inner, outer)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # the pin discriminates: an fp64 accumulator rounded once differs somewhere
    f64 = (W.astype(np.float64) @ x.astype(np.float64)).astype(np.float32)
    assert not np.array_equal(f64.view(np.uint32), want.view(np.uint32))


def test_gemm_f64_is_the_per_token_gemv():
    """The prefill oracle (src/ModelCPU.jl:1001-1017: one GEMV per token) must
    give, for every token, exactly the GEMV oracle's fp64 sums: same products,
    same column order.  Ragged shapes exercise the 8-row groups' tail."""
    rng = synth.rng_for(0x61)
    for t, T, outer, inner in ((synth.Q4_K, 7, 37, 512), (synth.Q6_K, 5, 16, 256),
                               (synth.Q8_0, 3, 9, 96), (synth.Q5_K, 1, 8, 256),
                               (synth.Q4_K, 0, 8, 256)):
        w = synth.weight(rng, t, outer, inner)
        X = rng.standard_normal((T, inner)).astype(np.float32)
        Y = oracle.gemm_f64(t, w, X, inner, outer)
        assert Y.shape == (T, outer)
        for k in range(T):
            assert np.array_equal(Y[k], oracle.gemv_f64(t, w, X[k], inner, outer)), (t, k)


def test_ffn_oracle_composition():
    rng = synth.rng_for(9)
    hidden, inter = 512, 768
    wg = synth.weight(rng, synth.Q4_K, inter, hidden)
    wu = synth.weight(rng, synth.Q4_K, inter, hidden)
    wd = synth.weight(rng, synth.Q6_K, hidden, inter)
    x = synth.activations(rng, hidden)
    g, u, h, y = oracle.ffn_swiglu_f64(synth.Q4_K, wg, synth.Q4_K, wu, synth.Q6_K, wd, x,
                                       hidden, inter)
    g2 = oracle.gemv_f64(synth.Q4_K, wg, x, hidden, inter)
    u2 = oracle.gemv_f64(synth.Q4_K, wu, x, hidden, inter)
    assert np.array_equal(g, g2) and np.array_equal(u, u2)
    h2 = g2 / (1 + np.exp(-g2)) * u2
    assert np.allclose(h, h2, rtol=1e-14)
    Wd = oracle.dequant(synth.Q6_K, wd, hidden * inter).reshape(hidden, inter).astype(np.float64)
    assert np.allclose(y, Wd @ h2, rtol=1e-10, atol=1e-9)


# ------------------------------------------- the reference's own C path ----

def _golden(golden_dir, t):
    return dict(np.load(golden_dir / f"ref_{NAMES[t]}.npz", allow_pickle=False))


def _block_scale_bound(t, w, outer, inner):
    """Per-element bound on one or two fp32 roundings of the reference's
    one-hot output, from the block's own d/dmin."""
    bb, be = synth.BLOCK_BYTES[t], synth.BLOCK_ELEMS[t]
    blocks = w.reshape(-1, bb)
    if t == synth.Q6_K:
        d = np.abs(blocks[:, 208:210].copy().view(np.float16).astype(np.float64)).ravel()
        mag = d * 32 * 32
    elif t == synth.Q8_0:
        d = np.abs(blocks[:, 0:2].copy().view(np.float16).astype(np.float64)).ravel()
        mag = d * 127
    else:
        d = np.abs(blocks[:, 0:2].copy().view(np.float16).astype(np.float64)).ravel()
        dm = np.abs(blocks[:, 2:4].copy().view(np.float16).astype(np.float64)).ravel()
        mag = d * 63 * 31 + dm * 63
    per_elem = np.repeat(mag, be).reshape(outer, inner)
    return 4 * 2.0**-24 * per_elem


@pytest.mark.parametrize("t", TYPES)
def test_onehot_pins_element_positions(golden_dir, t):
    g = _golden(golden_dir, t)
    outer, inner = int(g["outer"]), int(g["inner"])
    W = oracle.dequant(t, g["w"], outer * inner).reshape(outer, inner).astype(np.float64)
    bound = _block_scale_bound(t, g["w"], outer, inner)
    for i, c in enumerate(g["cols"]):
        got = g["ref_onehot"][i].astype(np.float64) / 127.0
        assert np.all(np.abs(got - W[:, c]) <= bound[:, c] + 1e-30), f"column {c}"


@pytest.mark.parametrize("t", TYPES)
def test_integer_x_matches_reference(golden_dir, t):
    g = _golden(golden_dir, t)
    outer, inner = int(g["outer"]), int(g["inner"])
    o = oracle.gemv_f64(t, g["w"], g["xi"], inner, outer)
    nrm = oracle.row_norms(t, g["w"], inner, outer)
    assert np.all(np.abs(g["ref_intx"] - o) <= 1e-6 * nrm * np.linalg.norm(g["xi"]))


@pytest.mark.parametrize("t", TYPES)
def test_int8_lane_restatement_bit_exact(golden_dir, t):
    g = _golden(golden_dir, t)
    outer, inner = int(g["outer"]), int(g["inner"])
    if t == synth.Q8_0:
        got = oracle.gemv_q8_0_lanes(g["w"], g["x"], inner, outer)
    else:
        assert np.array_equal(oracle.quantize_row_q8k(g["x"]), g["ref_q8k"])
        got = oracle.gemv_q8k(t, g["w"], g["x"], inner, outer)
    assert np.array_equal(got.view(np.uint32), g["ref_gauss"].view(np.uint32))


@pytest.mark.skipif(oracle.ref_lib() is None, reason="oracle/_ref not built")
@pytest.mark.parametrize("t", TYPES)
def test_int8_lane_restatement_vs_compiled_reference(t):
    rng = synth.rng_for(0x77 + t)
    for outer, inner in ((33, 256), (7, 2048), (64, 4096)):
        w = synth.weight(rng, t, outer, inner)
        x = synth.activations(rng, inner) * np.float32(rng.uniform(0.1, 30))
        if t == synth.Q8_0:
            got = oracle.gemv_q8_0_lanes(w, x, inner, outer)
        else:
            got = oracle.gemv_q8k(t, w, x, inner, outer)
        ref = oracle.ref_gemv(t, w, x, inner, outer)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_int8_path_is_not_the_tolerance_oracle():
    # The reference C path quantizes x to int8 and leaves the 1e-4 bound on
    # a 4096-wide Q4_K row, which is why the fp32-x semantics is the oracle.
    rng = synth.rng_for(0xC0)
    outer, inner = 256, 4096
    w = synth.weight(rng, synth.Q4_K, outer, inner)
    x = synth.activations(rng, inner)
    o = oracle.gemv_f64(synth.Q4_K, w, x, inner, outer)
    tol = oracle.tolerance(oracle.row_norms(synth.Q4_K, w, inner, outer), x)
    q = oracle.gemv_q8k(synth.Q4_K, w, x, inner, outer)
    assert np.max(np.abs(q - o) / tol) > 1.0


# -------------------------------------------------------------- argmax ----

def test_argmax_reference_cases():
    ninf = -np.inf
    # tests/unit/test_common_ops.jl:85-93 (1-based there, 0-based here)
    assert oracle.argmax(np.array([ninf, ninf], np.float32)) == (0, True)
    for bad in ([1, np.inf], [1, np.nan]):
        with pytest.raises(ValueError):
            oracle.argmax(np.array(bad, np.float32))
    with pytest.raises(ValueError):
        oracle.argmax(np.array([], np.float32))
    # greedy softmax_sample(temperature=0) on 0..5 picks the last (test :61-62)
    assert oracle.argmax(np.arange(6, dtype=np.float32))[0] == 5
    assert oracle.argmax(np.array([ninf, 0, ninf, 1], np.float32))[0] == 3
    assert oracle.argmax(np.array([3, 7, 7, 1], np.float32))[0] == 1
    assert oracle.argmax(np.array([-0.0, 0.0], np.float32))[0] == 0


def test_argmax_matches_numpy_first_occurrence():
    rng = np.random.default_rng(2)
    for n in (1, 2, 31, 32, 33, 1000, 151936):
        v = rng.integers(-50, 50, size=n).astype(np.float32)
        assert oracle.argmax(v)[0] == int(np.argmax(v))


# ---- rmsnorm and the decoder MLP half (src/ModelCPU.jl:111-123, 913-920) ----

def test_rmsnorm_oracle_properties():
    rng = np.random.default_rng(0x4E)
    x = rng.standard_normal(4096).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 4096).astype(np.float32)
    one = np.ones(4096, np.float32)
    # eps = 0: invariant under exact power-of-two scaling of x (a missing root
    # or a sum instead of a mean breaks it)
    a = oracle.rmsnorm_f64(x, w, 0.0)
    assert np.array_equal(a, oracle.rmsnorm_f64(x * np.float32(4.0), w, 0.0))
    # unit weights, eps = 0: mean of squares is 1
    assert abs(np.mean(oracle.rmsnorm_f64(x, one, 0.0) ** 2) - 1.0) < 1e-12
    # constant input c: c / sqrt(c^2 + eps) * w, elementwise
    c, eps = np.float32(0.37), np.float32(1e-2)
    got = oracle.rmsnorm_f64(np.full(64, c, np.float32), w[:64], float(eps))
    want = float(c) / np.sqrt(float(c) ** 2 + float(eps)) * w[:64].astype(np.float64)
    assert np.allclose(got, want, rtol=1e-14, atol=0)


def test_ffn_block_oracle_is_norm_then_ffn_then_residual():
    rng = synth.rng_for(0x4F)
    hidden, inter = 512, 768
    wg = synth.weight(rng, synth.Q4_K, inter, hidden)
    wu = synth.weight(rng, synth.Q4_K, inter, hidden)
    wd = synth.weight(rng, synth.Q6_K, hidden, inter) if inter % 2048 == 0 else \
        synth.weight(rng, synth.Q8_0, hidden, inter)
    dt = synth.Q6_K if inter % 2048 == 0 else synth.Q8_0
    x = synth.activations(rng, hidden) * np.float32(3.0)
    nw = rng.uniform(0.5, 1.5, hidden).astype(np.float32)
    n, g, u, h, y = oracle.ffn_block_f64(synth.Q4_K, wg, synth.Q4_K, wu, dt, wd, x, nw, 1e-6,
                                         hidden, inter)
    assert np.array_equal(n, oracle.rmsnorm_f64(x, nw, 1e-6))
    # the same FFN on the fp32-rounded normed input, plus the residual
    g2, u2, h2, y2 = oracle.ffn_swiglu_f64(synth.Q4_K, wg, synth.Q4_K, wu, dt, wd,
                                           n.astype(np.float32), hidden, inter)
    nrm = oracle.row_norms(dt, wd, inter, hidden)
    assert np.all(np.abs((y - x) - y2) <= 1e-5 * nrm * np.linalg.norm(h2))


# ---- IQ4_NL (src/Dequant.jl:655-693; grid src/QuantsData.jl:384) ----

def test_iq4_nl_oracle_reference_known_answers():
    """tests/unit/core_components.jl:177-205 of the reference, case by case."""
    def block(d_bits, qs0):
        b = np.zeros(18, np.uint8)
        b[0:2] = np.array([d_bits], np.uint16).view(np.uint8)
        b[2] = qs0
        return b
    y = oracle.dequant(synth.IQ4_NL, block(0x3C00, 0), 32)
    assert np.all(y == np.float32(-127.0))
    y = oracle.dequant(synth.IQ4_NL, block(0x3C00, 0x18), 32)
    assert (y[0], y[16], y[15], y[31]) == (1.0, -104.0, -127.0, -127.0)
    y = oracle.dequant(synth.IQ4_NL, block(0x4000, 0x18), 32)
    assert (y[0], y[16]) == (2.0, -208.0)
    y = oracle.dequant(synth.IQ4_NL, block(0x3C00, 0b1110_1011), 32)
    assert (y[0], y[16]) == (38.0, 89.0)
    # the whole grid, in nibble order, sorted and distinct (the reference's
    # table checks, core_components.jl:254-256)
    grid = [oracle.dequant(synth.IQ4_NL, block(0x3C00, v), 32)[0] for v in range(16)]
    assert grid[0] == -127 and grid[-1] == 113 and grid == sorted(grid) and len(set(grid)) == 16
