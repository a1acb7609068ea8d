"""GPU parity: the gfx950 kernels against the CPU oracle on seeded inputs.

Bars (the reference CPU semantics restated in oracle/):
* standalone dequant: bit-exact;
* fp32-accumulated GEMV / GEMM: |y - y_ref| <= 1e-4 * ||w_row||_2 * ||x||_2,
  y_ref accumulated in fp64 over the exact dequantized weights;
* argmax token ids: bit-exact (lowest index of the maximum).
Every call goes through the C ABI (libinferno_hip.so).
"""
import numpy as np
import pytest

import oracle
from inferno_hip import synth

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def say(*a):
    print("[case]", *a, flush=True)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from inferno_hip import _lib
    assert _lib.available(), "libinferno_hip.so reports no usable gfx950 device"
    yield
    torch.cuda.synchronize()


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.to("cuda") if dtype is None else t.to("cuda", dtype)


def dweight(w, t, inner, outer):
    from inferno_hip.device import DeviceWeight
    return DeviceWeight(dev(w), t, inner, outer)


def assert_within(y, ref, tol, what):
    err = np.abs(np.asarray(y, np.float64) - ref)
    ratio = float(np.max(err / tol))
    say(f"{what}: max err/tol = {ratio:.3e}")
    assert np.all(err <= tol), f"{what}: {np.sum(err > tol)} outputs over tolerance (max ratio {ratio})"


# ------------------------------------------------------------- dequant ----

def test_dequant_all_half_patterns_bit_exact():
    say("dequant Q8_0: all 65536 fp16 scale patterns")
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    blocks = np.zeros((65536, 34), dtype=np.uint8)
    blocks[:, 0:2] = h.view(np.uint8).reshape(-1, 2)
    blocks[:, 2:34] = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
    n = 65536 * 32
    from inferno_hip import device as D
    got = D.dequantize(dweight(blocks.reshape(-1), synth.Q8_0, n, 1)).cpu().numpy()
    want = oracle.dequant(synth.Q8_0, blocks.reshape(-1), n)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t,outer,inner", [
    (synth.Q8_0, 4096, 4096),   # the standalone-dequant workload, full size
    (synth.Q4_K, 1024, 4096),
    (synth.Q5_K, 512, 4096),
    (synth.Q6_K, 512, 2048),
    (synth.Q6_K, 3, 768),       # 9 blocks: not a multiple of 8 -> generic path
    (synth.Q8_0, 5, 96),        # 15 blocks -> generic path
    (synth.Q4_K, 1, 256),
    (synth.IQ4_NL, 1024, 4096),
    (synth.IQ4_NL, 3, 96),
])
def test_dequant_bit_exact(t, outer, inner):
    say(f"dequant type={t} {outer}x{inner}")
    rng = synth.rng_for(1000 + t + inner)
    w = synth.weight(rng, t, outer, inner)
    from inferno_hip import device as D
    got = D.dequantize(dweight(w, t, inner, outer)).cpu().numpy()
    want = oracle.dequant(t, w, outer * inner)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t", [synth.Q4_K, synth.Q5_K, synth.Q6_K, synth.Q8_0, synth.IQ4_NL])
def test_dequant_host_entry_point_and_misaligned_source(t):
    say(f"Dequant host mirror type={t}")
    from inferno_hip import Dequant, device as D
    rng = synth.rng_for(77 + t)
    inner = 2048
    w = synth.weight(rng, t, 4, inner)
    want = oracle.dequant(t, w, 4 * inner)
    got = Dequant.dequantize(t, w, 4 * inner)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # a source that starts 2 bytes past a 16-byte boundary takes the generic kernel
    buf = torch.zeros(w.size + 16, dtype=torch.uint8, device="cuda")
    buf[2:2 + w.size] = dev(w)
    dw = D.DeviceWeight(buf[2:2 + w.size], t, inner, 4)
    got2 = D.dequantize(dw).cpu().numpy()
    assert np.array_equal(got2.view(np.uint32), want.view(np.uint32))


def test_dequant_iq4_nl_reference_known_answers():
    """The IQ4_NL cases of the reference's tests/unit/core_components.jl:177-205."""
    from inferno_hip import Dequant
    blocks = np.zeros((4, 18), np.uint8)
    for i, (d_bits, qs0) in enumerate(((0x3C00, 0), (0x3C00, 0x18), (0x4000, 0x18),
                                       (0x3C00, 0b1110_1011))):
        blocks[i, 0:2] = np.array([d_bits], np.uint16).view(np.uint8)
        blocks[i, 2] = qs0
    say("IQ4_NL known answers")
    y = Dequant.dequantize_iq4_nl(blocks.reshape(-1), 128).reshape(4, 32)
    assert np.all(y[0] == -127.0)
    assert (y[1, 0], y[1, 16], y[1, 15], y[1, 31]) == (1.0, -104.0, -127.0, -127.0)
    assert (y[2, 0], y[2, 16]) == (2.0, -208.0)
    assert (y[3, 0], y[3, 16]) == (38.0, 89.0)


def test_iq4_nl_gemv_host_mirror():
    from inferno_hip import QuantizedKernels as QK
    rng = synth.rng_for(0x1A4)
    outer, inner = 257, 1024
    w = synth.weight(rng, synth.IQ4_NL, outer, inner)
    x = synth.activations(rng, inner)
    say("iq4_nl_gemv_ host mirror")
    out = np.zeros(outer, np.float32)
    QK.iq4_nl_gemv_(out, w, x, inner, outer)
    ref = oracle.gemv_f64(synth.IQ4_NL, w, x, inner, outer)
    assert_within(out, ref, oracle.tolerance(oracle.row_norms(synth.IQ4_NL, w, inner, outer), x),
                  "IQ4_NL host mirror")


# ---------------------------------------------------------------- GEMV ----

GEMV_CASES = [
    (synth.Q4_K, 4096, 4096),     # the headline decode GEMV
    (synth.Q4_K, 12288, 4096),    # FFN gate/up shape
    (synth.Q4_K, 37, 2304),       # ragged rows, partial 2048-column segment
    (synth.Q4_K, 1, 256),
    (synth.Q5_K, 4096, 4096),
    (synth.Q5_K, 9, 768),
    (synth.Q6_K, 4096, 12288),    # FFN down shape
    (synth.Q6_K, 300, 2048),
    (synth.Q6_K, 151936, 2048),   # the lm_head shape as a plain GEMV (one segment, staged digits)
    (synth.Q6_K, 7, 768),         # rows of 630 bytes: segments at byte phases (streamed kernel)
    (synth.Q8_0, 4096, 4096),
    (synth.Q8_0, 11, 2304),       # partial 64-block segment
    (synth.Q8_0, 6, 96),          # 3 blocks a row, at byte phases
    (synth.IQ4_NL, 2048, 1024),   # an SSM-projection-sized IQ4_NL matrix
    (synth.IQ4_NL, 1000, 4096),   # two 64-block segments per row
    (synth.IQ4_NL, 13, 2304),     # partial segment (72 blocks)
    (synth.IQ4_NL, 5, 96),        # 3 blocks a row, at byte phases
    (synth.Q4_K, 1536, 4096),     # one GPU's gate/up rows of the FFN over 8 GPUs
    (synth.Q6_K, 4096, 1536),     # one GPU's down-projection columns (6 blocks a row)
    (synth.Q4_K, 300, 5120),      # 16 + 4 blocks: persistent multi-pass kernel, 2-pass capacity
    (synth.Q5_K, 77, 11008),      # 43 blocks: 3 passes, the last partial (4-pass capacity)
    (synth.Q4_K, 2000, 13824),    # 54 blocks, many row groups per wave
    (synth.Q4_K, 64, 28672),      # 112 blocks: 7 passes (8-pass capacity)
    (synth.Q4_K, 10, 33024),      # 129 blocks: past the persistent kernel, serial passes
    (synth.Q4_K, 4096, 5120),     # 256 workgroups over 256 CUs: serial passes, the last partial
    (synth.IQ4_NL, 8200, 2048),   # IQ4_NL in the persistent wide kernel
    (synth.IQ4_NL, 4096, 4096),   # IQ4_NL in the wide kernel, one workgroup per CU
    (synth.Q8_0, 8200, 2048),     # Q8_0 in the persistent wide kernel
    (synth.Q8_0, 1024, 4096),     # Q8_0 in the wide kernel, one row per wave
]


@pytest.mark.parametrize("t,outer,inner", GEMV_CASES)
def test_gemv_device(t, outer, inner):
    say(f"gemv_dev type={t} {outer}x{inner}")
    rng = synth.rng_for(0xC0 + t * 7 + inner + outer)
    w = synth.weight(rng, t, outer, inner)
    x = synth.activations(rng, inner)
    from inferno_hip import device as D
    y = D.gemv(dweight(w, t, inner, outer), dev(x)).cpu().numpy()
    ref = oracle.gemv_f64(t, w, x, inner, outer)
    tol = oracle.tolerance(oracle.row_norms(t, w, inner, outer), x)
    assert_within(y, ref, tol, f"type {t} {outer}x{inner}")


@pytest.mark.parametrize("t", [synth.Q4_K, synth.Q5_K, synth.Q6_K, synth.Q8_0])
def test_gemv_host_mirror_and_weight_cache(t):
    from inferno_hip import QuantizedKernels as QK
    fn = {synth.Q4_K: QK.q4_k_gemv_, synth.Q5_K: QK.q5_k_gemv_, synth.Q6_K: QK.q6_k_gemv_,
          synth.Q8_0: QK.q8_0_gemv_}[t]
    rng = synth.rng_for(5 + t)
    outer, inner = 256, 4096
    w = synth.weight(rng, t, outer, inner)
    tol_n = oracle.row_norms(t, w, inner, outer)
    for rep in range(3):  # same weight buffer, new x: the cached device copy is reused
        say(f"host mirror type={t} rep={rep}")
        x = synth.activations(rng, inner) * np.float32(10.0 ** (rep - 1))
        out = np.zeros(outer, np.float32)
        fn(out, w, x, inner, outer)
        assert_within(out, oracle.gemv_f64(t, w, x, inner, outer), oracle.tolerance(tol_n, x),
                      f"host type {t} rep {rep}")
    # new bytes in the same host buffer: forget() drops the stale device copy
    w[:] = synth.weight(rng, t, outer, inner)
    QK.forget(w)
    x = synth.activations(rng, inner)
    out = np.zeros(outer, np.float32)
    fn(out, w, x, inner, outer)
    assert_within(out, oracle.gemv_f64(t, w, x, inner, outer),
                  oracle.tolerance(oracle.row_norms(t, w, inner, outer), x), "after forget")


# Shapes that reach every launch the host makes (one instantiation each):
#   Q4_K / Q5_K wide kernel, two rows per wave: ragged row counts, 1..9
#     passes of 4096 columns, the last one partial;
#   the persistent wide kernel: >= 8192 rows of at most 4096 columns;
#   the streamed digit kernel: 8 waves for one segment of 2048 columns and
#     for 7..8 Q8_0 segments, 12 waves for 2..6 (staged digits shared by two
#     or more waves of a segment) and 9..12, 16 waves for 7..8 Q6_K / IQ4_NL
#     segments and 13..16 (waves past the segments idle), partial last
#     segments, chunks that end inside a workgroup's last round;
#   rows that are not 16-byte multiples (Q6_K rows of any block count, Q8_0 and
#     IQ4_NL rows of any multiple of 32 columns): segments copied from the
#     unit below them, at byte phases 2..14, 1 to 16 segments;
#   rows past 16 segments: the byte-granular kernel.
LAUNCH_SHAPES = [
    (synth.Q4_K, 1037, 4096), (synth.Q5_K, 515, 4608), (synth.Q4_K, 9, 8448),
    (synth.Q4_K, 8195, 4096), (synth.Q5_K, 8199, 2560), (synth.Q4_K, 8192, 256),
    (synth.Q5_K, 1030, 14336), (synth.Q4_K, 3, 20480), (synth.Q4_K, 1031, 32768),
    (synth.Q4_K, 4100, 11008), (synth.Q4_K, 33, 36864),
    (synth.Q6_K, 1029, 12288), (synth.Q6_K, 77, 6144), (synth.Q6_K, 33, 10240),
    (synth.Q6_K, 65, 16384), (synth.Q8_0, 1031, 4096), (synth.Q8_0, 45, 2304),
    (synth.Q8_0, 19, 256), (synth.IQ4_NL, 517, 4608), (synth.Q8_0, 300, 14336),
    (synth.Q6_K, 300, 24576), (synth.Q8_0, 129, 18688), (synth.Q6_K, 40, 32768),
    (synth.IQ4_NL, 70, 30720), (synth.Q6_K, 1031, 20480),
    (synth.Q6_K, 1029, 14336), (synth.IQ4_NL, 260, 16384),
    (synth.Q6_K, 1029, 9728), (synth.Q6_K, 300, 2560), (synth.Q6_K, 5, 256), (synth.Q6_K, 77, 17408),
    (synth.Q6_K, 33, 2304), (synth.Q8_0, 13, 896), (synth.Q8_0, 1000, 2336), (synth.IQ4_NL, 9, 2336),
    (synth.IQ4_NL, 517, 4640), (synth.Q6_K, 1031, 32512), (synth.Q8_0, 3, 32),
    (synth.Q8_0, 5, 34816),
    (synth.Q5_K, 100, 5120),    # persistent multi-pass kernel, 2-pass capacity
]


@pytest.mark.parametrize("t", [synth.Q4_K, synth.Q6_K, synth.Q8_0])
def test_gemv_misaligned_weight_pointer(t):
    """A weight at an address that is not 16-byte aligned takes the
    byte-granular kernel and gives the same sums."""
    from inferno_hip import device as D
    outer, inner = 37, 2560
    say(f"gemv misaligned weight type={t}")
    rng = synth.rng_for(0x3A + t)
    w = synth.weight(rng, t, outer, inner)
    x = synth.activations(rng, inner)
    buf = torch.zeros(w.size + 16, dtype=torch.uint8, device="cuda")
    buf[2:2 + w.size] = dev(w)
    y = D.gemv(D.DeviceWeight(buf[2:2 + w.size], t, inner, outer), dev(x)).cpu().numpy()
    ref = oracle.gemv_f64(t, w, x, inner, outer)
    assert_within(y, ref, oracle.tolerance(oracle.row_norms(t, w, inner, outer), x), f"type {t} misaligned")


@pytest.mark.parametrize("t,outer,inner", LAUNCH_SHAPES)
def test_gemv_every_launch(t, outer, inner):
    from inferno_hip import device as D
    say(f"gemv type={t} {outer}x{inner}")
    rng = synth.rng_for(131 + t + inner + outer)
    w = synth.weight(rng, t, outer, inner)
    x = synth.activations(rng, inner)
    y = D.gemv(dweight(w, t, inner, outer), dev(x)).cpu().numpy()
    ref = oracle.gemv_f64(t, w, x, inner, outer)
    tol = oracle.tolerance(oracle.row_norms(t, w, inner, outer), x)
    assert_within(y, ref, tol, f"type {t} {outer}x{inner}")


@pytest.mark.parametrize("hidden,inter", [
    (4096, 1030),   # wide kernel, one gate and one up row per wave
    (8448, 515),    # three passes, the last partial (one row pair per wave: serial)
    (14336, 300),   # four passes, serial
    (5120, 600),    # two passes, serial
    (5120, 2056),   # persistent multi-pass kernel, 2-pass capacity
    (8448, 2100),   # persistent multi-pass kernel, 4-pass capacity, the last pass partial
    (5120, 2048),   # 256 workgroups over 256 CUs: serial passes
    (20480, 64),    # 80 blocks: past the persistent kernel, serial passes
    (4096, 8195),   # persistent kernel
    (2560, 8200),   # persistent kernel, partial pass
])
@pytest.mark.parametrize("t", [synth.Q4_K, synth.Q5_K])
def test_gate_up_every_launch(t, hidden, inter):
    from inferno_hip import device as D
    say(f"gate/up type={t} {hidden}->{inter}")
    rng = synth.rng_for(inter + 17 * t + hidden)
    wg = synth.weight(rng, t, inter, hidden)
    wu = synth.weight(rng, t, inter, hidden)
    x = synth.activations(rng, hidden)
    h = D.gate_up_swiglu(dweight(wg, t, hidden, inter), dweight(wu, t, hidden, inter), dev(x)).cpu().numpy()
    g = oracle.gemv_f64(t, wg, x, hidden, inter)
    u = oracle.gemv_f64(t, wu, x, hidden, inter)
    hb = _h_bound(g, u, oracle.row_norms(t, wg, hidden, inter), oracle.row_norms(t, wu, hidden, inter), x)
    assert_within(h, g / (1 + np.exp(-g)) * u, hb, "h")


@pytest.mark.parametrize("t", [synth.Q4_K, synth.Q5_K, synth.Q6_K, synth.Q8_0, synth.IQ4_NL])
def test_gemv_activation_dynamic_range(t):
    """Sub-blocks of x spread over 10^-30 .. 10^30 (fp32 subnormals included):
    the integer-digit activations scale every 32-element sub-block on its own,
    so small sub-blocks next to huge ones keep their precision."""
    from inferno_hip import device as D
    rng = synth.rng_for(777 + t)
    outer, inner = 96, 4096
    w = synth.weight(rng, t, outer, inner)
    x = synth.activations(rng, inner).astype(np.float64)
    x *= np.repeat(10.0 ** rng.uniform(-30, 30, inner // 32), 32)
    x[:32] *= 1e-10  # a subnormal sub-block
    x = x.astype(np.float32)
    say(f"dynamic range type={t}")
    y = D.gemv(dweight(w, t, inner, outer), dev(x)).cpu().numpy()
    ref = oracle.gemv_f64(t, w, x, inner, outer)
    tol = oracle.tolerance(oracle.row_norms(t, w, inner, outer), x)
    assert_within(y, ref, tol, f"type {t} dynamic range")
    # the small sub-blocks alone (the large ones zeroed) are not lost either
    xs = np.where(np.abs(x) < 1e-20, x, 0).astype(np.float32)
    ys = D.gemv(dweight(w, t, inner, outer), dev(xs)).cpu().numpy()
    refs = oracle.gemv_f64(t, w, xs, inner, outer)
    tols = oracle.tolerance(oracle.row_norms(t, w, inner, outer), xs)
    assert_within(ys, refs, tols, f"type {t} small sub-blocks only")


@pytest.mark.parametrize("t,outer,inner", [
    (synth.Q4_K, 64, 4096), (synth.Q5_K, 64, 4096), (synth.Q8_0, 64, 4096), (synth.IQ4_NL, 64, 4096),
    (synth.Q6_K, 64, 2048),      # one-segment rows: each row ends inside its wave
    (synth.Q6_K, 64, 4096),      # two segments meet in LDS
    (synth.Q6_K, 4096, 12288),   # the FFN down shape: six segments
    (synth.Q6_K, 40, 2560),      # 10-block rows (at byte phases): a short second segment
])
def test_gemv_nonfinite_activations(t, outer, inner):
    """A NaN or an infinity in x makes every output non-finite
    (src/ModelCPU.jl:333-355: the reference's fp32 sum gives +-Inf or NaN per
    row; the integer-digit path gives NaN for all of them), wherever in x it
    sits: the first and last column, and a column of every segment."""
    from inferno_hip import device as D
    rng = synth.rng_for(4343 + t + inner)
    w = synth.weight(rng, t, outer, inner)
    dw = dweight(w, t, inner, outer)
    cols = sorted({0, inner - 1, *range(1234 % inner, inner, 2048)})
    for c in cols:
        for bad in (np.nan, np.inf, -np.inf):
            x = synth.activations(rng, inner)
            x[c] = bad
            say(f"nonfinite type={t} {outer}x{inner} x[{c}]={bad}")
            y = D.gemv(dw, dev(x)).cpu().numpy()
            assert not np.any(np.isfinite(y)), (t, c, bad)


def test_gemv_special_inputs():
    from inferno_hip import device as D
    rng = synth.rng_for(4242)
    outer, inner = 64, 4096
    w = synth.weight(rng, synth.Q4_K, outer, inner)
    dw = dweight(w, synth.Q4_K, inner, outer)
    say("gemv zero x")
    y = D.gemv(dw, torch.zeros(inner, device="cuda")).cpu().numpy()
    assert np.all(y == 0)
    say("gemv one-hot x pins columns")
    W = oracle.dequant(synth.Q4_K, w, outer * inner).reshape(outer, inner)
    for c in (0, 31, 32, 63, 64, 255, 256, 2047, 2048, 4095):
        e = np.zeros(inner, np.float32)
        e[c] = 1.0
        y = D.gemv(dw, dev(e)).cpu().numpy()
        assert np.allclose(y, W[:, c], rtol=2e-6, atol=1e-9), c


# ---------------------------------------------------- SwiGLU / FFN block ----

def _ffn_case(hidden, inter, gt=synth.Q4_K, dt=synth.Q6_K, seed=0xC3):
    rng = synth.rng_for(seed)
    wg = synth.weight(rng, gt, inter, hidden)
    wu = synth.weight(rng, gt, inter, hidden)
    wd = synth.weight(rng, dt, hidden, inter)
    x = synth.activations(rng, hidden)
    return wg, wu, wd, x


def _h_bound(g, u, ng, nu, x):
    tg = oracle.tolerance(ng, x)
    tu = oracle.tolerance(nu, x)
    s = 1 / (1 + np.exp(-g))
    silu = g * s
    dsilu = s * (1 + g * (1 - s))
    return np.abs(dsilu * u) * tg + np.abs(silu) * tu + 1e-6 * np.abs(silu * u) + 1e-30


@pytest.mark.parametrize("hidden,inter,gt,dt", [
    (4096, 12288, synth.Q4_K, synth.Q6_K),   # the decode FFN block, full size
    (2048, 5632, synth.Q5_K, synth.Q6_K),
    (1024, 2816, synth.Q4_K, synth.Q8_0),
    (512, 768, synth.Q8_0, synth.Q4_K),      # unfused gate/up path
])
def test_ffn_block(hidden, inter, gt, dt):
    say(f"ffn hidden={hidden} inter={inter} gate/up={gt} down={dt}")
    wg, wu, wd, x = _ffn_case(hidden, inter, gt, dt)
    from inferno_hip import device as D
    h = torch.empty(inter, device="cuda")
    y = D.ffn_swiglu(dweight(wg, gt, hidden, inter), dweight(wu, gt, hidden, inter),
                     dweight(wd, dt, inter, hidden), dev(x), h=h).cpu().numpy()
    h = h.cpu().numpy()
    g, u, h_ref, y_ref = oracle.ffn_swiglu_f64(gt, wg, gt, wu, dt, wd, x, hidden, inter)
    hb = _h_bound(g, u, oracle.row_norms(gt, wg, hidden, inter),
                  oracle.row_norms(gt, wu, hidden, inter), x)
    assert_within(h, h_ref, hb, "h = silu(g)*u")
    nd = oracle.row_norms(dt, wd, inter, hidden)
    dh = np.linalg.norm(h.astype(np.float64) - h_ref)
    assert_within(y, y_ref, 1e-4 * nd * np.linalg.norm(h_ref) + nd * dh, "ffn y")


@pytest.mark.parametrize("gt,ut,hidden,inter", [
    (synth.Q8_0, synth.Q8_0, 2048, 1030),           # streamed digit kernel, SwiGLU epilogue
    (synth.Q6_K, synth.Q6_K, 4096, 515),
    (synth.IQ4_NL, synth.IQ4_NL, 1024, 777),
    (synth.Q4_K, synth.Q5_K, 1024, 1030),           # mixed pair: wide kernel, SwiGLU epilogue
    (synth.Q4_K, synth.Q5_K, 4096, 8200),           # mixed pair: persistent kernel (>= 8192 rows)
    (synth.Q8_0, synth.Q8_0, 18432, 300),           # 9 segments: 16-wave streamed kernel
    (synth.Q6_K, synth.Q6_K, 768, 301),             # 3-block rows: streamed kernel at byte phases
])
def test_gate_up_unfused_pairs(gt, ut, hidden, inter):
    """Pairs that are not a matching Q4_K/Q5_K pair: the gate GEMV writes g into
    h, and the up GEMV's epilogue makes h = silu(g) * u in place (no scratch)."""
    from inferno_hip import device as D
    say(f"unfused gate/up gate={gt} up={ut} {hidden}->{inter}")
    rng = synth.rng_for(0x6A7E + gt + 3 * ut + inter)
    wg = synth.weight(rng, gt, inter, hidden)
    wu = synth.weight(rng, ut, inter, hidden)
    x = synth.activations(rng, hidden)
    h = D.gate_up_swiglu(dweight(wg, gt, hidden, inter), dweight(wu, ut, hidden, inter), dev(x)).cpu().numpy()
    g = oracle.gemv_f64(gt, wg, x, hidden, inter)
    u = oracle.gemv_f64(ut, wu, x, hidden, inter)
    hb = _h_bound(g, u, oracle.row_norms(gt, wg, hidden, inter), oracle.row_norms(ut, wu, hidden, inter), x)
    assert_within(h, g / (1 + np.exp(-g)) * u, hb, "h = silu(g)*u")


def test_gate_up_misaligned_pair_takes_the_epilogue_path():
    from inferno_hip import device as D
    hidden, inter, t = 1024, 515, synth.Q4_K
    rng = synth.rng_for(0x6A7F)
    wg = synth.weight(rng, t, inter, hidden)
    wu = synth.weight(rng, t, inter, hidden)
    x = synth.activations(rng, hidden)
    say("gate/up Q4_K pair 4 bytes past alignment")
    wgd = dev(np.concatenate([np.zeros(4, np.uint8), wg]))[4:]
    h = D.gate_up_swiglu(D.DeviceWeight(wgd, t, hidden, inter), dweight(wu, t, hidden, inter),
                         dev(x)).cpu().numpy()
    g = oracle.gemv_f64(t, wg, x, hidden, inter)
    u = oracle.gemv_f64(t, wu, x, hidden, inter)
    hb = _h_bound(g, u, oracle.row_norms(t, wg, hidden, inter), oracle.row_norms(t, wu, hidden, inter), x)
    assert_within(h, g / (1 + np.exp(-g)) * u, hb, "h = silu(g)*u")


@pytest.mark.parametrize("t,hidden,inter", [(synth.Q6_K, 2048, 301), (synth.Q8_0, 1024, 515)])
def test_gate_up_misaligned_up_weight_takes_the_byte_granular_epilogue(t, hidden, inter):
    """An up weight off 16-byte alignment runs on the byte-granular kernel, so
    its SwiGLU epilogue (silu(g) * u against the gate row already in h) is the
    one that kernel carries."""
    from inferno_hip import device as D
    rng = synth.rng_for(0x6A80 + t)
    wg = synth.weight(rng, t, inter, hidden)
    wu = synth.weight(rng, t, inter, hidden)
    x = synth.activations(rng, hidden)
    say(f"gate/up type={t} {hidden}->{inter}: up weight 2 bytes past alignment")
    wud = dev(np.concatenate([np.zeros(2, np.uint8), wu]))[2:]
    h = D.gate_up_swiglu(dweight(wg, t, hidden, inter), D.DeviceWeight(wud, t, hidden, inter),
                         dev(x)).cpu().numpy()
    g = oracle.gemv_f64(t, wg, x, hidden, inter)
    u = oracle.gemv_f64(t, wu, x, hidden, inter)
    hb = _h_bound(g, u, oracle.row_norms(t, wg, hidden, inter), oracle.row_norms(t, wu, hidden, inter), x)
    assert_within(h, g / (1 + np.exp(-g)) * u, hb, "h = silu(g)*u")


def test_ffn_host_entry_point():
    from inferno_hip import _lib
    import ctypes as C
    hidden, inter = 1024, 2816
    wg, wu, wd, x = _ffn_case(hidden, inter, seed=11)
    y = np.zeros(hidden, np.float32)
    h = np.zeros(inter, np.float32)
    say("ihip_ffn_swiglu host")
    _lib.check(_lib.lib().ihip_ffn_swiglu(synth.Q4_K, wg.ctypes.data, synth.Q4_K, wu.ctypes.data,
                                          synth.Q6_K, wd.ctypes.data, x.ctypes.data, h.ctypes.data,
                                          y.ctypes.data, hidden, inter))
    g, u, h_ref, y_ref = oracle.ffn_swiglu_f64(synth.Q4_K, wg, synth.Q4_K, wu, synth.Q6_K, wd, x,
                                               hidden, inter)
    nd = oracle.row_norms(synth.Q6_K, wd, inter, hidden)
    dh = np.linalg.norm(h.astype(np.float64) - h_ref)
    assert_within(y, y_ref, 1e-4 * nd * np.linalg.norm(h_ref) + nd * dh, "host ffn y")


def test_fused_elementwise_kernels():
    from inferno_hip import FusedKernels as FK
    rng = np.random.default_rng(3)
    g = (rng.standard_normal(10007) * 4).astype(np.float32)
    u = rng.standard_normal(10007).astype(np.float32)
    say("fused_mlp_gate_mul_ / fused_silu_gate_mul_")
    gd = dev(g)
    FK.fused_mlp_gate_mul_(gd, dev(u))
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.allclose(gd.cpu().numpy(), ref, rtol=2e-6, atol=1e-7)
    out = torch.empty(10007, device="cuda")
    FK.fused_silu_gate_mul_(out, dev(g), dev(u))
    assert np.allclose(out.cpu().numpy(), ref, rtol=2e-6, atol=1e-7)


# ------------------------------------------------------ lm_head + argmax ----

@pytest.mark.parametrize("t,vocab,hidden,seed", [
    (synth.Q6_K, 151936, 2048, 0xC2),   # the lm_head workload, full size
    (synth.Q6_K, 151936, 2048, 0xC2 + 1),
    (synth.Q6_K, 1000, 2048, 5),
    (synth.Q8_0, 32000, 2048, 6),
    (synth.Q6_K, 4099, 8192, 8),       # four segments: rows meet in LDS per chunk
    (synth.Q8_0, 3001, 20480, 9),      # ten segments: 16-wave streamed kernel
    (synth.Q8_0, 777, 34816, 11),      # 17 segments: GEMV + standalone argmax
    (synth.Q6_K, 151936, 2560, 0xD1),  # 10 blocks a row (2100 bytes): segments at byte phases
    (synth.Q6_K, 4099, 2560, 0xD2),
    (synth.Q8_0, 3001, 2336, 0xD4),
    (synth.Q4_K, 5003, 1024, 7),       # GEMV + standalone argmax path
    (synth.Q6_K, 18992, 2048, 0xE0),   # one GPU's vocabulary rows of the lm_head over 8 GPUs
])
def test_lm_head_argmax(t, vocab, hidden, seed):
    say(f"lm_head type={t} vocab={vocab} hidden={hidden} seed={seed}")
    rng = synth.rng_for(seed)
    w = synth.weight(rng, t, vocab, hidden)
    x = synth.activations(rng, hidden)
    from inferno_hip import device as D
    ws = D.ArgmaxWorkspace()
    logits = torch.empty(vocab, device="cuda")
    dw = dweight(w, t, hidden, vocab)
    D.lm_head_argmax(dw, dev(x), ws, logits=logits)
    tok = ws.result()
    ref = oracle.gemv_f64(t, w, x, hidden, vocab)
    tol = oracle.tolerance(oracle.row_norms(t, w, hidden, vocab), x)
    assert_within(logits.cpu().numpy(), ref, tol, "logits")
    best = int(np.argmax(ref))
    gap = ref[best] - np.max(np.delete(ref, best))
    say(f"top-2 gap {gap:.4g} vs bound {2 * tol.max():.4g}")
    assert gap > 2 * tol.max(), "seed gives an ambiguous maximum"
    assert tok == best
    # without logits, twice in a row (the workspace must come back zeroed)
    for _ in range(2):
        D.lm_head_argmax(dw, dev(x), ws, logits=None)
        assert ws.result() == best


def test_lm_head_unfused_needs_logits():
    """Where the argmax is not fused into the GEMV the logits have to land
    somewhere: NULL logits is refused at the C ABI (no library scratch), and
    the Python mirror passes a buffer of its own."""
    from inferno_hip import _lib
    from inferno_hip import device as D
    t, vocab, hidden = synth.Q4_K, 5003, 1024
    rng = synth.rng_for(0x10)
    w = synth.weight(rng, t, vocab, hidden)
    x = synth.activations(rng, hidden)
    dw, xd, ws = dweight(w, t, hidden, vocab), dev(x), D.ArgmaxWorkspace()
    say("lm_head Q4_K without logits")
    L = _lib.lib()
    assert L.ihip_lm_head_fused(t, dw.data.data_ptr(), xd.data_ptr(), hidden, vocab) == 0
    assert L.ihip_lm_head_fused(synth.Q6_K, dw.data.data_ptr(), xd.data_ptr(), 2048, vocab) == 1
    rc = L.ihip_lm_head_argmax_dev(t, dw.data.data_ptr(), xd.data_ptr(), None, ws.token.data_ptr(),
                                   ws.flags.data_ptr(), hidden, vocab, ws.ws.data_ptr(),
                                   torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.IHIP_ERR_INVALID
    D.lm_head_argmax(dw, xd, ws, logits=None)
    assert ws.result() == int(np.argmax(oracle.gemv_f64(t, w, x, hidden, vocab)))


def test_host_weight_cache_sees_rewritten_bytes():
    """A weight rewritten in place (or freed and its address reused for other
    bytes) without ihip_weight_forget is uploaded again: the cache checks a
    sampled content fingerprint on every call."""
    from inferno_hip import QuantizedKernels as QK
    t, outer, inner = synth.Q4_K, 256, 4096
    rng = synth.rng_for(0xCAFE)
    w = synth.weight(rng, t, outer, inner)
    x = synth.activations(rng, inner)
    out = np.zeros(outer, np.float32)
    for rep in range(3):
        say(f"host mirror, weight rewritten in place, rep {rep}")
        QK.q4_k_gemv_(out, w, x, inner, outer)
        assert_within(out, oracle.gemv_f64(t, w, x, inner, outer),
                      oracle.tolerance(oracle.row_norms(t, w, inner, outer), x), f"rep {rep}")
        w[:] = synth.weight(rng, t, outer, inner)   # same address, new bytes, no forget()


def test_lm_head_host_entry_point_and_nonfinite():
    from inferno_hip import _lib
    import ctypes as C
    rng = synth.rng_for(99)
    vocab, hidden = 4096, 2048
    w = synth.weight(rng, synth.Q6_K, vocab, hidden)
    x = synth.activations(rng, hidden)
    tok = C.c_int32(-1)
    logits = np.zeros(vocab, np.float32)
    say("ihip_lm_head_argmax host")
    _lib.check(_lib.lib().ihip_lm_head_argmax(synth.Q6_K, w.ctypes.data, x.ctypes.data,
                                              logits.ctypes.data, C.byref(tok), hidden, vocab))
    ref = oracle.gemv_f64(synth.Q6_K, w, x, hidden, vocab)
    assert tok.value == int(np.argmax(ref))
    # a NaN scale in one block makes that logit NaN: an error, like CommonOps.jl:149-150
    w2 = w.copy()
    w2[208:210] = np.array([0x7E00], np.uint16).view(np.uint8)
    say("ihip_lm_head_argmax with a NaN logit")
    rc = _lib.lib().ihip_lm_head_argmax(synth.Q6_K, w2.ctypes.data, x.ctypes.data, None,
                                        C.byref(tok), hidden, vocab)
    assert rc == _lib.IHIP_ERR_NONFINITE
    assert b"NaN" in _lib.lib().ihip_last_error()
    # +Inf scale -> +Inf or NaN logit: still an error
    w3 = w.copy()
    w3[208:210] = np.array([0x7C00], np.uint16).view(np.uint8)
    rc = _lib.lib().ihip_lm_head_argmax(synth.Q6_K, w3.ctypes.data, x.ctypes.data, None,
                                        C.byref(tok), hidden, vocab)
    assert rc == _lib.IHIP_ERR_NONFINITE


@pytest.mark.parametrize("t,vocab,hidden", [
    (synth.Q4_K, 5003, 1024),    # the argmax runs as a second kernel over the logits
    (synth.Q8_0, 777, 34816),    # 17 segments: unfused Q8_0
    (synth.Q6_K, 3001, 2048),    # fused
])
def test_lm_head_host_entry_point_null_logits(t, vocab, hidden):
    """ihip_lm_head_argmax with logits NULL: the token is still the oracle's,
    whether or not the argmax is fused into the GEMV (the unfused path puts
    the logits in library staging)."""
    from inferno_hip import _lib
    import ctypes as C
    rng = synth.rng_for(0x4E55 + t)
    w = synth.weight(rng, t, vocab, hidden)
    x = synth.activations(rng, hidden)
    tok = C.c_int32(-1)
    say(f"ihip_lm_head_argmax host, type {t} {vocab}x{hidden}, NULL logits")
    _lib.check(_lib.lib().ihip_lm_head_argmax(t, w.ctypes.data, x.ctypes.data, None, C.byref(tok),
                                              hidden, vocab))
    ref = oracle.gemv_f64(t, w, x, hidden, vocab)
    order = np.argsort(ref)
    tol = oracle.tolerance(oracle.row_norms(t, w, hidden, vocab), x)
    assert ref[order[-1]] - ref[order[-2]] > 2 * tol.max(), "seed gives an ambiguous maximum"
    assert tok.value == int(order[-1])


ARGMAX_CASES = {
    # tests/unit/test_common_ops.jl:85-93 and :61-62 (0-based here)
    "all -inf": (np.array([-np.inf, -np.inf], np.float32), 0),
    "greedy 0..5": (np.arange(6, dtype=np.float32), 5),
    "skip -inf": (np.array([-np.inf, 0, -np.inf, 1], np.float32), 3),
    "tie lowest index": (np.array([3, 7, 7, 1], np.float32), 1),
    "signed zeros tie": (np.array([-0.0, 0.0, -1.0], np.float32), 0),
    "single": (np.array([-3.5], np.float32), 0),
}


@pytest.mark.parametrize("name", sorted(ARGMAX_CASES))
def test_argmax_reference_cases(name):
    from inferno_hip import FusedKernels as FK
    v, want = ARGMAX_CASES[name]
    say(f"argmax {name}")
    assert FK.gpu_argmax(dev(v)) == want
    assert oracle.argmax(v)[0] == want


def test_argmax_errors_and_large_ties():
    from inferno_hip import FusedKernels as FK, _lib
    for bad in ([1, np.inf], [1, np.nan], [np.nan, np.nan]):
        say(f"argmax error case {bad}")
        with pytest.raises(_lib.IHIPArgumentError):
            FK.gpu_argmax(dev(np.array(bad, np.float32)))
    with pytest.raises(_lib.IHIPArgumentError):
        FK.gpu_argmax(torch.empty(0, device="cuda"))
    rng = np.random.default_rng(8)
    for n in (151936, 1 << 20, 257, 65):
        v = rng.integers(-1000, 1000, size=n).astype(np.float32)
        v[rng.integers(0, n, size=5)] = 5000.0  # several equal maxima
        say(f"argmax ties n={n}")
        assert FK.gpu_argmax(dev(v)) == int(np.argmax(v))


# ------------------------------------------------------------- prefill ----

def prefill_operands(X):
    """The activations the matrix cores take: each token row scaled by 2^s,
    s = 15 - (the binary exponent of its largest magnitude), rounded to fp16
    and scaled back (exact); rows holding NaN or an infinity unscaled."""
    X = np.asarray(X, np.float32)
    m = np.max(np.abs(X), axis=1)
    e = np.frexp(np.where(np.isfinite(m), m, 1.0))[1]
    s = np.where(np.isfinite(m), 15 - e, 0).astype(np.int64)
    with np.errstate(over="ignore", invalid="ignore"):
        h = np.ldexp(X.astype(np.float64), s[:, None]).astype(np.float32).astype(np.float16)
    return np.ldexp(h.astype(np.float64), -s[:, None]).astype(np.float32)


def test_prefill_operand_rounding_matches_plain_fp16_in_range():
    """For rows whose values sit in fp16's normal range the per-row scale is a
    power of two, so the operands equal plain fp16 rounding (a check of the
    restatement above, on the CPU data the prefill tests use)."""
    rng = synth.rng_for(0xC5)
    X = rng.standard_normal((64, 512)).astype(np.float32)
    X[np.abs(X) < 1e-3] = 1e-3  # keep every value a normal fp16 number
    assert np.array_equal(prefill_operands(X), X.astype(np.float16).astype(np.float32))


@pytest.mark.parametrize("T,outer,inner", [
    (512, 4096, 4096),   # the batched prefill workload
    (70, 300, 2048),     # ragged tiles
    (1, 128, 256),
    (33, 129, 1792),     # 7 block columns: the ring wraps twice, ragged tiles
    (5, 64, 512),        # 2 block columns: no loop iteration, last column peeled
    (40, 200, 768),      # 3 block columns: the odd tail
    (64, 256, 1024),     # 4 block columns: one loop iteration, even tail
    (512, 512, 4096),    # one GPU's weight rows of the prefill over 8 GPUs: split over K
    (100, 384, 4096),    # eight splits of two block columns
    (17, 1000, 2816),    # 11 block columns in five uneven splits
    (7, 129, 2048),      # four splits, T x outer odd: the scalar sum of the splits
    (9, 300, 14336),     # token rows past 8192 values: the conversion reads them twice
    (3, 130, 8448),      # just past 8192 values, 33 block columns
    (515, 1141, 256),    # short rows (fp32 kernel): seeded shapes whose fp16-operand
    (487, 1645, 512),    #   errors reached 1.5x and 1.05x the row bound
    (66, 130, 768),      # the shortest rows on the fp16 matrix cores
    (582, 1758, 768),    # a seeded shape whose shared sub-block scale rounding reached 1.14x
    (100, 300, 2560),    # the first rows past the exactly rounded weights
])
def test_prefill_q4k(T, outer, inner):
    """Every token against the per-token GEMV oracle (src/ModelCPU.jl:1001-1017)
    on the fp32 activations; rows of more than 512 columns run on fp16
    matrix-core operands, and are also held to the oracle on the activations
    rounded as those operands."""
    say(f"prefill T={T} {outer}x{inner}")
    rng = synth.rng_for(0xC4 + T)
    w = synth.weight(rng, synth.Q4_K, outer, inner)
    X = rng.standard_normal((T, inner)).astype(np.float32)
    from inferno_hip import device as D
    Y = D.prefill_q4_k(dweight(w, synth.Q4_K, inner, outer), dev(X)).cpu().numpy()
    nrm = oracle.row_norms(synth.Q4_K, w, inner, outer)
    xn = np.linalg.norm(X.astype(np.float64), axis=1)
    ref32 = oracle.gemm_f64(synth.Q4_K, w, X, inner, outer)
    ratio32 = np.abs(Y.astype(np.float64) - ref32) / (1e-4 * nrm[None, :] * xn[:, None])
    bad = np.argwhere(ratio32 > 1.0)
    assert bad.size == 0, f"{len(bad)} outputs over the bound, first (token, row) {tuple(bad[0])}"
    say(f"prefill max err/tol = {float(np.max(ratio32)):.3e}")
    if inner > 512:
        Xh = prefill_operands(X)  # the matrix-core operand rounding
        xhn = np.linalg.norm(Xh.astype(np.float64), axis=1)
        ref = oracle.gemm_f64(synth.Q4_K, w, Xh, inner, outer)
        ratio = np.abs(Y.astype(np.float64) - ref) / (1e-4 * nrm[None, :] * xhn[:, None])
        assert np.all(ratio <= 1.0), f"fp16-x oracle: max err/tol {float(np.max(ratio)):.3g}"
    else:  # fp32 operands: fp32 rounding over K terms, a fraction of the bound
        assert float(np.max(ratio32)) < 0.25


@pytest.mark.parametrize("t,outer,inner,woff", [
    (synth.Q4_K, 4096, 4096, 0),    # the attention output projection's shape
    (synth.Q5_K, 1000, 2048, 0),
    (synth.Q6_K, 777, 12288, 0),    # streamed rows
    (synth.Q8_0, 515, 4096, 0),
    (synth.IQ4_NL, 300, 2048, 0),
    (synth.Q4_K, 129, 1024, 2),     # weight off 16-byte alignment: byte-granular kernel
])
def test_gemv_add_folds_the_residual(t, outer, inner, woff):
    """out = resid + W x (the attention output projection and the layer's
    residual add, src/ModelCPU.jl:885, 909) in one launch: bit-identical to
    the GEMV followed by an fp32 add, in place and not; x overlapping out is
    refused."""
    from inferno_hip import device as D
    from inferno_hip._lib import IHIPArgumentError
    say(f"gemv_add type={t} {outer}x{inner} weight offset {woff}")
    rng = synth.rng_for(0x5F0 + t + outer)
    w = synth.weight(rng, t, outer, inner)
    buf = torch.zeros(w.size + 16, dtype=torch.uint8, device="cuda")
    buf[woff:woff + w.size] = dev(w)
    dw = D.DeviceWeight(buf[woff:woff + w.size], t, inner, outer)
    x = dev(synth.activations(rng, inner))
    resid = dev(rng.standard_normal(outer).astype(np.float32))
    want = (D.gemv(dw, x) + resid).cpu().numpy()
    out = torch.full((outer,), float("nan"), device="cuda")
    got = D.gemv_add(dw, x, resid, out).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    inplace = resid.clone()
    D.gemv_add(dw, x, inplace)
    assert np.array_equal(inplace.cpu().numpy().view(np.uint32), want.view(np.uint32))
    both = torch.zeros(inner + outer, device="cuda")
    with pytest.raises(IHIPArgumentError, match="overlaps"):
        D.gemv_add(dw, both[:inner], resid, both[inner - 1:inner - 1 + outer])
    shifted = torch.zeros(outer + 4, device="cuda")
    with pytest.raises(IHIPArgumentError, match="resid overlaps out"):
        D.gemv_add(dw, x, shifted[4:4 + outer], shifted[:outer])


@pytest.mark.parametrize("inner", [2048, 4096])
def test_prefill_shared_activations_match_the_one_call_entry_point(inner):
    """One rounding of X, then products with several weights, as the
    attention's wq, wk and wv share their input (src/ModelCPU.jl:789-791):
    each output bit-identical to prefill_q4_k's for that weight, within the
    row bound of the oracle, and the rounded rows in xh untouched by the
    products (the 320-row weight splits K and writes partial sums into xh)."""
    from inferno_hip import device as D
    T = 300
    rng = synth.rng_for(0x5E0 + inner)
    X = rng.standard_normal((T, inner)).astype(np.float32)
    X[7] *= np.float32(3e5)  # a row past fp16's range: its own scale
    Xd = dev(X)
    say(f"prefill shared activations T={T} inner={inner}: rows 4096, 320, 1000")
    xh = D.prefill_convert(Xd)
    kept = (2 * T * inner + 15) // 16 * 16 + 4 * T  # rounded rows and per-token scales
    rounded = xh[:kept].clone()
    for outer in (4096, 320, 1000):
        w = synth.weight(rng, synth.Q4_K, outer, inner)
        dw = dweight(w, synth.Q4_K, inner, outer)
        Y = D.prefill_q4_k_xh(dw, xh, T).cpu().numpy()
        want = D.prefill_q4_k(dw, Xd).cpu().numpy()
        assert np.array_equal(Y.view(np.uint32), want.view(np.uint32)), f"outer {outer}"
        assert torch.equal(xh[:kept], rounded), f"the product with outer {outer} changed the rounded rows"
        ref = oracle.gemm_f64(synth.Q4_K, w, X, inner, outer)
        nrm = oracle.row_norms(synth.Q4_K, w, inner, outer)
        xn = np.linalg.norm(X.astype(np.float64), axis=1)
        ratio = np.abs(Y.astype(np.float64) - ref) / (1e-4 * nrm[None, :] * xn[:, None])
        assert np.all(ratio <= 1.0), f"outer {outer}: max err/tol {float(np.max(ratio)):.3g}"


def test_prefill_shared_activations_refuse_short_rows():
    """Rows of at most 512 columns run on fp32 operands straight from X, so
    the two halves refuse them."""
    from inferno_hip import device as D
    from inferno_hip._lib import IHIPArgumentError
    say("prefill halves refuse 512-column rows")
    T, outer, inner = 16, 64, 512
    rng = synth.rng_for(0x5E9)
    Xd = dev(rng.standard_normal((T, inner)).astype(np.float32))
    dw = dweight(synth.weight(rng, synth.Q4_K, outer, inner), synth.Q4_K, inner, outer)
    xh = D.prefill_scratch(T, inner)
    with pytest.raises(IHIPArgumentError):
        D.prefill_convert(Xd, xh)
    with pytest.raises(IHIPArgumentError):
        D.prefill_q4_k_xh(dw, xh, T)


@pytest.mark.parametrize("scale", [1e5, 1e-6, 1e30, 1e-38])
def test_prefill_any_finite_activations(scale):
    """Token rows scaled to 1e5 (past fp16's 65504) and to 1e-6 (below its
    normal range), beside unscaled rows; rows of 1e30 and of fp32 subnormals;
    an all-zero row: every output against the fp32-x oracle (the reference
    multiplies fp32 activations of any size, src/ModelCPU.jl:285-307)."""
    from inferno_hip import device as D
    T, outer, inner = 48, 320, 2048
    rng = synth.rng_for(0xC6)
    w = synth.weight(rng, synth.Q4_K, outer, inner)
    X = rng.standard_normal((T, inner)).astype(np.float64)
    X[::3] *= scale                                  # every third row scaled
    X[1::7] *= float(np.clip(1.0 / scale, 1e-30, 1e30))  # and some the other way
    X[5] = 0.0
    X = X.astype(np.float32)
    say(f"prefill rows scaled by {scale:g}")
    Y = D.prefill_q4_k(dweight(w, synth.Q4_K, inner, outer), dev(X)).cpu().numpy()
    assert np.all(np.isfinite(Y))
    nrm = oracle.row_norms(synth.Q4_K, w, inner, outer)
    xn = np.linalg.norm(X.astype(np.float64), axis=1)
    ref = oracle.gemm_f64(synth.Q4_K, w, X, inner, outer)
    tol = 1e-4 * nrm[None, :] * xn[:, None] + 1e-45
    ratio = np.abs(Y.astype(np.float64) - ref) / tol
    assert np.all(ratio <= 1.0), f"max err/tol {float(np.max(ratio)):.3g} at {np.unravel_index(np.argmax(ratio), ratio.shape)}"
    assert np.all(Y[5] == 0.0)
    # the operands the matrix cores took: the restatement's rounding
    refh = oracle.gemm_f64(synth.Q4_K, w, prefill_operands(X), inner, outer)
    xhn = np.linalg.norm(prefill_operands(X).astype(np.float64), axis=1)
    assert np.all(np.abs(Y.astype(np.float64) - refh) <= 1e-4 * nrm[None, :] * xhn[:, None] + 1e-45)


@pytest.mark.parametrize("inner", [512, 1024, 2048])  # 512: the fp32 kernel; 2048: K split four ways
def test_prefill_nonfinite_activations_reach_their_rows(inner):
    """A NaN or an infinity in a token row makes that row's outputs
    non-finite, as the reference's fp32 sum does, and leaves the other rows
    exact to the bound."""
    from inferno_hip import device as D
    T, outer = 8, 128
    rng = synth.rng_for(0xC7)
    w = synth.weight(rng, synth.Q4_K, outer, inner)
    X = rng.standard_normal((T, inner)).astype(np.float32)
    X[2, 17] = np.nan
    X[4, min(1000, inner - 2)] = np.inf
    X[6, 3] = -np.inf
    X[6, inner - 1] = np.inf  # -Inf and +Inf in one row (in different splits at 2048)
    say(f"prefill with NaN / +Inf / -Inf rows, inner {inner}")
    Y = D.prefill_q4_k(dweight(w, synth.Q4_K, inner, outer), dev(X)).cpu().numpy()
    for r in (2, 4, 6):
        assert not np.any(np.isfinite(Y[r])), r
    good = [0, 1, 3, 5, 7]
    nrm = oracle.row_norms(synth.Q4_K, w, inner, outer)
    ref = oracle.gemm_f64(synth.Q4_K, w, X[good], inner, outer)
    xn = np.linalg.norm(X[good].astype(np.float64), axis=1)
    assert np.all(np.abs(Y[good].astype(np.float64) - ref) <= 1e-4 * nrm[None, :] * xn[:, None])


def test_device_calls_launch_on_the_current_stream():
    """Without a stream argument the device entry points launch on torch's
    current stream (read without building a Stream object): the same handle
    as torch.cuda.current_stream() by default, inside a stream context and
    inside a graph capture."""
    from inferno_hip import device as D
    from inferno_hip.device import _stream
    assert _stream() == torch.cuda.current_stream().cuda_stream
    s2 = torch.cuda.Stream()
    with torch.cuda.stream(s2):
        assert _stream() == s2.cuda_stream
    rng = synth.rng_for(0x57)
    t, outer, inner = synth.Q4_K, 256, 4096
    w = synth.weight(rng, t, outer, inner)
    x = synth.activations(rng, inner)
    dw, xd = dweight(w, t, inner, outer), dev(x)
    y = torch.zeros(outer, device="cuda")
    g = torch.cuda.CUDAGraph()
    cs = torch.cuda.Stream()
    with torch.cuda.graph(g, stream=cs):
        assert _stream() == cs.cuda_stream
        D.gemv(dw, xd, y)
    ref = oracle.gemv_f64(t, w, x, inner, outer)
    tol = oracle.tolerance(oracle.row_norms(t, w, inner, outer), x)
    for _ in range(3):  # replays, with eager work between them
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert_within(y.cpu().numpy(), ref, tol, "graph replay")


@pytest.mark.parametrize("T,outer,inner", [(64, 300, 4096), (33, 129, 1792), (9, 130, 256)])
def test_prefill_f32_operands_meet_the_bound_for_aligned_activations(T, outer, inner):
    """Token rows equal to weight rows (x = w_row, the worst case for operand
    rounding: the fp16 path reaches 2-3x the bound there) through
    ihip_prefill_q4_k_f32_dev, and random rows beside them, against the
    per-token GEMV oracle (src/ModelCPU.jl:1001-1017)."""
    from inferno_hip import device as D
    say(f"prefill fp32 operands T={T} {outer}x{inner}")
    rng = synth.rng_for(0xC8 + T)
    w = synth.weight(rng, synth.Q4_K, outer, inner)
    X = rng.standard_normal((T, inner)).astype(np.float32)
    wf = oracle.dequant(synth.Q4_K, w, outer * inner).reshape(outer, inner)
    X[::2] = wf[np.arange(0, T, 2) % outer]
    Y = D.prefill_q4_k_f32(dweight(w, synth.Q4_K, inner, outer), dev(X)).cpu().numpy()
    ref = oracle.gemm_f64(synth.Q4_K, w, X, inner, outer)
    nrm = oracle.row_norms(synth.Q4_K, w, inner, outer)
    xn = np.linalg.norm(X.astype(np.float64), axis=1)
    ratio = np.abs(Y.astype(np.float64) - ref) / (1e-4 * nrm[None, :] * xn[:, None])
    # fp32 rounding over K terms of one sign (x = w_row): 0.06 of the bound at K = 4096
    assert float(np.max(ratio)) < 0.25, f"max err/tol {float(np.max(ratio)):.3g}"


@pytest.mark.parametrize("t,outer,inner", [
    (synth.Q4_K, 300, 4096), (synth.Q5_K, 64, 2048), (synth.Q6_K, 300, 12288),
    (synth.Q8_0, 64, 4096), (synth.IQ4_NL, 64, 4096), (synth.Q4_K, 9, 256),
])
def test_gemv_activations_equal_to_a_weight_row(t, outer, inner):
    """x equal to a weight row (the input that defeats fp16 operands, where
    both roundings fall the same way): the integer-digit GEMV stays inside
    the row bound, which its representation guarantees for every input."""
    from inferno_hip import device as D
    say(f"gemv x = w_row type={t} {outer}x{inner}")
    rng = synth.rng_for(0xC9 + t + inner)
    w = synth.weight(rng, t, outer, inner)
    wf = oracle.dequant(t, w, outer * inner).reshape(outer, inner)
    dw = dweight(w, t, inner, outer)
    for r in (0, outer // 2, outer - 1):
        x = wf[r].astype(np.float32)
        y = D.gemv(dw, dev(x)).cpu().numpy()
        assert_within(y, oracle.gemv_f64(t, w, x, inner, outer),
                      oracle.tolerance(oracle.row_norms(t, w, inner, outer), x), f"x = row {r}")


def test_prefill_f32_operands_take_weights_past_fp16_range():
    """Block scales d ~ 200 put dequantized weights past fp16's 65504 (the
    fp16-operand prefill requires |w| < 65504): the fp32-operand entry point
    meets the per-token GEMV oracle (src/ModelCPU.jl:285-307) there, and at
    tiny scales (d ~ 1e-7, fp16 subnormal)."""
    from inferno_hip import device as D
    T, outer, inner = 40, 130, 1024
    for dval in (200.0, 1e-7):
        say(f"prefill fp32 operands, block scales ~ {dval:g}")
        rng = synth.rng_for(0xCA)
        w = synth.weight(rng, synth.Q4_K, outer, inner)
        b = w.reshape(outer, inner // 256, 144)
        d = np.abs(rng.standard_normal((outer, inner // 256))) * dval
        b[:, :, 0:2] = d.astype(np.float16).view(np.uint8).reshape(outer, inner // 256, 2)
        b[:, :, 2:4] = (d * 0.5).astype(np.float16).view(np.uint8).reshape(outer, inner // 256, 2)
        X = rng.standard_normal((T, inner)).astype(np.float32)
        Y = D.prefill_q4_k_f32(dweight(w, synth.Q4_K, inner, outer), dev(X)).cpu().numpy()
        ref = oracle.gemm_f64(synth.Q4_K, w, X, inner, outer)
        nrm = oracle.row_norms(synth.Q4_K, w, inner, outer)
        xn = np.linalg.norm(X.astype(np.float64), axis=1)
        assert np.all(np.isfinite(Y))
        assert np.all(np.abs(Y.astype(np.float64) - ref) <= 1e-4 * nrm[None, :] * xn[:, None])


def _set_block_scales(w, t, outer, inner, rng, dval):
    """Overwrite every block's fp16 scale(s) with |N(0,1)| * dval."""
    be = {synth.Q4_K: 256, synth.Q5_K: 256, synth.Q6_K: 256, synth.Q8_0: 32, synth.IQ4_NL: 32}[t]
    bb = {synth.Q4_K: 144, synth.Q5_K: 176, synth.Q6_K: 210, synth.Q8_0: 34, synth.IQ4_NL: 18}[t]
    b = w.reshape(outer, inner // be, bb)
    d = (np.abs(rng.standard_normal((outer, inner // be))) * dval).astype(np.float16)
    off = 208 if t == synth.Q6_K else 0
    b[:, :, off:off + 2] = d.view(np.uint8).reshape(outer, inner // be, 2)
    if t in (synth.Q4_K, synth.Q5_K):
        b[:, :, 2:4] = (d * np.float16(0.5)).view(np.uint8).reshape(outer, inner // be, 2)


@pytest.mark.parametrize("t", [synth.Q4_K, synth.Q5_K, synth.Q6_K, synth.Q8_0, synth.IQ4_NL])
@pytest.mark.parametrize("dval", [3000.0, 1e-7])
def test_gemv_extreme_block_scales(t, dval):
    """Block scales near fp16's top (~3000, weights up to ~3e6) and in its
    subnormal range (~1e-7): the GEMV's scales and sums are fp32, so the row
    bound holds for any finite weights (src/ModelCPU.jl:285-379)."""
    from inferno_hip import device as D
    outer, inner = 70, 4096
    say(f"gemv type {t} block scales ~ {dval:g}")
    rng = synth.rng_for(0xCB + t)
    w = synth.weight(rng, t, outer, inner)
    _set_block_scales(w, t, outer, inner, rng, dval)
    x = synth.activations(rng, inner)
    y = D.gemv(dweight(w, t, inner, outer), dev(x)).cpu().numpy()
    assert np.all(np.isfinite(y))
    assert_within(y, oracle.gemv_f64(t, w, x, inner, outer),
                  oracle.tolerance(oracle.row_norms(t, w, inner, outer), x), f"type {t} d ~ {dval:g}")
