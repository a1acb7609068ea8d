"""GPU parity of the int8-activation variant (the reference C numerics):
quantize_row_q8_K and the q{4,5,6}_k_gemv / vec_dot_q{4,5,6}_K_q8_K path of
src/kernels/quant_kernels.c, bit-exact against

* the reference's own outputs in tests/golden/ (written from the compiled
  reference C by tests/golden/make_golden.py),
* the oracle's restatement (oracle/kquant_oracle.c, itself pinned to those
  vectors and to the compiled reference), and
* the compiled reference C in oracle/_ref when it is present.

Every call goes through the C ABI (libinferno_hip.so).
"""
from pathlib import Path

import numpy as np
import pytest

import oracle
from inferno_hip import synth

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

GOLDEN = Path(__file__).resolve().parent / "golden"
K_TYPES = [synth.Q4_K, synth.Q5_K, synth.Q6_K]
NAMES = {synth.Q4_K: "q4_k", synth.Q5_K: "q5_k", synth.Q6_K: "q6_k"}


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


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


def x_cases():
    rng = np.random.default_rng(0x5A)
    ties = np.zeros(256, np.float32)  # amax = 127 gives d = 1, id = 1: x * id is x
    ties[0], ties[1] = 127.0, -127.0
    halves = np.arange(127, dtype=np.float32) + np.float32(0.5)
    ties[2:129], ties[129:256] = halves, -halves  # every .5 tie, both signs
    mixed = np.concatenate([
        np.zeros(256, np.float32),                                   # d = 0, id = 0
        ties,
        (rng.standard_normal(256) * 1e-30).astype(np.float32),      # tiny scale
        (rng.standard_normal(256) * 1e30).astype(np.float32),       # huge scale
        rng.standard_normal(256).astype(np.float32),
    ])
    return {
        "gauss_4096": rng.standard_normal(4096).astype(np.float32),
        "scaled_12288": (rng.standard_normal(12288) * 37.5).astype(np.float32),
        "edge_blocks": mixed,
    }


@pytest.mark.parametrize("name", sorted(x_cases()))
def test_quantize_row_q8k_bit_exact(name):
    from inferno_hip import device as D
    x = x_cases()[name]
    say(f"quantize_row_q8_K {name}: {x.size} values")
    got = D.quantize_row_q8k(dev(x)).cpu().numpy()
    assert np.array_equal(got, oracle.quantize_row_q8k(x))
    if oracle.ref_lib() is not None:
        assert np.array_equal(got, oracle.ref_quantize_row_q8k(x))


@pytest.mark.parametrize("t", K_TYPES)
def test_q8k_path_reproduces_reference_golden_vectors(t):
    from inferno_hip import QuantizedKernels as QK
    g = np.load(GOLDEN / f"ref_{NAMES[t]}.npz")
    outer, inner = int(g["outer"]), int(g["inner"])
    nb = inner // 256
    say(f"golden {NAMES[t]}: {outer}x{inner}")
    q8 = np.zeros(nb * QK.Q8_K_BYTES, np.uint8)
    QK.quantize_q8_k_(q8, g["x"], inner)
    assert np.array_equal(q8, g["ref_q8k"])
    gemv = {synth.Q4_K: QK.q4_k_gemv_q8k_, synth.Q5_K: QK.q5_k_gemv_q8k_,
            synth.Q6_K: QK.q6_k_gemv_q8k_}[t]
    out = np.zeros(outer, np.float32)
    q8b = np.zeros_like(q8)
    gemv(out, g["w"], g["x"], inner, outer, q8_buf=q8b)
    assert np.array_equal(q8b, g["ref_q8k"])
    assert same_bits(out, g["ref_gauss"])
    dot = {synth.Q4_K: QK.vec_dot_q4_k_q8_k, synth.Q5_K: QK.vec_dot_q5_k_q8_k,
           synth.Q6_K: QK.vec_dot_q6_k_q8_k}[t]
    rb = nb * synth.BLOCK_BYTES[t]
    for r in range(outer):
        v = dot(np.ascontiguousarray(g["w"][r * rb:(r + 1) * rb]), q8, nb)
        assert same_bits([v], [g["ref_gauss"][r]]), r


Q8K_CASES = [(33, 256), (7, 2048), (64, 4096), (1031, 4096), (96, 12288)]


@pytest.mark.parametrize("t", K_TYPES)
@pytest.mark.parametrize("outer,inner", Q8K_CASES)
def test_gemv_q8k_bit_exact(t, outer, inner):
    from inferno_hip import device as D
    rng = synth.rng_for(0x900 + 16 * t + inner % 251)
    w = synth.weight(rng, t, outer, inner)
    x = synth.activations(rng, inner) * np.float32(rng.uniform(0.1, 30))
    say(f"gemv_q8k type {t} {outer}x{inner}")
    q8 = D.quantize_row_q8k(dev(x))
    y = D.gemv_q8k(D.DeviceWeight(dev(w), t, inner, outer), q8).cpu().numpy()
    assert same_bits(y, oracle.gemv_q8k(t, w, x, inner, outer))
    if oracle.ref_lib() is not None:
        assert same_bits(y, oracle.ref_gemv(t, w, x, inner, outer))


@pytest.mark.parametrize("t", K_TYPES)
@pytest.mark.parametrize("outer,inner", Q8K_CASES)
def test_gemv_q8k_x_bit_exact(t, outer, inner):
    """x as fp32, quantized inside the call (one launch for Q4_K / Q5_K): the
    same bits as the reference, and the same Q8_K blocks in q8."""
    from inferno_hip import device as D
    rng = synth.rng_for(0x980 + 16 * t + inner % 251)
    w = synth.weight(rng, t, outer, inner)
    x = synth.activations(rng, inner) * np.float32(rng.uniform(0.1, 30))
    say(f"gemv_q8k_x type {t} {outer}x{inner}")
    dw = D.DeviceWeight(dev(w), t, inner, outer)
    want = oracle.gemv_q8k(t, w, x, inner, outer)
    q8 = torch.full((inner // 256 * 292,), 0xAB, dtype=torch.uint8, device="cuda")
    y = D.gemv_q8k_x(dw, dev(x), q8=q8).cpu().numpy()
    assert same_bits(y, want)
    assert np.array_equal(q8.cpu().numpy(), oracle.quantize_row_q8k(x))
    if t != synth.Q6_K:  # one launch, no Q8_K output
        assert same_bits(D.gemv_q8k_x(dw, dev(x)).cpu().numpy(), want)
    if oracle.ref_lib() is not None:
        assert same_bits(y, oracle.ref_gemv(t, w, x, inner, outer))


def _random_shape(seed):
    """Rows of 1..159 Q8_K blocks and 1..9000 of them, capped near 30 M weights."""
    r = np.random.default_rng(seed)
    inner = 256 * int(r.integers(1, [16, 64, 160][seed % 3]))
    outer = int(r.integers(1, [300, 3000, 9000][(seed // 3) % 3]))
    return max(1, min(outer, 30_000_000 // inner)), inner


@pytest.mark.parametrize("seed", range(9))
def test_gemv_q8k_x_random_shapes(seed):
    """Random shapes over every launch plan of the int8 path: with q8 given,
    and in one launch for Q4_K / Q5_K rows of at most 32768 columns (longer
    rows need q8, and the call says so)."""
    from inferno_hip import device as D
    from inferno_hip._lib import IHIPArgumentError
    outer, inner = _random_shape(seed)
    for t in K_TYPES:
        rng = synth.rng_for(0x9A0 + seed * 7 + t)
        w = synth.weight(rng, t, outer, inner)
        x = synth.activations(rng, inner) * np.float32(rng.uniform(0.1, 30))
        say(f"gemv_q8k_x random seed {seed} type {t} {outer}x{inner}")
        dw = D.DeviceWeight(dev(w), t, inner, outer)
        want = oracle.gemv_q8k(t, w, x, inner, outer)
        q8 = torch.empty(inner // 256 * 292, dtype=torch.uint8, device="cuda")
        assert same_bits(D.gemv_q8k_x(dw, dev(x), q8=q8).cpu().numpy(), want)
        if t == synth.Q6_K:
            continue
        if inner <= 32768:
            assert same_bits(D.gemv_q8k_x(dw, dev(x)).cpu().numpy(), want)
        else:
            with pytest.raises(IHIPArgumentError):
                D.gemv_q8k_x(dw, dev(x))


@pytest.mark.parametrize("t", [synth.Q4_K, synth.Q5_K])
def test_gemv_q8k_x_quantizer_edge_blocks(t):
    """Zero blocks (d = 0), every .5 tie of both signs, tiny and huge scales,
    quantized inside the GEMV launch."""
    from inferno_hip import device as D
    x = x_cases()["edge_blocks"]
    inner, outer = x.size, 37
    rng = synth.rng_for(0x9E0 + t)
    w = synth.weight(rng, t, outer, inner)
    say(f"gemv_q8k_x edge blocks type {t}")
    q8 = torch.zeros(inner // 256 * 292, dtype=torch.uint8, device="cuda")
    y = D.gemv_q8k_x(D.DeviceWeight(dev(w), t, inner, outer), dev(x), q8=q8).cpu().numpy()
    assert np.array_equal(q8.cpu().numpy(), oracle.quantize_row_q8k(x))
    assert same_bits(y, oracle.gemv_q8k(t, w, x, inner, outer))


def test_gemv_q8k_x_fallbacks():
    """x not 16-byte aligned: quantized into q8 first, same bits; Q6_K needs q8."""
    from inferno_hip import device as D
    from inferno_hip._lib import IHIPArgumentError
    outer, inner = 65, 2048
    rng = synth.rng_for(0x9F0)
    x = synth.activations(rng, inner)
    say("gemv_q8k_x fallbacks")
    for t in (synth.Q4_K, synth.Q6_K):
        w = synth.weight(rng, t, outer, inner)
        dw = D.DeviceWeight(dev(w), t, inner, outer)
        buf = torch.zeros(inner + 4, dtype=torch.float32, device="cuda")
        buf[1:1 + inner] = dev(x)
        q8 = torch.zeros(inner // 256 * 292, dtype=torch.uint8, device="cuda")
        y = D.gemv_q8k_x(dw, buf[1:1 + inner], q8=q8).cpu().numpy()
        assert same_bits(y, oracle.gemv_q8k(t, w, x, inner, outer))
        with pytest.raises(IHIPArgumentError):
            D.gemv_q8k_x(dw, buf[1:1 + inner])


def test_gemv_q8k_full_size_q4k():
    from inferno_hip import QuantizedKernels as QK
    rng = synth.rng_for(0xC0)
    w = synth.weight(rng, synth.Q4_K, 4096, 4096)
    x = synth.activations(rng, 4096)
    say("gemv_q8k Q4_K 4096x4096 (host mirror)")
    out = np.zeros(4096, np.float32)
    QK.q4_k_gemv_q8k_(out, w, x, 4096, 4096)
    assert same_bits(out, oracle.gemv_q8k(synth.Q4_K, w, x, 4096, 4096))


def test_q8k_argument_errors():
    from inferno_hip import QuantizedKernels as QK
    from inferno_hip import device as D
    from inferno_hip._lib import IHIPArgumentError
    say("q8k argument errors")
    with pytest.raises(IHIPArgumentError):
        QK.quantize_q8_k_(np.zeros(292, np.uint8), np.zeros(300, np.float32), 300)
    with pytest.raises(IHIPArgumentError):
        QK.vec_dot_q4_k_q8_k(np.zeros(144, np.uint8), np.zeros(100, np.uint8), 1)
    q8 = D.quantize_row_q8k(dev(np.ones(256, np.float32)))
    w = D.DeviceWeight(dev(np.zeros(34 * 8, np.uint8)), synth.Q8_0, 256, 1)
    with pytest.raises(IHIPArgumentError):
        D.gemv_q8k(w, q8)
