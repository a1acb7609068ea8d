"""Every device entry point captured in a HIP graph and replayed.

A serving loop captures its decode step once and replays it; the benchmark
times the kernels the same way.  Each case here runs the entry point eagerly,
captures the same call (same buffers) into a graph on a side stream, and
replays it three times.  Before each replay the outputs are filled with NaN
and other eager work runs on torch's stream (a GEMV of another weight, an
elementwise op), with a synchronization between; after each replay every
output must equal the eager one bit for bit.  The kernels use no float atomics
and reduce in a fixed order, so a replay that differs in one bit has read
stale or uninitialised memory.  (The entry points record no memset nodes:
every workspace word they read is written earlier in the same call.)

The eager results themselves are held to the oracle by test_gpu_parity.py,
test_gpu_block.py and test_gpu_q8k.py; one GEMV case here also checks its
eager output against the row bound, so a graph that replays a wrong result
consistently cannot pass.
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


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def dweight(rng, t, outer, inner):
    from inferno_hip.device import DeviceWeight
    w = synth.weight(rng, t, outer, inner)
    return w, DeviceWeight(dev(w), t, inner, outer)


@pytest.fixture(scope="module")
def other_work():
    """Unrelated eager work run between replays."""
    from inferno_hip import device as D
    rng = synth.rng_for(0x6A0)
    _, w = dweight(rng, synth.Q4_K, 1024, 2048)
    x = dev(synth.activations(rng, 2048))
    y = torch.empty(1024, device="cuda")

    def run():
        D.gemv(w, x, y)
        y.mul_(0.5).add_(1.0)
    return run


def replay_matches_eager(call, outputs, other_work, inputs_reset=None):
    """call() launches on the current stream and writes `outputs` (tensors);
    inputs_reset() restores inputs an in-place call overwrote."""
    if inputs_reset:
        inputs_reset()
    call()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outputs]
    g = torch.cuda.CUDAGraph()
    cs = torch.cuda.Stream()
    if inputs_reset:
        inputs_reset()
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=cs):
        call()
    torch.cuda.synchronize()
    for rep in range(3):
        for o in outputs:
            o.fill_(float("nan")) if o.is_floating_point() else o.fill_(0x5A)
        if inputs_reset:
            inputs_reset()
        other_work()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outputs, eager)):
            same = torch.equal(o, e) if not o.is_floating_point() else \
                torch.equal(o.view(torch.int32), e.view(torch.int32))
            assert same, f"replay {rep}: output {i} differs from the eager call"
    return eager


@pytest.mark.parametrize("t,outer,inner", [
    (synth.Q4_K, 4096, 4096),    # wide kernel, two rows per wave
    (synth.Q5_K, 12288, 4096),   # persistent wide kernel
    (synth.Q6_K, 4096, 12288),   # streamed kernel, six segments (the FFN down)
    (synth.Q8_0, 4096, 4096),    # Q8_0 on the wide kernel
    (synth.IQ4_NL, 2048, 4096),
    (synth.Q6_K, 3, 768),        # rows below one wave's worth
])
def test_gemv_graph(t, outer, inner, other_work):
    from inferno_hip import device as D
    say(f"graph gemv type {t} {outer}x{inner}")
    rng = synth.rng_for(0x6A1 + t + outer)
    w, dw = dweight(rng, t, outer, inner)
    x = synth.activations(rng, inner)
    xd, y = dev(x), torch.empty(outer, device="cuda")
    (e,) = replay_matches_eager(lambda: D.gemv(dw, xd, y), [y], other_work)
    if t == synth.Q6_K and outer == 4096:  # the eager result itself against the row bound
        ref = oracle.gemv_f64(t, w, x, inner, outer)
        tol = oracle.tolerance(oracle.row_norms(t, w, inner, outer), x)
        assert np.all(np.abs(e.cpu().numpy().astype(np.float64) - ref) <= tol)


def test_gemv_add_graph(other_work):
    from inferno_hip import device as D
    say("graph gemv_add Q4_K 4096x4096")
    rng = synth.rng_for(0x6AD)
    _, dw = dweight(rng, synth.Q4_K, 4096, 4096)
    xd = dev(synth.activations(rng, 4096))
    resid = dev(rng.standard_normal(4096).astype(np.float32))
    out = torch.empty(4096, device="cuda")
    replay_matches_eager(lambda: D.gemv_add(dw, xd, resid, out), [out], other_work)


def test_gemv_norm_graph(other_work):
    from inferno_hip import device as D
    say("graph gemv of the normed x, Q4_K 6144x4096 (folded)")
    rng = synth.rng_for(0x6AE)
    _, dw = dweight(rng, synth.Q4_K, 6144, 4096)
    xd = dev(synth.activations(rng, 4096))
    nw = dev(rng.uniform(0.5, 1.5, 4096).astype(np.float32))
    out, xn = torch.empty(6144, device="cuda"), torch.empty(4096, device="cuda")
    replay_matches_eager(lambda: D.gemv_norm(dw, nw, 1e-6, xd, out, xn), [out], other_work)


def test_dequantize_graph(other_work):
    from inferno_hip import device as D
    say("graph dequantize Q6_K 512x2048")
    _, dw = dweight(synth.rng_for(0x6A2), synth.Q6_K, 512, 2048)
    out = torch.empty(512 * 2048, device="cuda")
    replay_matches_eager(lambda: D.dequantize(dw, out), [out], other_work)


@pytest.mark.parametrize("hidden,inter,gt,dt", [
    (4096, 12288, synth.Q4_K, synth.Q6_K),   # the decode FFN block
    (1024, 2816, synth.Q5_K, synth.Q4_K),
])
def test_ffn_swiglu_graph(hidden, inter, gt, dt, other_work):
    from inferno_hip import device as D
    say(f"graph ffn {hidden}/{inter}")
    rng = synth.rng_for(0x6A3 + hidden)
    _, wg = dweight(rng, gt, inter, hidden)
    _, wu = dweight(rng, gt, inter, hidden)
    _, wd = dweight(rng, dt, hidden, inter)
    xd = dev(synth.activations(rng, hidden))
    h, y = torch.empty(inter, device="cuda"), torch.empty(hidden, device="cuda")
    replay_matches_eager(lambda: D.ffn_swiglu(wg, wu, wd, xd, h=h, y=y), [h, y], other_work)


def test_ffn_block_graph(other_work):
    """In place on x: x is restored before the eager call, the capture and
    every replay."""
    from inferno_hip import device as D
    from inferno_hip import _lib
    hidden, inter = 4096, 12288
    say(f"graph ffn block {hidden}/{inter}")
    rng = synth.rng_for(0x6A4)
    _, wg = dweight(rng, synth.Q4_K, inter, hidden)
    _, wu = dweight(rng, synth.Q4_K, inter, hidden)
    _, wd = dweight(rng, synth.Q6_K, hidden, inter)
    x0 = dev(synth.activations(rng, hidden))
    nw = dev(rng.uniform(0.5, 1.5, hidden).astype(np.float32))
    x = x0.clone()
    n = _lib.lib().ihip_ffn_block_scratch_floats(synth.Q4_K, synth.Q4_K, hidden, inter)
    h = torch.empty(n, device="cuda")
    replay_matches_eager(lambda: D.ffn_block(wg, wu, wd, nw, 1e-6, x, h=h), [x], other_work,
                         inputs_reset=lambda: x.copy_(x0))


@pytest.mark.parametrize("t,vocab,hidden", [
    (synth.Q6_K, 151936, 2048),  # fused argmax partials + finalize
    (synth.Q4_K, 5003, 1024),    # GEMV, then the standalone argmax
])
def test_lm_head_argmax_graph(t, vocab, hidden, other_work):
    from inferno_hip import device as D
    say(f"graph lm_head type {t} {vocab}x{hidden}")
    rng = synth.rng_for(0x6A5 + vocab)
    _, dw = dweight(rng, t, vocab, hidden)
    xd = dev(synth.activations(rng, hidden))
    ws = D.ArgmaxWorkspace()
    logits = torch.empty(vocab, device="cuda")
    replay_matches_eager(lambda: D.lm_head_argmax(dw, xd, ws, logits=logits),
                         [logits, ws.token, ws.flags], other_work)


def test_lm_head_argmax_norm_graph(other_work):
    from inferno_hip import device as D
    vocab, hidden = 32000, 2048
    say(f"graph final norm + lm_head {vocab}x{hidden}")
    rng = synth.rng_for(0x6A6)
    _, dw = dweight(rng, synth.Q6_K, vocab, hidden)
    xd = dev(synth.activations(rng, hidden))
    nw = dev(rng.uniform(0.5, 1.5, hidden).astype(np.float32))
    ws = D.ArgmaxWorkspace()
    xn, logits = torch.empty(hidden, device="cuda"), torch.empty(vocab, device="cuda")
    replay_matches_eager(lambda: D.lm_head_argmax_norm(dw, nw, 1e-6, xd, ws, xn=xn, logits=logits),
                         [xn, logits, ws.token, ws.flags], other_work)


@pytest.mark.parametrize("T,outer,inner", [
    (512, 4096, 4096),   # the prefill workload: one workgroup per tile
    (64, 4096, 4096),    # K split eight ways, the partial planes summed
    (17, 1000, 2816),    # ragged tiles, K split
    (100, 300, 512),     # short rows: the fp32 kernel
])
def test_prefill_graph(T, outer, inner, other_work):
    from inferno_hip import device as D
    say(f"graph prefill T={T} {outer}x{inner}")
    rng = synth.rng_for(0x6A7 + T)
    _, dw = dweight(rng, synth.Q4_K, outer, inner)
    X = dev(rng.standard_normal((T, inner)).astype(np.float32))
    Y = torch.empty(T, outer, device="cuda")
    xh = D.prefill_scratch(T, inner)
    replay_matches_eager(lambda: D.prefill_q4_k(dw, X, Y, xh), [Y], other_work)


def test_prefill_shared_rounding_graph(other_work):
    """One rounding of X, then two products (one of them splitting K)."""
    from inferno_hip import device as D
    T, inner = 64, 4096
    say(f"graph prefill halves T={T} inner={inner}: rows 4096 and 320")
    rng = synth.rng_for(0x6AB)
    _, dw1 = dweight(rng, synth.Q4_K, 4096, inner)
    _, dw2 = dweight(rng, synth.Q4_K, 320, inner)
    X = dev(rng.standard_normal((T, inner)).astype(np.float32))
    Y1, Y2 = torch.empty(T, 4096, device="cuda"), torch.empty(T, 320, device="cuda")
    xh = D.prefill_scratch(T, inner)

    def call():
        D.prefill_convert(X, xh)
        D.prefill_q4_k_xh(dw1, xh, T, Y1)
        D.prefill_q4_k_xh(dw2, xh, T, Y2)
    replay_matches_eager(call, [Y1, Y2], other_work)


def test_prefill_f32_operands_graph(other_work):
    from inferno_hip import device as D
    T, outer, inner = 96, 1000, 2048
    say(f"graph prefill on fp32 operands T={T} {outer}x{inner}")
    rng = synth.rng_for(0x6AC)
    _, dw = dweight(rng, synth.Q4_K, outer, inner)
    X = dev(rng.standard_normal((T, inner)).astype(np.float32))
    Y = torch.empty(T, outer, device="cuda")
    replay_matches_eager(lambda: D.prefill_q4_k_f32(dw, X, Y), [Y], other_work)


@pytest.mark.parametrize("t", [synth.Q4_K, synth.Q6_K])
def test_int8_activation_gemv_graph(t, other_work):
    from inferno_hip import device as D
    from inferno_hip import _lib
    outer, inner = 4096, 4096
    say(f"graph int8-activation gemv type {t}")
    rng = synth.rng_for(0x6A8 + t)
    _, dw = dweight(rng, t, outer, inner)
    xd = dev(synth.activations(rng, inner))
    y = torch.empty(outer, device="cuda")
    q8 = torch.empty(inner // 256 * _lib.Q8_K_BYTES, dtype=torch.uint8, device="cuda")
    replay_matches_eager(lambda: D.gemv_q8k_x(dw, xd, y, q8=q8), [y, q8], other_work)


def test_rmsnorm_graph(other_work):
    from inferno_hip import device as D
    n = 4096
    say("graph rmsnorm")
    rng = np.random.default_rng(0x6A9)
    x = dev(rng.standard_normal(n).astype(np.float32))
    w = dev(rng.uniform(0.5, 1.5, n).astype(np.float32))
    out = torch.empty(n, device="cuda")
    replay_matches_eager(lambda: D.rmsnorm(x, w, 1e-6, out=out), [out], other_work)
