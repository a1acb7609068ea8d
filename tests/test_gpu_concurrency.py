"""Concurrent callers of the C ABI.

The reference's kernels are plain C functions behind `ccall`
(src/QuantizedKernels.jl:84-148), so a Julia engine may call them from
several threads at once.  Here:
* the device entry points run from four host threads at once, each on its
  own stream with its own buffers and workspaces (an FFN, an lm_head with its
  argmax, a prefill whose K is split over workgroups, and the composite calls:
  a grouped wq/wk/wv GEMV, wo with its residual, one prefill rounding for two
  weights), 12 calls each; every
  call's outputs are copied aside on the caller's stream and must equal an
  eager call's bit for bit (nothing a `*_dev` call touches is shared between
  callers);
* the host-pointer entry points run from four threads at once over four
  weights (and a device-pointer caller beside them), and must equal a serial
  call bit for bit (the host path's staging buffers and weight cache are
  shared and held under the library's lock).
ctypes releases the GIL during the foreign call, so the calls do overlap in
the library.
"""
import threading

import numpy as np
import pytest

from inferno_hip import synth

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

REPS = 12


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
    return DeviceWeight(dev(synth.weight(rng, t, outer, inner)), t, inner, outer)


def run_threads(fns):
    errors = []

    def wrap(fn):
        try:
            fn()
        except BaseException as e:  # reported after the join
            errors.append(e)
    ts = [threading.Thread(target=wrap, args=(f,)) for f in fns]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=300)
    assert not any(t.is_alive() for t in ts), "a caller thread did not finish"
    if errors:
        raise errors[0]


def same_bits(a, b):
    if a.is_floating_point():
        return torch.equal(a.view(torch.int32), b.view(torch.int32))
    return torch.equal(a, b)


def test_device_entry_points_from_threads_on_their_own_streams():
    from inferno_hip import device as D
    rng = synth.rng_for(0x6B0)
    say("concurrent device callers: ffn 2048/5632, lm_head 32000x2048, prefill 64x4096x2048")
    # FFN (gate/up Q4_K, down Q6_K)
    hidden, inter = 2048, 5632
    wg, wu = dweight(rng, synth.Q4_K, inter, hidden), dweight(rng, synth.Q4_K, inter, hidden)
    wd = dweight(rng, synth.Q6_K, hidden, inter)
    fx = dev(synth.activations(rng, hidden))
    fh, fy = torch.empty(inter, device="cuda"), torch.empty(hidden, device="cuda")
    # lm_head with the fused argmax
    vocab, lh = 32000, 2048
    wl = dweight(rng, synth.Q6_K, vocab, lh)
    lx = dev(synth.activations(rng, lh))
    ws = D.ArgmaxWorkspace()
    logits = torch.empty(vocab, device="cuda")
    # prefill with K split over workgroups
    T, outer, inner = 64, 4096, 2048
    wp = dweight(rng, synth.Q4_K, outer, inner)
    X = dev(rng.standard_normal((T, inner)).astype(np.float32))
    Y, xh = torch.empty(T, outer, device="cuda"), D.prefill_scratch(T, inner)

    # the composite calls: wq/wk/wv as one group, wo with the residual, and
    # the prefill's two halves over two weights
    qkv = D.WeightGroup([synth.weight(rng, synth.Q4_K, o, 2048) for o in (2048, 512, 512)],
                        synth.Q4_K, 2048, (2048, 512, 512))
    wo = dweight(rng, synth.Q4_K, 2048, 2048)
    ax, ar = dev(synth.activations(rng, 2048)), dev(synth.activations(rng, 2048))
    qout, aout = torch.empty(3072, device="cuda"), torch.empty(2048, device="cuda")
    wp2 = dweight(rng, synth.Q4_K, 1024, inner)
    X2 = dev(rng.standard_normal((T, inner)).astype(np.float32))
    Y2a, Y2b, xh2 = torch.empty(T, outer, device="cuda"), torch.empty(T, 1024, device="cuda"), \
        D.prefill_scratch(T, inner)

    def composite(s):
        qkv.gemv(ax, qout, stream=s)
        D.gemv_add(wo, ax, ar, aout, stream=s)
        D.prefill_convert(X2, xh2, stream=s)
        D.prefill_q4_k_xh(wp, xh2, T, Y2a, stream=s)
        D.prefill_q4_k_xh(wp2, xh2, T, Y2b, stream=s)

    jobs = [
        (lambda s: D.ffn_swiglu(wg, wu, wd, fx, h=fh, y=fy, stream=s), [fh, fy]),
        (lambda s: D.lm_head_argmax(wl, lx, ws, logits=logits, stream=s), [logits, ws.token, ws.flags]),
        (lambda s: D.prefill_q4_k(wp, X, Y, xh, stream=s), [Y]),
        (composite, [qout, aout, Y2a, Y2b]),
    ]
    eager = []
    for call, outs in jobs:
        call(None)
        torch.cuda.synchronize()
        eager.append([o.clone() for o in outs])
    kept = [[[torch.empty_like(o) for o in outs] for _ in range(REPS)] for _, outs in jobs]
    for _, outs in jobs:
        for o in outs:
            o.fill_(float("nan")) if o.is_floating_point() else o.fill_(0x5A)
    torch.cuda.synchronize()

    def caller(j):
        call, outs = jobs[j]
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            for r in range(REPS):
                call(s)
                for o, k in zip(outs, kept[j][r]):
                    k.copy_(o)
        s.synchronize()
    run_threads([lambda j=j: caller(j) for j in range(len(jobs))])
    torch.cuda.synchronize()
    for j in range(len(jobs)):
        for r in range(REPS):
            for i, (k, e) in enumerate(zip(kept[j][r], eager[j])):
                assert same_bits(k, e), f"job {j} call {r} output {i} differs from the eager call"
    qkv.release()


def test_host_entry_points_from_threads():
    from inferno_hip import QuantizedKernels as QK
    from inferno_hip import device as D
    say("concurrent host-pointer callers: four GEMVs, plus a device caller")
    rng = synth.rng_for(0x6B1)
    cases = [(synth.Q4_K, QK.q4_k_gemv_, 1024, 4096), (synth.Q5_K, QK.q5_k_gemv_, 777, 2048),
             (synth.Q6_K, QK.q6_k_gemv_, 2048, 4096), (synth.Q8_0, QK.q8_0_gemv_, 515, 4096)]
    ops = []
    for t, fn, outer, inner in cases:
        w = synth.weight(rng, t, outer, inner)
        xs = [synth.activations(rng, inner) for _ in range(4)]
        want = []
        for x in xs:  # serial calls first
            out = np.zeros(outer, np.float32)
            fn(out, w, x, inner, outer)
            want.append(out)
        ops.append((fn, w, xs, want, outer, inner))
    # a device-pointer caller on its own stream at the same time
    dw = dweight(rng, synth.Q6_K, 4096, 12288)
    dx = dev(synth.activations(rng, 12288))
    dy = torch.empty(4096, device="cuda")
    D.gemv(dw, dx, dy)
    torch.cuda.synchronize()
    dwant = dy.clone()
    dkept = [torch.empty_like(dy) for _ in range(REPS)]
    bad = []

    def host_caller(fn, w, xs, want, outer, inner):
        for r in range(REPS):
            i = r % len(xs)
            out = np.zeros(outer, np.float32)
            fn(out, w, xs[i], inner, outer)
            if not np.array_equal(out.view(np.int32), want[i].view(np.int32)):
                bad.append((fn.__name__, r))

    def dev_caller():
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            for r in range(REPS):
                D.gemv(dw, dx, dy, stream=s)
                dkept[r].copy_(dy)
        s.synchronize()
    run_threads([lambda op=op: host_caller(*op) for op in ops] + [dev_caller])
    torch.cuda.synchronize()
    assert not bad, f"host calls that differ from the serial ones: {bad[:5]}"
    for r in range(REPS):
        assert same_bits(dkept[r], dwant), f"device call {r} differs"
