"""GPU parity of the path's fused neighbours: rmsnorm_cpu! (src/ModelCPU.jl:
111-123) folded into the gate/up pass, the residual add of the decoder's MLP
half (src/ModelCPU.jl:913-920) folded into the down projection, and the final
norm ahead of the lm_head (src/ModelCPU.jl:1014-1015), against the fp64
oracle (oracle.rmsnorm_f64, oracle.ffn_block_f64).

Bars: rmsnorm within 4 fp32 ulps of the fp64 value; the FFN under the same
per-row GEMV bound as the plain FFN tests, with x' = rmsnorm(x) .* w as the
GEMV input; the residual adds one fp32 rounding; token ids exact.
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


def dweight(w, t, inner, outer):
    from inferno_hip.device import DeviceWeight
    return DeviceWeight(dev(w), t, inner, outer)


def check_within(y, ref, tol, what):
    err = np.abs(np.asarray(y, np.float64) - ref)
    say(f"{what}: max err/tol = {float(np.max(err / tol)):.3e}")
    assert np.all(err <= tol), f"{what}: {int(np.sum(err > tol))} over tolerance"


def h_bound(g, u, ng, nu, xin):
    tg = oracle.tolerance(ng, xin)
    tu = oracle.tolerance(nu, xin)
    s = 1 / (1 + np.exp(-g))
    silu = g * s
    dsilu = s * (1 + g * (1 - s))
    return np.abs(dsilu * u) * tg + np.abs(silu) * tu + 1e-6 * np.abs(silu * u) + 1e-30


@pytest.mark.parametrize("n,eps", [(4096, 1e-6), (2048, 1e-5), (1000, 0.5)])
def test_rmsnorm(n, eps):
    from inferno_hip import device as D
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    w = rng.uniform(0.5, 1.5, n).astype(np.float32)
    say(f"rmsnorm n={n} eps={eps}")
    ref = oracle.rmsnorm_f64(x, w, eps)
    tol = 4 * np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64) + 1e-30
    check_within(D.rmsnorm(dev(x), dev(w), eps).cpu().numpy(), ref, tol, "rmsnorm")
    xd = dev(x)
    D.rmsnorm(xd, dev(w), eps, out=xd)  # in place
    check_within(xd.cpu().numpy(), ref, tol, "rmsnorm in place")


FFN_CASES = [
    (4096, 12288, synth.Q4_K, synth.Q6_K),   # decode FFN block, full size: fused norm + residual
    (2048, 5632, synth.Q5_K, synth.Q6_K),
    (1024, 2816, synth.Q4_K, synth.Q4_K),    # residual in the wide kernel's epilogue
    (5120, 1280, synth.Q5_K, synth.Q5_K),    # norm folded into a two-pass gate/up
    (1024, 8448, synth.Q4_K, synth.Q4_K),    # residual in a three-pass down; persistent gate/up
    (2560, 9728, synth.Q4_K, synth.Q6_K),    # down rows of 38 blocks at byte phases
    (512, 768, synth.Q8_0, synth.Q8_0),      # unfused gate/up: norm kernel first
    (4096, 1536, synth.Q4_K, synth.Q6_K),    # one GPU's share of the decode FFN over 8 GPUs
    (2048, 5120, synth.Q5_K, synth.Q5_K),    # residual in a persistent two-pass down
    (12288, 512, synth.Q4_K, synth.Q4_K),    # norm folded into a serial four-pass gate/up
    (5120, 2560, synth.Q5_K, synth.Q5_K),    # norm folded into a persistent two-pass gate/up
    (12288, 2304, synth.Q4_K, synth.Q4_K),   # norm folded into a persistent four-pass gate/up
    (1024, 2048, synth.IQ4_NL, synth.IQ4_NL),  # SwiGLU and residual epilogues of the IQ4_NL wide kernel
]


def _block_case(hidden, inter, gt, dt, seed):
    rng = synth.rng_for(seed)
    wg = synth.weight(rng, gt, inter, hidden)
    wu = synth.weight(rng, gt, inter, hidden)
    wd = synth.weight(rng, dt, hidden, inter)
    x = synth.activations(rng, hidden) * np.float32(2.5)
    nw = rng.uniform(0.5, 1.5, hidden).astype(np.float32)
    return wg, wu, wd, x, nw


def _check_block(x_out, h, x, case, gt, dt, hidden, inter, eps):
    wg, wu, wd, _, nw = case
    n, g, u, h_ref, y_ref = oracle.ffn_block_f64(gt, wg, gt, wu, dt, wd, x, nw, eps, hidden, inter)
    ng = oracle.row_norms(gt, wg, hidden, inter)
    nu = oracle.row_norms(gt, wu, hidden, inter)
    if h is not None:
        check_within(h, h_ref, h_bound(g, u, ng, nu, n), "h = silu(g)*u of the normed x")
    nd = oracle.row_norms(dt, wd, inter, hidden)
    dh = 0.0 if h is None else np.linalg.norm(np.asarray(h, np.float64) - h_ref)
    if h is None:  # host entry point: bound h by its own tolerance
        dh = np.linalg.norm(h_bound(g, u, ng, nu, n))
    tol = 1e-4 * nd * np.linalg.norm(h_ref) + nd * dh + 2 * np.spacing(np.abs(y_ref).astype(np.float32))
    check_within(x_out, y_ref, tol, "x + Wd h")


@pytest.mark.parametrize("t,outer,inner", [
    (synth.Q4_K, 6144, 4096),   # wq + wk + wv rows: the norm folded, two rows per wave
    (synth.Q5_K, 1000, 2048),   # folded, one row per wave
    (synth.Q4_K, 8192, 4096),   # the persistent kernel's rows: folded there too
    (synth.Q5_K, 10240, 2048),  # wq 8192 + wk/wv 1024 rows of a larger model, persistent
    (synth.Q6_K, 777, 2048),    # another format: the norm first
    (synth.Q4_K, 300, 5120),    # rows of two passes: the norm first
])
def test_gemv_norm(t, outer, inner):
    """out = W (rmsnorm(x) .* norm_w) (src/ModelCPU.jl:903 then :789-791)
    within the row bound of the fp64 oracle's normed input, the norm folded
    into the GEMV or run first into xn."""
    from inferno_hip import device as D
    eps = 1e-6
    rng = synth.rng_for(0xB20 + outer + inner)
    w = synth.weight(rng, t, outer, inner)
    x = synth.activations(rng, inner) * np.float32(2.5)
    nw = rng.uniform(0.5, 1.5, inner).astype(np.float32)
    say(f"gemv of the normed x type={t} {outer}x{inner}")
    xn = torch.full((inner,), float("nan"), device="cuda")
    y = D.gemv_norm(dweight(w, t, inner, outer), dev(nw), eps, dev(x), xn=xn).cpu().numpy()
    n = oracle.rmsnorm_f64(x, nw, eps)
    ref = oracle.gemv_f64(t, w, n, inner, outer)
    nrm = oracle.row_norms(t, w, inner, outer)
    check_within(y, ref, 1e-4 * nrm * np.linalg.norm(n) + 1e-6 * nrm * np.linalg.norm(n), "W rmsnorm(x)")


@pytest.mark.parametrize("hidden,inter,gt,dt", FFN_CASES)
def test_ffn_block_with_norm_and_residual(hidden, inter, gt, dt):
    from inferno_hip import device as D
    eps = 1e-6
    case = _block_case(hidden, inter, gt, dt, 0xB10C + hidden)
    wg, wu, wd, x, nw = case
    say(f"ffn block hidden={hidden} inter={inter} gate/up={gt} down={dt}")
    xd = dev(x)
    # caller scratch: inter + hidden floats for every pair
    from inferno_hip import _lib
    nh = _lib.lib().ihip_ffn_block_scratch_floats(gt, gt, hidden, inter)
    assert nh == inter + hidden
    h = torch.full((nh,), float("nan"), device="cuda")
    D.ffn_block(dweight(wg, gt, hidden, inter), dweight(wu, gt, hidden, inter),
                dweight(wd, dt, inter, hidden), dev(nw), eps, xd, h=h)
    _check_block(xd.cpu().numpy(), h[:inter].cpu().numpy(), x, case, gt, dt, hidden, inter, eps)
    if gt not in (synth.Q4_K, synth.Q5_K):  # the unfused pair's normed input went to h + inter
        n = oracle.rmsnorm_f64(x, nw, eps)
        check_within(h[inter:].cpu().numpy(), n, 4 * np.spacing(np.abs(n).astype(np.float32)) + 1e-30,
                     "normed x in h + inter")


def test_ffn_block_misaligned_fused_pair_takes_the_unfused_path():
    """A Q4_K pair whose gate weight is off 16-byte alignment cannot run as
    one fused pass: it runs unfused (norm kernel, gate GEMV, up GEMV with the
    SwiGLU epilogue) inside the inter + hidden floats of scratch the header
    asks for, and matches the oracle; nothing is written past h."""
    from inferno_hip import _lib
    hidden, inter, eps = 1024, 2816, 1e-6
    case = _block_case(hidden, inter, synth.Q4_K, synth.Q4_K, 0xB10E)
    wg, wu, wd, x, nw = case
    say("ffn block: misaligned Q4_K pair")
    wgd = dev(np.concatenate([np.zeros(4, np.uint8), wg]))[4:]   # 4 bytes past 16-byte alignment
    nh = _lib.lib().ihip_ffn_block_scratch_floats(synth.Q4_K, synth.Q4_K, hidden, inter)
    xd, wud, wdd, nwd = dev(x), dev(wu), dev(wd), dev(nw)  # held until the queued kernels have run
    h = torch.full((nh + 64,), 7.0, device="cuda")  # 64 guard floats after the scratch
    _lib.check(_lib.lib().ihip_ffn_block_dev(synth.Q4_K, wgd.data_ptr(), synth.Q4_K, wud.data_ptr(),
                                             synth.Q4_K, wdd.data_ptr(), nwd.data_ptr(), eps,
                                             xd.data_ptr(), h.data_ptr(), hidden, inter,
                                             torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    _check_block(xd.cpu().numpy(), h[:inter].cpu().numpy(), x, case, synth.Q4_K, synth.Q4_K, hidden,
                 inter, eps)
    assert torch.all(h[nh:] == 7.0).item(), "write past the scratch"


def test_ffn_block_host_entry_point():
    from inferno_hip import _lib
    hidden, inter, gt, dt = 1024, 2816, synth.Q4_K, synth.Q6_K if 2816 % 2048 == 0 else synth.Q8_0
    eps = 1e-5
    case = _block_case(hidden, inter, gt, dt, 0xB10D)
    wg, wu, wd, x, nw = case
    say("ihip_ffn_block host")
    xo = x.copy()
    _lib.check(_lib.lib().ihip_ffn_block(gt, wg.ctypes.data, gt, wu.ctypes.data, dt, wd.ctypes.data,
                                         nw.ctypes.data, eps, xo.ctypes.data, hidden, inter))
    _check_block(xo, None, x, case, gt, dt, hidden, inter, eps)


@pytest.mark.parametrize("t,vocab,hidden,seed", [(synth.Q6_K, 32000, 2048, 0x7E), (synth.Q4_K, 5003, 1024, 0x7F)])
def test_lm_head_with_final_norm(t, vocab, hidden, seed):
    from inferno_hip import device as D
    rng = synth.rng_for(seed)
    w = synth.weight(rng, t, vocab, hidden)
    x = synth.activations(rng, hidden) * np.float32(4.0)
    nw = rng.uniform(0.5, 1.5, hidden).astype(np.float32)
    eps = 1e-6
    say(f"final norm + lm_head type={t} vocab={vocab}")
    ws = D.ArgmaxWorkspace()
    logits = torch.empty(vocab, device="cuda")
    xn = D.lm_head_argmax_norm(dweight(w, t, hidden, vocab), dev(nw), eps, dev(x), ws, logits=logits)
    tok = ws.result()
    n = oracle.rmsnorm_f64(x, nw, eps)
    ref = np.empty(vocab)
    ref[:] = oracle.gemv_f64(t, w, n.astype(np.float32), hidden, vocab)
    tol = oracle.tolerance(oracle.row_norms(t, w, hidden, vocab), n) + 1e-6 * np.abs(ref)
    check_within(logits.cpu().numpy(), ref, tol, "logits of the normed x")
    check_within(xn.cpu().numpy(), n, 4 * np.spacing(np.abs(n).astype(np.float32)) + 1e-30, "xn")
    best = int(np.argmax(ref))
    gap = ref[best] - np.max(np.delete(ref, best))
    assert gap > 2 * tol.max(), "seed gives an ambiguous maximum"
    assert tok == best
