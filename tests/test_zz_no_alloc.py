"""The allocation-free lm_head entry point, ihip_lm_head_argmax_noalloc_dev,
against the entry point it varies, ihip_lm_head_argmax_dev (same kernels, the
argmax partials in a caller workspace instead of the library's per-device
scratch array), through the C ABI.

Two calls in a row on one GPU, the second smaller than the first, so the
second runs over scratch the first left full of its own partials: token ids
and flags must be identical, the logits bit-identical, and the token the
oracle's.
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from inferno_hip import synth

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def say(*a):
    print("[case]", *a, flush=True)


def _both(L, t, w, x, vocab, hidden, with_logits):
    s = torch.cuda.current_stream().cuda_stream
    out = []
    for noalloc in (False, True):
        tok = torch.full((1,), -1, dtype=torch.int32, device="cuda")
        fl = torch.full((1,), 0x7F, dtype=torch.int32, device="cuda")
        lg = torch.full((vocab,), float("nan"), device="cuda") if with_logits else None
        lp = lg.data_ptr() if lg is not None else None
        if noalloc:
            rc = L.ihip_lm_head_argmax_noalloc_dev(t, w.data_ptr(), x.data_ptr(), lp, tok.data_ptr(),
                                                   fl.data_ptr(), hidden, vocab, s)
        else:
            ws = torch.empty(262144, dtype=torch.uint8, device="cuda")
            rc = L.ihip_lm_head_argmax_dev(t, w.data_ptr(), x.data_ptr(), lp, tok.data_ptr(),
                                           fl.data_ptr(), hidden, vocab, ws.data_ptr(), s)
        assert rc == 0, L.ihip_last_error().decode()
        torch.cuda.synchronize()
        out.append((int(tok.item()), int(fl.item()), None if lg is None else lg.cpu().numpy()))
    return out


@pytest.mark.parametrize("with_logits", [True, False])
def test_noalloc_lm_head_matches_the_workspace_entry_point(with_logits):
    from inferno_hip import _lib
    L = _lib.lib()
    cases = [(synth.Q6_K, 151936, 2048, 0xC2),   # the lm_head workload: 768 partials
             (synth.Q6_K, 32000, 2048, 0x33),    # smaller: fewer partials over stale ones
             (synth.Q8_0, 1000, 2048, 0x34)]
    if with_logits:
        cases.append((synth.Q4_K, 5003, 1024, 0x35))  # GEMV, then the standalone argmax
    for t, vocab, hidden, seed in cases:
        say(f"noalloc lm_head type={t} vocab={vocab} hidden={hidden} logits={with_logits}")
        rng = synth.rng_for(seed)
        w = synth.weight(rng, t, vocab, hidden)
        x = synth.activations(rng, hidden)
        wd, xd = torch.from_numpy(w).cuda(), torch.from_numpy(x).cuda()
        (t0, f0, l0), (t1, f1, l1) = _both(L, t, wd, xd, vocab, hidden, with_logits)
        assert (t1, f1) == (t0, f0)
        if with_logits:
            assert np.array_equal(l1.view(np.uint32), l0.view(np.uint32))
        ref = oracle.gemv_f64(t, w, x, hidden, vocab)
        assert t1 == int(np.argmax(ref)) and f1 == 0


def test_noalloc_lm_head_flags_nonfinite_logits():
    from inferno_hip import _lib
    L = _lib.lib()
    t, vocab, hidden = synth.Q6_K, 4096, 2048
    rng = synth.rng_for(0x36)
    w = synth.weight(rng, t, vocab, hidden)
    x = synth.activations(rng, hidden)
    x[5] = np.nan
    say("noalloc lm_head with a NaN in x")
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    fl = torch.zeros(1, dtype=torch.int32, device="cuda")
    wd, xd = torch.from_numpy(w).cuda(), torch.from_numpy(x).cuda()  # held until the kernels have run
    rc = L.ihip_lm_head_argmax_noalloc_dev(t, wd.data_ptr(), xd.data_ptr(), None,
                                           tok.data_ptr(), fl.data_ptr(), hidden, vocab,
                                           torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert int(fl.item()) & _lib.FLAG_NAN
