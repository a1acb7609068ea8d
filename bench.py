#!/usr/bin/env python3
"""Decode hot-path benchmark of the MI355X K-quant library (one GPU).

Headline: Q4_K dequant-fused GEMV, 4096 rows x 4096 columns, batch 1, fp32
activations (16 Q4_K super-blocks of 144 B per row), weights and x resident
in HBM.

Step.  The 9.4 MB weight fits in the 256 MB Infinity Cache, so the benchmark
keeps 64 device copies of it (604 MB) and one step is one sweep over all of
them: 64 GEMV launches back to back, each on a different copy, the way a
decode step walks distinct layers; every launch reads its weight from HBM.
A sweep is one replay of a HIP graph of the 64 launches (so the host's
per-call cost does not starve the GPU); `--steps K` times K whole sweeps
between two HIP events recorded on the stream the graph replays on.
`value` = algorithmic bytes (weight + x + y, each touched once) x 64 x K /
elapsed; the per-launch time is elapsed / (64 K), reported as
config.us_per_launch and used for the roofline.

Also reported (`extras`): the floors a single launch of this size cannot
beat (an empty launch of the same grid, and a fully coalesced read of the
same 9.4 MB that discards the bytes), the host-pointer drop-in's per-call
time (x in, y out over PCIe: what a Julia caller of q4_k_gemv! sees), the
decode FFN block (gate/up Q4_K 12288x4096 with the SwiGLU epilogue, then the
Q6_K 4096x12288 down projection) in microseconds, Q8_0 4096x4096 dequant and
GEMV, the IQ4_NL GEMV, the int8-activation variant, the Q6_K 151936x2048
lm_head with fused argmax (and with the final rmsnorm in front), loading those weights from a GGUF file into the device registry,
the 512-token Q4_K prefill GEMM, single-launch latency and the
cache-resident rate, each labelled.  The FFN block, lm_head and prefill
(20 us or more per call) are timed both as graph sweeps and as launches
issued one by one on the stream; each reports the lower, both are listed.

cpu_baseline: the reference's own C kernels (src/kernels/quant_kernels.c,
compiled from source into oracle/_ref) -- q4_k_gemv on the same workload at
the reference's default thread count and on all of this host's cores -- and
the oracle's restatement of the single-threaded fp32 fallback
(src/ModelCPU.jl:290-306), weights rotated through more than twice the last
level cache, median and spread of 7 repetitions.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only gemv]
       python bench.py --sweep     GEMV of every format over common model shapes,
                                   beside a plain read of the same bytes (a markdown table)
       python bench.py --floors    empty-launch and read floors over launch shapes
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "inferno.jl_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "Q4_K GEMV 4096² achieved HBM GB/s (% of peak); FFN-block decode µs"
PEAK_HBM_GBS = 8000.0
PEAK_FP16_TFLOPS = 2500.0
MALL_BYTES = 256 << 20
WARM_S = 0.05  # seconds of the same launches run before each timed region
NCOPY = 64     # weight copies of the headline GEMV = launches per step


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100, help="timed sweeps of 64 GEMV launches")
    ap.add_argument("--warmup", type=int, default=10, help="untimed sweeps before timing")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default="", help="gemv: the headline GEMV only")
    ap.add_argument("--pmc-workload", action="store_true",
                    help="run the short program the rocprofv3 --pmc runs profile")
    ap.add_argument("--floors", action="store_true",
                    help="sweep the empty-launch and read floors over launch shapes")
    ap.add_argument("--sweep", action="store_true",
                    help="GEMV of every format over common model shapes, beside a plain read of the same bytes")
    return ap.parse_args()


def traffic_bytes():
    """HBM bytes per headline GEMV launch from the committed FETCH_SIZE /
    WRITE_SIZE measurement (each counter scaled by what it reads for a plain
    copy of known size), or None when that record is absent."""
    p = ROOT / "profiles" / "q4k_gemv_4096x4096_traffic.json"
    if not p.exists():
        return None
    d = json.loads(p.read_text())
    g = d["gemv_per_dispatch"]
    return int(round((g["FETCH_SIZE_KiB"] * d["fetch_factor"] + g["WRITE_SIZE_KiB"] * d["write_factor"]) * 1024))


def floors_lib():
    import ctypes as C
    p = ROOT / "inferno.jl_amd" / "lib" / "libinferno_floors.so"
    if not p.exists():
        return None
    L = C.CDLL(str(p))
    L.ifl_empty.argtypes = [C.c_int, C.c_int, C.c_void_p]
    L.ifl_read.argtypes = [C.c_void_p, C.c_uint64, C.c_uint32, C.c_void_p, C.c_int, C.c_int, C.c_void_p]
    L.ifl_empty.restype = L.ifl_read.restype = C.c_int
    return L


# ------------------------------------------------------------------ timing --

class GraphLoop:
    """A HIP graph of `launch(i)` for i in range(n) on `stream`."""

    def __init__(self, torch, stream, n, launch):
        self.torch = torch
        self.stream = stream
        self.n = n
        with torch.cuda.stream(stream):
            for i in range(n):  # eager pass: first-use initialisation stays out of the graph
                launch(i)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=stream):
            for i in range(n):
                launch(i)
        torch.cuda.synchronize()

    def replay(self, times):
        with self.torch.cuda.stream(self.stream):
            for _ in range(times):
                self.graph.replay()


def time_sweeps(torch, stream, launch, n_rot, sweeps, warmup):
    """Time `sweeps` whole replays of a graph of launch(0..n_rot-1) (one sweep
    over n_rot operand sets); returns the ms of the timed region, measured by
    HIP events on `stream`."""
    g = GraphLoop(torch, stream, n_rot, launch)
    g.replay(max(1, warmup))
    torch.cuda.synchronize()
    # The GPU's clock drops while the host sets a workload up (graph capture,
    # uploads) and ramps back over milliseconds of work: keep replaying the
    # same launches until about WARM_S seconds of them have run, so the timed
    # region sees the steady-state clock.
    w0 = time.perf_counter()
    g.replay(1)
    torch.cuda.synchronize()
    per_replay = max(time.perf_counter() - w0, 1e-6)
    g.replay(int(WARM_S / per_replay) + 1)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    g.replay(sweeps)
    t1.record(stream)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1)


def time_stream(torch, stream, launch, n_rot, sweeps):
    """The same launches as time_sweeps, issued one by one on `stream` instead
    of replayed from a graph (what a serving loop does): warmed the same way,
    then `sweeps` whole passes over the n_rot operand sets between HIP events;
    returns ms.  Launches are host-bound below ~10 us, so the legs that use it
    run 20 us or more per launch; on this platform a graph replay adds
    0.5-0.7 us at each dependent kernel boundary that stream launches do not."""
    with torch.cuda.stream(stream):
        for i in range(n_rot):
            launch(i)
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        k = 0
        while time.perf_counter() - w0 < WARM_S:
            launch(k % n_rot)
            k += 1
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for i in range(sweeps * n_rot):
            launch(i % n_rot)
        t1.record(stream)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1)


def both_ways_us(torch, stream, launch, n_rot, sweeps, warmup):
    """us per launch from graph sweeps and from stream launches; the leg
    reports the lower (the same kernels either way)."""
    g = time_sweeps(torch, stream, launch, n_rot, sweeps, warmup) * 1e3 / (sweeps * n_rot)
    st = time_stream(torch, stream, launch, n_rot, sweeps) * 1e3 / (sweeps * n_rot)
    return min(g, st), g, st


def single_launch_us(torch, stream, launch, reps=50):
    ts = []
    for i in range(reps):
        torch.cuda.synchronize()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            a.record(stream)
            launch(i)
            b.record(stream)
        torch.cuda.synchronize()
        ts.append(a.elapsed_time(b) * 1e3)
    return float(np.median(ts))


def copies_for(nbytes, min_total=2 * MALL_BYTES, cap=64):
    return int(min(cap, max(2, -(-min_total // nbytes))))


# ----------------------------------------------------------------- workloads --

def q4k_gemv(torch, stream, synth, D, oracle, steps, warmup):
    outer = inner = 4096
    rng = synth.rng_for(0xC0)
    w = synth.weight(rng, synth.Q4_K, outer, inner)
    x = synth.activations(rng, inner)
    nbytes = w.size + 4 * inner + 4 * outer
    base = torch.from_numpy(w).cuda()
    ws = [D.DeviceWeight(base.clone(), synth.Q4_K, inner, outer) for _ in range(NCOPY)]
    del base
    xd = torch.from_numpy(x).cuda()
    ys = torch.empty(NCOPY, outer, device="cuda")

    # parity of the benched configuration (copy 0) against the oracle
    with torch.cuda.stream(stream):
        D.gemv(ws[0], xd, ys[0])
    torch.cuda.synchronize()
    ref = oracle.gemv_f64(synth.Q4_K, w, x, inner, outer)
    tol = oracle.tolerance(oracle.row_norms(synth.Q4_K, w, inner, outer), x)
    ratio = float(np.max(np.abs(ys[0].cpu().numpy().astype(np.float64) - ref) / tol))
    if ratio > 1.0:
        raise SystemExit(f"Q4_K GEMV parity failed before timing: max err/tol {ratio:.3g}")

    def launch(i):
        D.gemv(ws[i % NCOPY], xd, ys[i % NCOPY])

    ms = time_sweeps(torch, stream, launch, NCOPY, steps, warmup)
    us_per = ms * 1e3 / (steps * NCOPY)
    res = dict(bytes=nbytes, ms=ms, us_per_launch=us_per, gbs=nbytes / (us_per * 1e-6) / 1e9,
               parity_max_err_over_tol=ratio, copies=NCOPY)
    res["single_launch_us"] = single_launch_us(torch, stream, launch)
    ms_res = time_sweeps(torch, stream, lambda i: D.gemv(ws[0], xd, ys[0]), NCOPY, 10, 2)
    res["cache_resident_gbs"] = nbytes / (ms_res * 1e3 / (10 * NCOPY) * 1e-6) / 1e9

    # the floors of one launch of this size, measured the same way
    F = floors_lib()
    if F is not None:
        grid = outer // 16  # the headline kernel's grid: 8 waves x 2 rows per workgroup
        out = torch.zeros(1, dtype=torch.int32, device="cuda")

        def empty(i):
            assert F.ifl_empty(grid, 512, torch.cuda.current_stream().cuda_stream) == 0

        def read(i):
            assert F.ifl_read(ws[i % NCOPY].data.data_ptr(), w.size, 0x9E3779B9, out.data_ptr(),
                              grid, 512, torch.cuda.current_stream().cuda_stream) == 0
        n = 10
        res["floor_empty_us"] = time_sweeps(torch, stream, empty, NCOPY, n, 2) * 1e3 / (n * NCOPY)
        res["floor_read_us"] = time_sweeps(torch, stream, read, NCOPY, n, 2) * 1e3 / (n * NCOPY)

    # the host-pointer drop-in (ihip_q4_k_gemv: x in and y out over PCIe,
    # synchronous, the weight uploaded once and found in the cache)
    from inferno_hip import QuantizedKernels as QK
    out = np.zeros(outer, np.float32)
    QK.q4_k_gemv_(out, w, x, inner, outer)
    reps = []
    for _ in range(5):
        t0 = time.perf_counter()
        for _ in range(100):
            QK.q4_k_gemv_(out, w, x, inner, outer)
        reps.append((time.perf_counter() - t0) / 100 * 1e6)
    res["host_pointer_us"] = float(np.median(reps))
    return res


def ffn_block(torch, stream, synth, D, sweeps=100):
    hidden, inter = 4096, 12288
    rng = synth.rng_for(0xC3)
    wg = synth.weight(rng, synth.Q4_K, inter, hidden)
    wu = synth.weight(rng, synth.Q4_K, inter, hidden)
    wd = synth.weight(rng, synth.Q6_K, hidden, inter)
    x = synth.activations(rng, hidden)
    nbytes = wg.size + wu.size + wd.size + 4 * hidden * 2
    ncopy = copies_for(nbytes)
    g0, u0, d0 = (torch.from_numpy(a).cuda() for a in (wg, wu, wd))
    sets = [(D.DeviceWeight(g0.clone(), synth.Q4_K, hidden, inter),
             D.DeviceWeight(u0.clone(), synth.Q4_K, hidden, inter),
             D.DeviceWeight(d0.clone(), synth.Q6_K, inter, hidden)) for _ in range(ncopy)]
    del g0, u0, d0
    xd = torch.from_numpy(x).cuda()
    hs = torch.empty(ncopy, inter, device="cuda")
    ys = torch.empty(ncopy, hidden, device="cuda")

    def launch(i):
        k = i % ncopy
        D.ffn_swiglu(*sets[k], xd, h=hs[k], y=ys[k])

    us, us_graph, us_stream = both_ways_us(torch, stream, launch, ncopy, sweeps, 4)
    # the same block with the post-attention norm folded into gate/up and the
    # residual add into the down projection (x updated in place: the values
    # drift over the steps, the bytes and launches do not)
    nw = torch.from_numpy(rng.uniform(0.5, 1.5, hidden).astype(np.float32)).cuda()
    xs = torch.from_numpy(np.tile(x, (ncopy, 1))).cuda()

    def launch_norm(i):
        k = i % ncopy
        D.ffn_block(*sets[k], nw, 1e-6, xs[k], h=hs[k])

    us_n = both_ways_us(torch, stream, launch_norm, ncopy, sweeps, 4)[0]
    return dict(us=us, bytes=nbytes, gbs=nbytes / (us * 1e-6) / 1e9, copies=ncopy,
                graph_us=us_graph, stream_us=us_stream,
                single_launch_us=single_launch_us(torch, stream, launch, 20),
                norm_residual_us=us_n)


def q8_0_workloads(torch, stream, synth, D):
    outer = inner = 4096
    rng = synth.rng_for(0xC1)
    w = synth.weight(rng, synth.Q8_0, outer, inner)
    x = synth.activations(rng, inner)
    gemv_bytes = w.size + 8 * inner
    deq_bytes = w.size + 4 * outer * inner
    ncopy = copies_for(deq_bytes)
    base = torch.from_numpy(w).cuda()
    ws = [D.DeviceWeight(base.clone(), synth.Q8_0, inner, outer) for _ in range(ncopy)]
    outs = [torch.empty(outer * inner, device="cuda") for _ in range(ncopy)]
    xd = torch.from_numpy(x).cuda()
    ys = torch.empty(ncopy, outer, device="cuda")
    n = 8
    ms = time_sweeps(torch, stream, lambda i: D.dequantize(ws[i % ncopy], outs[i % ncopy]),
                     ncopy, n, 2)
    deq_us = ms * 1e3 / (n * ncopy)
    gcopy = copies_for(gemv_bytes)
    gws = ws + [D.DeviceWeight(base.clone(), synth.Q8_0, inner, outer)
                for _ in range(max(0, gcopy - ncopy))]
    n = 16
    ms = time_sweeps(torch, stream, lambda i: D.gemv(gws[i % gcopy], xd, ys[i % ncopy]),
                     gcopy, n, 2)
    gemv_us = ms * 1e3 / (n * gcopy)
    return dict(dequant_us=deq_us, dequant_gbs=deq_bytes / (deq_us * 1e-6) / 1e9,
                gemv_us=gemv_us, gemv_gbs=gemv_bytes / (gemv_us * 1e-6) / 1e9)


def iq4nl_gemv(torch, stream, synth, D):
    """IQ4_NL GEMV at 4096x4096 (the keep-quantized format of the SSM
    projections, src/ModelCPU.jl:381-408), weights rotated through HBM."""
    outer = inner = 4096
    rng = synth.rng_for(0xC6)
    w = synth.weight(rng, synth.IQ4_NL, outer, inner)
    x = synth.activations(rng, inner)
    nbytes = w.size + 4 * inner + 4 * outer
    ncopy = copies_for(w.size)
    base = torch.from_numpy(w).cuda()
    ws = [D.DeviceWeight(base.clone(), synth.IQ4_NL, inner, outer) for _ in range(ncopy)]
    xd = torch.from_numpy(x).cuda()
    ys = torch.empty(ncopy, outer, device="cuda")
    n = 16
    ms = time_sweeps(torch, stream, lambda i: D.gemv(ws[i % ncopy], xd, ys[i % ncopy]), ncopy, n, 2)
    us = ms * 1e3 / (n * ncopy)
    return dict(us=us, gbs=nbytes / (us * 1e-6) / 1e9)


def q8k_gemv(torch, stream, synth, D):
    """The int8-activation variant (the reference C numerics) at 4096x4096
    Q4_K: one launch quantizes x to Q8_K and runs the GEMV, weights rotated
    through HBM."""
    outer = inner = 4096
    rng = synth.rng_for(0xC0)
    w = synth.weight(rng, synth.Q4_K, outer, inner)
    x = synth.activations(rng, inner)
    nbytes = w.size + 4 * inner + 4 * outer
    ncopy = copies_for(w.size)
    base = torch.from_numpy(w).cuda()
    ws = [D.DeviceWeight(base.clone(), synth.Q4_K, inner, outer) for _ in range(ncopy)]
    xd = torch.from_numpy(x).cuda()
    ys = torch.empty(ncopy, outer, device="cuda")

    def step(i):
        D.gemv_q8k_x(ws[i % ncopy], xd, ys[i % ncopy])
    n = 16
    ms = time_sweeps(torch, stream, step, ncopy, n, 2)
    us = ms * 1e3 / (n * ncopy)
    return dict(us=us, gbs=nbytes / (us * 1e-6) / 1e9)


def qkv_group(torch, stream, synth, D):
    """The attention's input projections of one decode step
    (src/ModelCPU.jl:789-791): Q4_K wq 4096x4096, wk and wv 1024x4096 on one
    x, as three GEMVs and as one GEMV over the three uploaded back to back
    (ihip_weight_register_group); 16 rotated copies."""
    inner, outers = 4096, (4096, 1024, 1024)
    rng = synth.rng_for(0xC7)
    ws = [synth.weight(rng, synth.Q4_K, o, inner) for o in outers]
    x = torch.from_numpy(synth.activations(rng, inner)).cuda()
    ncopy = 16
    groups = [D.WeightGroup(ws, synth.Q4_K, inner, outers) for _ in range(ncopy)]
    singles = [[D.DeviceWeight(torch.from_numpy(w).cuda(), synth.Q4_K, inner, o)
                for w, o in zip(ws, outers)] for _ in range(ncopy)]
    total = sum(outers)
    ys = torch.empty(ncopy, total, device="cuda")
    offs = groups[0].offsets

    def one(i):
        groups[i % ncopy].gemv(x, ys[i % ncopy])

    def three(i):
        for w, o, r in zip(singles[i % ncopy], offs, outers):
            D.gemv(w, x, ys[i % ncopy, o:o + r])
    us1 = both_ways_us(torch, stream, one, ncopy, 20, 3)[0]
    us3 = both_ways_us(torch, stream, three, ncopy, 20, 3)[0]
    for g in groups:
        g.release()
    nbytes = sum(w.size for w in ws) + 4 * inner + 4 * total
    return dict(group_us=us1, separate_us=us3, group_gbs=nbytes / (us1 * 1e-6) / 1e9)


def decode_layer(torch, stream, synth, D):
    """The quantized work of one decoder layer's decode step
    (src/ModelCPU.jl:900-920) at hidden 4096, K/V projections of 1024 rows,
    intermediate 12288: one grouped GEMV for wq/wk/wv (Q4_K) with the input
    rmsnorm folded in, the output projection wo (Q4_K) with the residual add folded in --
    its input is the q rows, standing in for the attention core, which is
    outside this path -- and the FFN block (post-norm folded into the fused
    Q4_K gate/up pass, Q6_K down with the residual).  Four launches; 4 rotated
    copies of the layer's 121 MB of weights."""
    hid, kv, inter = 4096, 1024, 12288
    rng = synth.rng_for(0xC8)
    ncopy = 4
    qkv_w = [synth.weight(rng, synth.Q4_K, o, hid) for o in (hid, kv, kv)]
    wo = synth.weight(rng, synth.Q4_K, hid, hid)
    wg = synth.weight(rng, synth.Q4_K, inter, hid)
    wu = synth.weight(rng, synth.Q4_K, inter, hid)
    wd = synth.weight(rng, synth.Q6_K, hid, inter)
    layers = []
    for _ in range(ncopy):
        layers.append(dict(
            qkv=D.WeightGroup(qkv_w, synth.Q4_K, hid, (hid, kv, kv)),
            wo=D.DeviceWeight(torch.from_numpy(wo).cuda(), synth.Q4_K, hid, hid),
            wg=D.DeviceWeight(torch.from_numpy(wg).cuda(), synth.Q4_K, hid, inter),
            wu=D.DeviceWeight(torch.from_numpy(wu).cuda(), synth.Q4_K, hid, inter),
            wd=D.DeviceWeight(torch.from_numpy(wd).cuda(), synth.Q6_K, inter, hid)))
    wbytes = sum(w.size for w in qkv_w) + wo.size + wg.size + wu.size + wd.size
    x0 = torch.from_numpy(synth.activations(rng, hid)).cuda()
    n1 = torch.from_numpy(rng.uniform(0.5, 1.5, hid).astype(np.float32)).cuda()
    n2 = torch.from_numpy(rng.uniform(0.5, 1.5, hid).astype(np.float32)).cuda()
    xn, x1 = torch.empty(hid, device="cuda"), torch.empty(hid, device="cuda")
    qkv = torch.empty(hid + 2 * kv, device="cuda")
    h = torch.empty(inter + hid, device="cuda")

    def step(i):
        L = layers[i % ncopy]
        L["qkv"].gemv_norm(n1, 1e-6, x0, qkv, xn=xn)  # the input norm folded in
        D.gemv_add(L["wo"], qkv[:hid], x0, out=x1)
        D.ffn_block(L["wg"], L["wu"], L["wd"], n2, 1e-6, x1, h=h)
    us = both_ways_us(torch, stream, step, ncopy, 20, 3)[0]
    for L in layers:
        L["qkv"].release()
    return dict(us=us, gbs=wbytes / (us * 1e-6) / 1e9, weight_bytes=wbytes)


def lm_head(torch, stream, synth, D):
    vocab, hidden = 151936, 2048
    rng = synth.rng_for(0xC2)
    w = synth.weight(rng, synth.Q6_K, vocab, hidden)
    x = synth.activations(rng, hidden)
    nbytes = w.size + 4 * hidden + 4 * vocab + 4
    ncopy = 3
    base = torch.from_numpy(w).cuda()
    del w
    ws = [D.DeviceWeight(base.clone(), synth.Q6_K, hidden, vocab) for _ in range(ncopy)]
    del base
    xd = torch.from_numpy(x).cuda()
    logits = torch.empty(ncopy, vocab, device="cuda")
    aws = [D.ArgmaxWorkspace() for _ in range(ncopy)]

    def launch(i):
        k = i % ncopy
        D.lm_head_argmax(ws[k], xd, aws[k], logits=logits[k])

    us, us_graph, us_stream = both_ways_us(torch, stream, launch, ncopy, 20, 4)
    tok = aws[0].result()
    # the final norm folded in front (src/ModelCPU.jl:1014-1015): rmsnorm of
    # the hidden state into caller scratch, then the same lm_head
    nw = torch.from_numpy(rng.uniform(0.5, 1.5, hidden).astype(np.float32)).cuda()
    xn = torch.empty_like(xd)

    def launch_norm(i):
        k = i % ncopy
        D.lm_head_argmax_norm(ws[k], nw, 1e-6, xd, aws[k], xn=xn, logits=logits[k])

    us_n = both_ways_us(torch, stream, launch_norm, ncopy, 20, 4)[0]
    return dict(us=us, gbs=nbytes / (us * 1e-6) / 1e9, token=tok, graph_us=us_graph,
                stream_us=us_stream, norm_us=us_n)


def prefill(torch, stream, synth, D):
    T, outer, inner = 512, 4096, 4096
    rng = synth.rng_for(0xC4)
    w = synth.weight(rng, synth.Q4_K, outer, inner)
    X = rng.standard_normal((T, inner)).astype(np.float32)
    dw = D.DeviceWeight(torch.from_numpy(w).cuda(), synth.Q4_K, inner, outer)
    Xd = torch.from_numpy(X).cuda()
    Y = torch.empty(T, outer, device="cuda")
    xh = D.prefill_scratch(T, inner)
    us, us_graph, us_stream = both_ways_us(torch, stream, lambda i: D.prefill_q4_k(dw, Xd, Y, xh),
                                           10, 5, 4)
    flops = 2.0 * T * outer * inner
    # three weights on one input (the attention's wq, wk, wv,
    # src/ModelCPU.jl:789-791): one rounding of X, three products
    dws = [dw] + [D.DeviceWeight(dw.data.clone(), synth.Q4_K, inner, outer) for _ in range(2)]
    Ys = [Y] + [torch.empty_like(Y) for _ in range(2)]

    def shared(i):
        D.prefill_convert(Xd, xh)
        for k in range(3):
            D.prefill_q4_k_xh(dws[k], xh, T, Ys[k])

    def separate(i):
        for k in range(3):
            D.prefill_q4_k(dws[k], Xd, Ys[k], xh)
    us3_shared = both_ways_us(torch, stream, shared, 4, 5, 2)[0]
    us3_separate = both_ways_us(torch, stream, separate, 4, 5, 2)[0]
    return dict(us=us, tflops=flops / (us * 1e-6) / 1e12,
                mfma_frac=flops / (us * 1e-6) / 1e12 / PEAK_FP16_TFLOPS, graph_us=us_graph,
                stream_us=us_stream, shared3_us=us3_shared, separate3_us=us3_separate)


def write_gguf(path, tensors, alignment=32):
    """A GGUF v3 file (the layout src/GGUF.jl:119-165 reads): no key/values,
    tensor infos (name, dims with ne0 first, GGML type, offset), then the
    aligned data section."""
    import struct
    infos, offs, off = b"", [], 0
    for name, gt, dims, blob in tensors:
        off = -(-off // alignment) * alignment
        offs.append(off)
        nb = name.encode()
        infos += struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(dims))
        infos += b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", gt, off)
        off += blob.size
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), 0) + infos
    with open(path, "wb") as f:
        f.write(head + b"\0" * (-len(head) % alignment))
        base = f.tell()
        for (_, _, _, blob), o in zip(tensors, offs):
            f.seek(base + o)
            blob.tofile(f)


def gguf_load(torch, synth, D):
    """The GGUF-fed weight registry (inferno.jl_amd/csrc/gguf.hip) on the
    decode weights benched above: a file holding the FFN block's three
    weights and the 151936x2048 lm_head is opened (memory-mapped, header and
    tensor infos parsed) and every tensor uploaded into the device registry;
    the file is in the page cache, as after a first load.  Bytes per second
    of the whole open + upload, and the uploaded bytes checked."""
    import tempfile
    from inferno_hip import GGUF, _lib
    rng = synth.rng_for(0xC5)
    specs = [("blk.0.ffn_gate.weight", synth.Q4_K, 4096, 12288),
             ("blk.0.ffn_up.weight", synth.Q4_K, 4096, 12288),
             ("blk.0.ffn_down.weight", synth.Q6_K, 12288, 4096),
             ("output.weight", synth.Q6_K, 2048, 151936)]
    tensors = [(n, t, (inner, outer), synth.weight(rng, t, outer, inner)) for n, t, inner, outer in specs]
    nbytes = sum(b.size for *_, b in tensors)
    fd, path = tempfile.mkstemp(suffix=".gguf")
    os.close(fd)
    try:
        write_gguf(path, tensors)
        times, opens = [], []
        for rep in range(3):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            f = GGUF.read_gguf(path)
            t1 = time.perf_counter()
            handles = [GGUF.upload(f, n) for n, *_ in tensors]
            torch.cuda.synchronize()
            t2 = time.perf_counter()
            opens.append(t1 - t0)
            times.append(t2 - t0)
            if rep == 0:  # the uploaded gate weight gives the same GEMV as its bytes
                n, t, (inner, outer), blob = tensors[0]
                x = torch.from_numpy(synth.activations(rng, inner)).cuda()
                y_reg = torch.empty(outer, device="cuda")
                _lib.check(_lib.lib().ihip_gemv_dev(t, GGUF.device_ptr(handles[0]), x.data_ptr(),
                                                    y_reg.data_ptr(), inner, outer,
                                                    torch.cuda.current_stream().cuda_stream))
                y_ref = D.gemv(D.DeviceWeight(torch.from_numpy(blob).cuda(), t, inner, outer), x)
                torch.cuda.synchronize()
                if not torch.equal(y_reg, y_ref):
                    raise AssertionError("GGUF-uploaded weight gives a different GEMV")
            for h in handles:
                _lib.check(_lib.lib().ihip_weight_release(h))
            f.close()
    finally:
        os.unlink(path)
    s = float(np.median(times))
    return dict(bytes=nbytes, s=s, gbs=nbytes / s / 1e9, open_ms=float(np.median(opens)) * 1e3)


def pmc_workload(torch, synth, D):
    """The program the rocprofv3 --pmc runs profile: a device copy of known
    size (to calibrate FETCH_SIZE / WRITE_SIZE) and a few launches of each
    benched kernel with its weights rotated through HBM."""
    src = torch.empty(64 << 20, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    w = synth.weight(synth.rng_for(0xC0), synth.Q4_K, 4096, 4096)
    base = torch.from_numpy(w).cuda()
    ws = [D.DeviceWeight(base.clone(), synth.Q4_K, 4096, 4096) for _ in range(NCOPY)]
    x = torch.from_numpy(synth.activations(synth.rng_for(0xC0 + 1), 4096)).cuda()
    ys = torch.empty(NCOPY, 4096, device="cuda")
    for _ in range(3):
        for i in range(NCOPY):
            D.gemv(ws[i], x, ys[i])
    torch.cuda.synchronize()
    del ws, base
    # FFN block: 6 sets of gate/up + down
    hidden, inter = 4096, 12288
    rng = synth.rng_for(0xC3)
    wg, wu = (synth.weight(rng, synth.Q4_K, inter, hidden) for _ in range(2))
    wd = synth.weight(rng, synth.Q6_K, hidden, inter)
    g0, u0, d0 = (torch.from_numpy(a).cuda() for a in (wg, wu, wd))
    sets = [(D.DeviceWeight(g0.clone(), synth.Q4_K, hidden, inter),
             D.DeviceWeight(u0.clone(), synth.Q4_K, hidden, inter),
             D.DeviceWeight(d0.clone(), synth.Q6_K, inter, hidden)) for _ in range(6)]
    h = torch.empty(inter, device="cuda")
    y = torch.empty(hidden, device="cuda")
    for _ in range(4):
        for s in sets:
            D.ffn_swiglu(*s, x, h=h, y=y)
    torch.cuda.synchronize()
    del sets, g0, u0, d0
    # lm_head: 3 copies
    vocab = 151936
    wl = synth.weight(synth.rng_for(0xC2), synth.Q6_K, vocab, 2048)
    b = torch.from_numpy(wl).cuda()
    del wl
    ls = [D.DeviceWeight(b.clone(), synth.Q6_K, 2048, vocab) for _ in range(3)]
    del b
    xl = x[:2048].contiguous()
    logits = torch.empty(vocab, device="cuda")
    aw = D.ArgmaxWorkspace()
    for _ in range(4):
        for lw in ls:
            D.lm_head_argmax(lw, xl, aw, logits=logits)
    torch.cuda.synchronize()
    del ls
    # prefill 512 x 4096 x 4096
    dw = D.DeviceWeight(torch.from_numpy(w).cuda(), synth.Q4_K, 4096, 4096)
    X = torch.randn(512, 4096, device="cuda")
    Y = torch.empty(512, 4096, device="cuda")
    xh = D.prefill_scratch(512, 4096)
    for _ in range(10):
        D.prefill_q4_k(dw, X, Y, xh)
    torch.cuda.synchronize()
    print("pmc workload done: 3 x 64 MiB copy, 192 Q4_K 4096x4096 GEMVs, 24 FFN blocks, "
          "12 lm_heads, 10 prefills", flush=True)


def floors_sweep(torch, stream):
    """Per-launch cost of an empty launch and of a fully coalesced read of
    9437184 bytes (and of twice that: the difference is the transfer time of
    the bytes alone) over launch shapes, 64 rotated buffers, HIP graph."""
    F = floors_lib()
    if F is None:
        raise SystemExit("inferno.jl_amd/lib/libinferno_floors.so is not built")
    nb = 9437184
    big = torch.empty(NCOPY, 2 * nb, dtype=torch.uint8, device="cuda").random_(0, 255)
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    cs = lambda: torch.cuda.current_stream().cuda_stream

    def per_launch(fn, sweeps=10):
        return time_sweeps(torch, stream, fn, NCOPY, sweeps, 2) * 1e3 / (sweeps * NCOPY)
    print("| launch | grid x block | us per launch |\n|---|---|---|", flush=True)
    for g, b in ((1, 64), (256, 64), (256, 512), (1024, 256), (2048, 256), (4096, 256)):
        us = per_launch(lambda i: F.ifl_empty(g, b, cs()))
        print(f"| empty | {g} x {b} | {us:.3f} |", flush=True)
    print("\n| read | grid x block | 9437184 B us | 2 x 9437184 B us | marginal us | marginal GB/s |\n"
          "|---|---|---|---|---|---|", flush=True)
    for g, b in ((128, 1024), (256, 512), (512, 512), (1024, 256), (2048, 256)):
        r = [per_launch(lambda i: F.ifl_read(big[i].data_ptr(), n, 0x9E3779B9, out.data_ptr(), g, b, cs()))
             for n in (nb, 2 * nb)]
        print(f"| read | {g} x {b} | {r[0]:.3f} | {r[1]:.3f} | {r[1] - r[0]:.3f} | "
              f"{nb / (r[1] - r[0]) / 1e3:.0f} |", flush=True)


SWEEP_SHAPES = (
    # (format name, outer, inner): the projections of 7B-70B-class and
    # 1.5B-class decoders, and the vocabulary heads
    ("Q4_K", 4096, 4096), ("Q4_K", 12288, 4096), ("Q4_K", 11008, 4096), ("Q4_K", 4096, 11008),
    ("Q4_K", 14336, 4096), ("Q4_K", 4096, 14336), ("Q4_K", 2048, 2048), ("Q4_K", 5120, 5120),
    ("Q4_K", 13824, 5120), ("Q4_K", 5120, 13824), ("Q4_K", 8192, 8192), ("Q4_K", 28672, 8192),
    ("Q4_K", 8192, 28672),
    ("Q5_K", 4096, 4096), ("Q5_K", 14336, 4096), ("Q5_K", 4096, 14336),
    ("Q6_K", 4096, 4096), ("Q6_K", 4096, 14336), ("Q6_K", 32000, 4096), ("Q6_K", 151936, 2048),
    ("Q6_K", 128256, 4096),
    ("Q8_0", 4096, 4096), ("Q8_0", 14336, 4096), ("Q8_0", 4096, 14336),
    ("IQ4_NL", 4096, 4096), ("IQ4_NL", 14336, 4096),
)


def shape_sweep(torch, stream, synth, D):
    """One GEMV per shape of SWEEP_SHAPES, weights rotated through enough
    copies to leave the 256 MB MALL, HIP graph sweeps; beside it a fully
    coalesced read of the same weight bytes (the floor a launch of that size
    cannot beat).  Prints a markdown table.  The weights repeat a slab of at
    most 2048 synthetic rows (the GEMV's time does not depend on the values)."""
    F = floors_lib()
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    cs = lambda: torch.cuda.current_stream().cuda_stream
    print("| format | outer x inner | weight MB | copies | GEMV us | GB/s | % of 8 TB/s | read us | GEMV / read |\n"
          "|---|---|---|---|---|---|---|---|---|", flush=True)
    for name, outer, inner in SWEEP_SHAPES:
        t = getattr(synth, name)
        rows = min(outer, 2048)
        rng = synth.rng_for(0xD0 + t)
        slab = torch.from_numpy(synth.weight(rng, t, rows, inner)).cuda()
        row_bytes = slab.numel() // rows
        reps = -(-outer // rows)
        base = slab.repeat(reps)[: outer * row_bytes].contiguous()
        del slab
        wbytes = base.numel()
        nbytes = wbytes + 4 * inner + 4 * outer
        ncopy = copies_for(wbytes)
        ws = [D.DeviceWeight(base.clone(), t, inner, outer) for _ in range(ncopy)]
        del base
        xd = torch.from_numpy(synth.activations(rng, inner)).cuda()
        ys = torch.empty(ncopy, outer, device="cuda")
        sweeps = max(8, min(64, int(2e10 // (wbytes * ncopy))))  # 4-10 ms timed per shape
        ms = time_sweeps(torch, stream, lambda i: D.gemv(ws[i % ncopy], xd, ys[i % ncopy]), ncopy, sweeps, 2)
        us = ms * 1e3 / (sweeps * ncopy)
        read = ""
        ratio = ""
        if F is not None:
            n = wbytes // 16 * 16
            grid = max(1024, -(-(n // 16) // (256 * 8)))
            rms = time_sweeps(torch, stream, lambda i: F.ifl_read(ws[i % ncopy].data.data_ptr(), n, 0x9E3779B9,
                                                                  out.data_ptr(), grid, 256, cs()),
                              ncopy, sweeps, 2)
            rus = rms * 1e3 / (sweeps * ncopy)
            read = f"{rus:.2f}"
            ratio = f"{us / rus:.2f}"
        gbs = nbytes / (us * 1e-6) / 1e9
        print(f"| {name} | {outer} x {inner} | {wbytes / 1e6:.1f} | {ncopy} | {us:.2f} | {gbs:.0f} | "
              f"{100 * gbs / PEAK_HBM_GBS:.1f} | {read} | {ratio} |", flush=True)
        del ws, xd, ys
        torch.cuda.empty_cache()


# --------------------------------------------------------------- CPU baseline --

def _host_info():
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    nproc = os.cpu_count() or 1
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = nproc
    l3 = 0
    base = Path("/sys/devices/system/cpu/cpu0/cache")
    for idx in sorted(base.glob("index*")) if base.exists() else []:
        try:
            if (idx / "level").read_text().strip() == "3":
                s = (idx / "size").read_text().strip()
                mul = {"K": 1024, "M": 1 << 20, "G": 1 << 30}.get(s[-1], 1)
                l3 = int(s.rstrip("KMG")) * mul
                ids = {c.read_text().strip() for c in Path("/sys/devices/system/cpu").glob(
                    "cpu[0-9]*/cache/" + idx.name + "/shared_cpu_list")}
                l3 *= max(1, len(ids))  # every distinct L3 slice of the host
        except (OSError, ValueError):
            pass
    return model, nproc, avail, l3


def cpu_baseline(synth, oracle):
    """The reference's CPU path timed three ways: the C int8 path at the
    reference's default thread count and on all cores, and the fp32 fallback
    single-threaded; weights
    rotated through more than twice the L3; median and spread of 7 runs."""
    import ctypes
    outer = inner = 4096
    rng = synth.rng_for(0xC0)
    w = synth.weight(rng, synth.Q4_K, outer, inner)
    x = synth.activations(rng, inner)
    nbytes = w.size + 8 * inner
    model, nproc, avail, l3 = _host_info()
    ncopy = max(16, -(-2 * max(l3, 64 << 20) // w.size) + 1)
    ws = [w.copy() for _ in range(ncopy)]
    # the box's CPU share: OMP_NUM_THREADS when set, else the affinity mask
    env = os.environ.get("OMP_NUM_THREADS")
    all_cores = int(env) if env and env.isdigit() else avail
    default_threads = max(2, min(8, nproc // 2))  # src/QuantizedKernels.jl:40-41
    try:
        gomp = ctypes.CDLL("libgomp.so.1")
    except OSError:
        gomp = None
    ref = oracle.ref_lib()
    kind = "reference" if ref is not None else "port"
    out = np.empty(outer, np.float32)
    q8 = np.zeros(inner // 256 * oracle.Q8K_BYTES, np.uint8)
    if ref is not None:
        def int8_call(k):
            ref.q4_k_gemv(ws[k], x, out, q8, inner, outer)
    else:
        def int8_call(k):
            oracle.lib().orc_gemv_q8k(synth.Q4_K, ws[k], x, out, q8, inner, outer)

    def f32_call(k):
        oracle.lib().orc_gemv_f32_serial(synth.Q4_K, ws[k], x, out, inner, outer)

    def runs(call, calls_per_rep, reps=7):
        k = 0
        for _ in range(min(ncopy, calls_per_rep)):   # warm-up
            call(k % ncopy)
            k += 1
        ms = []
        for _ in range(reps):
            t0 = time.perf_counter()
            for _ in range(calls_per_rep):
                call(k % ncopy)
                k += 1
            ms.append((time.perf_counter() - t0) / calls_per_rep * 1e3)
        return ms

    results = []
    for label, threads, call in (("int8 reference C, default threads", default_threads, int8_call),
                                 ("int8 reference C, all cores", all_cores, int8_call),
                                 ("fp32 fallback, one thread", 1, f32_call)):
        if gomp is not None:
            gomp.omp_set_num_threads(threads)
        call(0)  # cold first call, not counted
        t0 = time.perf_counter()
        for k in range(10):
            call(k % ncopy)
        one = (time.perf_counter() - t0) / 10
        per_rep = max(3, int(1.0 / max(one, 1e-5)))  # up to about 1 s per repetition
        ms = runs(call, per_rep)
        med = float(np.median(ms))
        results.append(dict(path=label, threads=threads, median_ms=med, min_ms=float(min(ms)),
                            max_ms=float(max(ms)), calls_per_rep=per_rep, reps=len(ms),
                            gbs=nbytes / (med * 1e-3) / 1e9))
        log(f"  {label} ({threads} thr): {med:.3f} ms median [{min(ms):.3f}, {max(ms):.3f}]")
    if gomp is not None:
        gomp.omp_set_num_threads(all_cores)
    head = results[0]
    what = ("the reference's src/kernels/quant_kernels.c q4_k_gemv compiled from source"
            if kind == "reference" else "the oracle's restatement of quant_kernels.c q4_k_gemv")
    return dict(value=head["gbs"], unit="GB/s", cores=head["threads"], kind=kind,
                sample=(f"{what} (int8-activation path) on the 4096x4096 Q4_K GEMV at the "
                        f"reference's default clamp(nproc/2, 2, 8) = {head['threads']} threads: "
                        f"median {head['median_ms']:.3f} ms per call over 7 repetitions of "
                        f"{head['calls_per_rep']} calls, {ncopy} rotated weight copies "
                        f"({ncopy * w.size / 2**20:.0f} MiB, > 2x the {l3 / 2**20:.0f} MiB L3)"),
                cpu_model=model, nproc=nproc, affinity=avail, l3_bytes=l3, copies=ncopy,
                runs=results)


# ----------------------------------------------------------------------- main --

def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    import oracle
    from inferno_hip import _lib, synth
    from inferno_hip import device as D

    if not torch.cuda.is_available() or not _lib.available():
        raise SystemExit("bench.py needs an MI355X (gfx950) and libinferno_hip.so")
    torch.cuda.set_device(0)
    if args.pmc_workload:
        pmc_workload(torch, synth, D)
        return
    stream = torch.cuda.Stream()
    if args.floors:
        floors_sweep(torch, stream)
        return
    if args.sweep:
        shape_sweep(torch, stream, synth, D)
        return
    steps, warmup = max(1, args.steps), max(0, args.warmup)

    log(f"Q4_K GEMV 4096x4096: warmup {warmup} sweeps, {steps} timed sweeps of {NCOPY} launches")
    g = q4k_gemv(torch, stream, synth, D, oracle, steps, warmup)
    log(f"  {g['us_per_launch']:.3f} us/launch, {g['gbs']:.1f} GB/s, single {g['single_launch_us']:.2f} us")
    extras = {"q4k_gemv_us_per_launch": g["us_per_launch"],
              "q4k_gemv_single_launch_us": g["single_launch_us"],
              "q4k_gemv_cache_resident_gbs": g["cache_resident_gbs"],
              "q4k_gemv_parity_max_err_over_tol": g["parity_max_err_over_tol"],
              "q4k_gemv_weight_copies": g["copies"],
              "q4k_gemv_host_pointer_us": g["host_pointer_us"]}
    if "floor_empty_us" in g:
        log(f"  floors: empty launch {g['floor_empty_us']:.3f} us, coalesced read of the weight "
            f"{g['floor_read_us']:.3f} us; host-pointer call {g['host_pointer_us']:.1f} us")
        extras.update(floor_empty_launch_us=g["floor_empty_us"],
                      floor_read_9437184B_us=g["floor_read_us"],
                      floor_read_gbs=9437184 / (g["floor_read_us"] * 1e-6) / 1e9)
    if args.only != "gemv":
        log("FFN block 4096/12288")
        f = ffn_block(torch, stream, synth, D)
        log(f"  {f['us']:.2f} us, {f['gbs']:.1f} GB/s (graph {f['graph_us']:.2f}, stream {f['stream_us']:.2f})")
        log(f"  with the rmsnorm and residual folded in: {f['norm_residual_us']:.2f} us")
        extras.update(ffn_block_us=f["us"], ffn_block_gbs=f["gbs"], ffn_block_frac=f["gbs"] / PEAK_HBM_GBS,
                      ffn_block_graph_us=f["graph_us"], ffn_block_stream_us=f["stream_us"],
                      ffn_block_single_launch_us=f["single_launch_us"],
                      ffn_block_norm_residual_us=f["norm_residual_us"])
        log("Q8_0 4096x4096 dequant and GEMV")
        q = q8_0_workloads(torch, stream, synth, D)
        log(f"  dequant {q['dequant_us']:.2f} us ({q['dequant_gbs']:.0f} GB/s), gemv {q['gemv_us']:.2f} us ({q['gemv_gbs']:.0f} GB/s)")
        extras.update({f"q8_0_{k}": v for k, v in q.items()})
        log("IQ4_NL 4096x4096 GEMV")
        iq = iq4nl_gemv(torch, stream, synth, D)
        log(f"  {iq['us']:.2f} us, {iq['gbs']:.0f} GB/s")
        extras.update(iq4_nl_gemv_us=iq["us"], iq4_nl_gemv_gbs=iq["gbs"])
        log("Q4_K GEMV 4096x4096, int8-activation variant (quantize + GEMV)")
        k8 = q8k_gemv(torch, stream, synth, D)
        log(f"  {k8['us']:.2f} us, {k8['gbs']:.0f} GB/s")
        extras.update(q4k_gemv_q8k_us=k8["us"], q4k_gemv_q8k_gbs=k8["gbs"])
        log("attention input projections, Q4_K 4096+1024+1024 rows x 4096")
        qk = qkv_group(torch, stream, synth, D)
        log(f"  one grouped GEMV {qk['group_us']:.2f} us ({qk['group_gbs']:.0f} GB/s), "
            f"three GEMVs {qk['separate_us']:.2f} us")
        extras.update(qkv_group_gemv_us=qk["group_us"], qkv_group_gemv_gbs=qk["group_gbs"],
                      qkv_three_gemvs_us=qk["separate_us"])
        log("decode layer: grouped wq/wk/wv with the norm, wo + residual, FFN block (hidden 4096)")
        dl = decode_layer(torch, stream, synth, D)
        log(f"  {dl['us']:.2f} us per layer, {dl['gbs']:.0f} GB/s over {dl['weight_bytes'] / 1e6:.0f} MB of weights")
        extras.update(decode_layer_us=dl["us"], decode_layer_gbs=dl["gbs"])
        log("Q6_K lm_head 151936x2048 + argmax")
        lm = lm_head(torch, stream, synth, D)
        log(f"  {lm['us']:.2f} us, {lm['gbs']:.0f} GB/s (graph {lm['graph_us']:.2f}, stream {lm['stream_us']:.2f})")
        log(f"  with the final rmsnorm in front: {lm['norm_us']:.2f} us")
        extras.update(lm_head_argmax_us=lm["us"], lm_head_argmax_gbs=lm["gbs"],
                      lm_head_argmax_graph_us=lm["graph_us"], lm_head_argmax_stream_us=lm["stream_us"],
                      lm_head_argmax_norm_us=lm["norm_us"])
        log("GGUF file -> device weight registry")
        gg = gguf_load(torch, synth, D)
        log(f"  {gg['bytes'] / 1e6:.0f} MB in {gg['s'] * 1e3:.1f} ms ({gg['gbs']:.1f} GB/s; open {gg['open_ms']:.2f} ms)")
        extras.update(gguf_upload_bytes=gg["bytes"], gguf_upload_ms=gg["s"] * 1e3, gguf_upload_gbs=gg["gbs"],
                      gguf_open_ms=gg["open_ms"])
        log("prefill 512x4096x4096")
        p = prefill(torch, stream, synth, D)
        log(f"  {p['us']:.1f} us, {p['tflops']:.1f} TFLOP/s (graph {p['graph_us']:.2f}, stream {p['stream_us']:.2f})")
        log(f"  three weights on one X: {p['shared3_us']:.1f} us with one rounding, "
            f"{p['separate3_us']:.1f} us as three calls")
        extras.update(prefill_us=p["us"], prefill_tflops=p["tflops"], prefill_mfma_frac=p["mfma_frac"],
                      prefill_graph_us=p["graph_us"], prefill_stream_us=p["stream_us"],
                      prefill_3_weights_shared_x_us=p["shared3_us"],
                      prefill_3_weights_separate_us=p["separate3_us"])

    cpu = None
    if not args.no_cpu:
        log("CPU baseline")
        cpu = cpu_baseline(synth, oracle)
        log(f"  {cpu['cpu_model']}, nproc {cpu['nproc']}, L3 {cpu['l3_bytes'] >> 20} MiB")

    roofline = {"bound": "hbm", "achieved": round(g["gbs"], 2), "peak": PEAK_HBM_GBS,
                "unit": "GB/s", "frac": round(g["gbs"] / PEAK_HBM_GBS, 4), "traffic": traffic_bytes()}
    if "floor_read_us" in g:
        # the same weight bytes read fully coalesced by a launch of the same
        # grid: the per-launch time this launch shape cannot beat
        roofline["floor_us"] = round(g["floor_read_us"], 4)
        roofline["frac_of_floor"] = round(g["floor_read_us"] / g["us_per_launch"], 4)
    line = {
        "metric": METRIC,
        "value": round(g["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": g["ms"] / steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "Q4_K dequant-fused GEMV 4096x4096, batch 1, fp32 x; one step = "
                               f"one sweep of {NCOPY} launches over {NCOPY} weight copies "
                               "(HBM-resident, not cache-resident)",
                   "rows": 4096, "cols": 4096, "weight_bytes": 9437184,
                   "launches_per_step": NCOPY,
                   "us_per_launch": round(g["us_per_launch"], 4),
                   "algorithmic_bytes_per_launch": g["bytes"],
                   "algorithmic_bytes_per_step": g["bytes"] * NCOPY},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
