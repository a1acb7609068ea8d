#!/usr/bin/env python3
"""Decode hot-path benchmark of the MI355X K-quant library (one GPU).

Headline: Q4_K dequant-fused GEMV, 4096 rows x 4096 columns, batch 1, fp32
activations (16 Q4_K super-blocks of 144 B per row).  One step = one GEMV
launch over one weight matrix with x already resident in HBM.

Timing.  The 9.4 MB weight fits in the 256 MB Infinity Cache, so the timed
loop cycles through 64 device copies of the weight (604 MB), the way a
decode step walks distinct layers; every launch must come from HBM.  The
launches are captured in a HIP graph (one replay = 64 launches) so that the
host's per-call cost does not starve the GPU, and the timed region is a pair
of HIP events recorded on the stream the graph replays on.  `value` is
algorithmic bytes (weight + x + y, each touched once) x steps / elapsed.

Also reported (the `extras` object): the decode FFN block (gate/up Q4_K
12288x4096 with the SwiGLU epilogue, then the Q6_K 4096x12288 down
projection) in microseconds, Q8_0 4096x4096 dequant and GEMV, the Q6_K
151936x2048 lm_head with fused argmax, the 512-token Q4_K prefill GEMM,
single-launch latency and the cache-resident rate, each labelled.

cpu_baseline: the reference's own C kernel (src/kernels/quant_kernels.c,
compiled from source into oracle/_ref) -- q4_k_gemv on the same workload,
timed on this host's cores; the oracle's restatement of it when oracle/_ref
is absent.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only gemv]
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


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=6400)
    ap.add_argument("--warmup", type=int, default=640)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default="", help="gemv: the headline GEMV only")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--pmc-workload", action="store_true",
                    help="run the short program the rocprofv3 --pmc traffic runs profile")
    return ap.parse_args()


def traffic_bytes():
    """HBM bytes per Q4_K GEMV launch from the committed FETCH_SIZE / WRITE_SIZE
    measurement (each counter scaled by what it reads for a plain copy of
    known size), or None when that record is absent."""
    p = ROOT / "profiles" / "q4k_gemv_4096x4096_traffic.json"
    if not p.exists():
        return None
    d = json.loads(p.read_text())
    g = d["gemv_per_dispatch"]
    return int(round((g["FETCH_SIZE_KiB"] * d["fetch_factor"] + g["WRITE_SIZE_KiB"] * d["write_factor"]) * 1024))


def pmc_workload(torch, synth, D):
    src = torch.empty(64 << 20, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    w = synth.weight(synth.rng_for(0xC0), synth.Q4_K, 4096, 4096)
    base = torch.from_numpy(w).cuda()
    ws = [D.DeviceWeight(base.clone(), synth.Q4_K, 4096, 4096) for _ in range(64)]
    x = torch.from_numpy(synth.activations(synth.rng_for(0xC0 + 1), 4096)).cuda()
    ys = torch.empty(64, 4096, device="cuda")
    for _ in range(3):
        for i in range(64):
            D.gemv(ws[i], x, ys[i])
    torch.cuda.synchronize()
    print("pmc workload done: 3 x 64 MiB copy, 192 Q4_K 4096x4096 GEMV launches", flush=True)


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


def time_steps(torch, stream, launch, n_rot, steps, warmup):
    """Time exactly `steps` launches cycling through n_rot operand sets;
    returns ms for the whole timed region (HIP events on `stream`)."""
    full = GraphLoop(torch, stream, n_rot, launch)
    rem = steps % n_rot
    part = GraphLoop(torch, stream, rem, launch) if rem else None
    full.replay(max(1, warmup // n_rot))
    torch.cuda.synchronize()
    # The GPU's clock drops while the host sets a workload up (graph capture,
    # uploads) and ramps back over milliseconds of work: keep replaying the
    # same launches until about WARM_S seconds of them have run, so the timed
    # region sees the steady-state clock.
    w0 = time.perf_counter()
    full.replay(1)
    torch.cuda.synchronize()
    per_replay = max(time.perf_counter() - w0, 1e-6)
    full.replay(int(WARM_S / per_replay) + 1)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    full.replay(steps // n_rot)
    if part:
        part.replay(1)
    t1.record(stream)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1)


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
    ncopy = 64
    base = torch.from_numpy(w).cuda()
    ws = [D.DeviceWeight(base.clone(), synth.Q4_K, inner, outer) for _ in range(ncopy)]
    del base
    xd = torch.from_numpy(x).cuda()
    ys = torch.empty(ncopy, outer, device="cuda")

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
        D.gemv(ws[i % ncopy], xd, ys[i % ncopy])

    ms = time_steps(torch, stream, launch, ncopy, steps, warmup)
    us_per = ms * 1e3 / steps
    res = dict(bytes=nbytes, ms=ms, us_per_launch=us_per, gbs=nbytes / (us_per * 1e-6) / 1e9,
               parity_max_err_over_tol=ratio, copies=ncopy)
    res["single_launch_us"] = single_launch_us(torch, stream, launch)
    ms_res = time_steps(torch, stream, lambda i: D.gemv(ws[0], xd, ys[0]), 64, 640, 64)
    res["cache_resident_gbs"] = nbytes / (ms_res * 1e3 / 640 * 1e-6) / 1e9
    return res


def ffn_block(torch, stream, synth, D, steps=600):
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

    steps = steps - steps % ncopy
    ms = time_steps(torch, stream, launch, ncopy, steps, 4 * ncopy)
    us = ms * 1e3 / steps
    # the same block with the post-attention norm folded into gate/up and the
    # residual add into the down projection (x updated in place: the values
    # drift over the steps, the bytes and launches do not)
    nw = torch.from_numpy(rng.uniform(0.5, 1.5, hidden).astype(np.float32)).cuda()
    xs = torch.from_numpy(np.tile(x, (ncopy, 1))).cuda()

    def launch_norm(i):
        k = i % ncopy
        D.ffn_block(*sets[k], nw, 1e-6, xs[k], h=hs[k])

    ms_n = time_steps(torch, stream, launch_norm, ncopy, steps, 4 * ncopy)
    return dict(us=us, bytes=nbytes, gbs=nbytes / (us * 1e-6) / 1e9, copies=ncopy,
                single_launch_us=single_launch_us(torch, stream, launch, 20),
                norm_residual_us=ms_n * 1e3 / steps)


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
    n = 8 * ncopy
    ms = time_steps(torch, stream, lambda i: D.dequantize(ws[i % ncopy], outs[i % ncopy]),
                    ncopy, n, 2 * ncopy)
    deq_us = ms * 1e3 / n
    gcopy = copies_for(gemv_bytes)
    gws = ws + [D.DeviceWeight(base.clone(), synth.Q8_0, inner, outer)
                for _ in range(max(0, gcopy - ncopy))]
    n = 16 * gcopy
    ms = time_steps(torch, stream, lambda i: D.gemv(gws[i % gcopy], xd, ys[i % ncopy]),
                    gcopy, n, 2 * gcopy)
    gemv_us = ms * 1e3 / n
    return dict(dequant_us=deq_us, dequant_gbs=deq_bytes / (deq_us * 1e-6) / 1e9,
                gemv_us=gemv_us, gemv_gbs=gemv_bytes / (gemv_us * 1e-6) / 1e9)


def q8k_gemv(torch, stream, synth, D):
    """The int8-activation variant (the reference C numerics) at 4096x4096
    Q4_K: one step = quantize x to Q8_K + the GEMV, weights rotated through HBM."""
    outer = inner = 4096
    rng = synth.rng_for(0xC0)
    w = synth.weight(rng, synth.Q4_K, outer, inner)
    x = synth.activations(rng, inner)
    nbytes = w.size + 4 * inner + 4 * outer
    ncopy = copies_for(w.size)
    base = torch.from_numpy(w).cuda()
    ws = [D.DeviceWeight(base.clone(), synth.Q4_K, inner, outer) for _ in range(ncopy)]
    xd = torch.from_numpy(x).cuda()
    q8 = torch.empty(inner // 256 * 292, dtype=torch.uint8, device="cuda")
    ys = torch.empty(ncopy, outer, device="cuda")

    def step(i):
        D.quantize_row_q8k(xd, q8)
        D.gemv_q8k(ws[i % ncopy], q8, ys[i % ncopy])
    n = 16 * ncopy
    ms = time_steps(torch, stream, step, ncopy, n, 2 * ncopy)
    us = ms * 1e3 / n
    return dict(us=us, gbs=nbytes / (us * 1e-6) / 1e9)


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

    n = 60
    ms = time_steps(torch, stream, launch, ncopy, n, 4 * ncopy)
    us = ms * 1e3 / n
    tok = aws[0].result()
    return dict(us=us, gbs=nbytes / (us * 1e-6) / 1e9, token=tok)


def prefill(torch, stream, synth, D):
    T, outer, inner = 512, 4096, 4096
    rng = synth.rng_for(0xC4)
    w = synth.weight(rng, synth.Q4_K, outer, inner)
    X = rng.standard_normal((T, inner)).astype(np.float32)
    dw = D.DeviceWeight(torch.from_numpy(w).cuda(), synth.Q4_K, inner, outer)
    Xd = torch.from_numpy(X).cuda()
    Y = torch.empty(T, outer, device="cuda")
    xh = torch.empty(T * inner, dtype=torch.float16, device="cuda")
    n = 50
    ms = time_steps(torch, stream, lambda i: D.prefill_q4_k(dw, Xd, Y, xh), 10, n, 40)
    us = ms * 1e3 / n
    flops = 2.0 * T * outer * inner
    return dict(us=us, tflops=flops / (us * 1e-6) / 1e12,
                mfma_frac=flops / (us * 1e-6) / 1e12 / PEAK_FP16_TFLOPS)


# --------------------------------------------------------------- CPU baseline --

def cpu_baseline(synth, oracle, seconds):
    import ctypes
    outer = inner = 4096
    rng = synth.rng_for(0xC0)
    w = synth.weight(rng, synth.Q4_K, outer, inner)
    x = synth.activations(rng, inner)
    nbytes = w.size + 8 * inner
    ncopy = 16  # 151 MB: larger than the host's last-level cache
    ws = [w.copy() for _ in range(ncopy)]
    env = os.environ.get("OMP_NUM_THREADS")
    # the reference's default when OMP_NUM_THREADS is unset (src/QuantizedKernels.jl:40-41)
    threads = int(env) if env and env.isdigit() else max(2, min(8, (os.cpu_count() or 2) // 2))
    try:
        ctypes.CDLL("libgomp.so.1").omp_set_num_threads(threads)
    except OSError:
        pass
    ref = oracle.ref_lib()
    kind = "reference" if ref is not None else "port"
    out = np.empty(outer, np.float32)
    q8 = np.zeros(inner // 256 * oracle.Q8K_BYTES, np.uint8)
    if ref is not None:
        def call(k):
            ref.q4_k_gemv(ws[k], x, out, q8, inner, outer)
    else:
        def call(k):
            oracle.lib().orc_gemv_q8k(synth.Q4_K, ws[k], x, out, q8, inner, outer)
    for k in range(ncopy):
        call(k)
    n = 0
    t0 = time.perf_counter()
    while True:
        call(n % ncopy)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds and n >= ncopy:
            break
    gbs = nbytes * n / el / 1e9
    what = ("the reference's src/kernels/quant_kernels.c q4_k_gemv compiled from source"
            if kind == "reference" else "the oracle's restatement of quant_kernels.c q4_k_gemv")
    return dict(value=gbs, unit="GB/s", cores=threads, kind=kind,
                sample=(f"{what} (int8-activation path, OpenMP {threads} threads): "
                        f"{n} calls of the 4096x4096 Q4_K GEMV over {ncopy} rotated weight "
                        f"copies in {el:.1f} s, {el / n * 1e3:.3f} ms per call"))


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
    steps, warmup = max(1, args.steps), max(0, args.warmup)

    log(f"Q4_K GEMV 4096x4096: warmup {warmup}, steps {steps}")
    g = q4k_gemv(torch, stream, synth, D, oracle, steps, warmup)
    log(f"  {g['us_per_launch']:.3f} us/launch, {g['gbs']:.1f} GB/s, single {g['single_launch_us']:.2f} us")
    extras = {"q4k_gemv_single_launch_us": g["single_launch_us"],
              "q4k_gemv_cache_resident_gbs": g["cache_resident_gbs"],
              "q4k_gemv_parity_max_err_over_tol": g["parity_max_err_over_tol"],
              "q4k_gemv_weight_copies": g["copies"]}
    if args.only != "gemv":
        log("FFN block 4096/12288")
        f = ffn_block(torch, stream, synth, D)
        log(f"  {f['us']:.2f} us, {f['gbs']:.1f} GB/s")
        log(f"  with the rmsnorm and residual folded in: {f['norm_residual_us']:.2f} us")
        extras.update(ffn_block_us=f["us"], ffn_block_gbs=f["gbs"], ffn_block_frac=f["gbs"] / PEAK_HBM_GBS,
                      ffn_block_single_launch_us=f["single_launch_us"],
                      ffn_block_norm_residual_us=f["norm_residual_us"])
        log("Q8_0 4096x4096 dequant and GEMV")
        q = q8_0_workloads(torch, stream, synth, D)
        log(f"  dequant {q['dequant_us']:.2f} us ({q['dequant_gbs']:.0f} GB/s), gemv {q['gemv_us']:.2f} us ({q['gemv_gbs']:.0f} GB/s)")
        extras.update({f"q8_0_{k}": v for k, v in q.items()})
        log("Q4_K GEMV 4096x4096, int8-activation variant (quantize + GEMV)")
        k8 = q8k_gemv(torch, stream, synth, D)
        log(f"  {k8['us']:.2f} us, {k8['gbs']:.0f} GB/s")
        extras.update(q4k_gemv_q8k_us=k8["us"], q4k_gemv_q8k_gbs=k8["gbs"])
        log("Q6_K lm_head 151936x2048 + argmax")
        lm = lm_head(torch, stream, synth, D)
        log(f"  {lm['us']:.2f} us, {lm['gbs']:.0f} GB/s")
        extras.update(lm_head_argmax_us=lm["us"], lm_head_argmax_gbs=lm["gbs"])
        log("prefill 512x4096x4096")
        p = prefill(torch, stream, synth, D)
        log(f"  {p['us']:.1f} us, {p['tflops']:.1f} TFLOP/s")
        extras.update(prefill_us=p["us"], prefill_tflops=p["tflops"], prefill_mfma_frac=p["mfma_frac"])

    cpu = None
    if not args.no_cpu:
        log(f"CPU baseline (~{args.cpu_seconds:.0f} s)")
        cpu = cpu_baseline(synth, oracle, args.cpu_seconds)
        log(f"  {cpu['value']:.2f} GB/s on {cpu['cores']} threads ({cpu['kind']})")

    ms_per_step = g["ms"] / steps
    line = {
        "metric": METRIC,
        "value": round(g["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "Q4_K dequant-fused GEMV 4096x4096, batch 1, fp32 x; "
                               "64 rotated weight copies (HBM-resident, not cache-resident)",
                   "rows": 4096, "cols": 4096, "weight_bytes": 9437184,
                   "algorithmic_bytes_per_step": g["bytes"]},
        "roofline": {"bound": "hbm", "achieved": round(g["gbs"], 2), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(g["gbs"] / PEAK_HBM_GBS, 4), "traffic": traffic_bytes()},
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
