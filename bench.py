#!/usr/bin/env python3
"""Forward throughput of the MI355X DEQ path at the north-star shape.

Workload (BASELINE.json metric, configs[1] shape at batch 32): d_r=512, h_slots=8,
vocab=50257, d_state=16, B=32 sequences x ctx=256 tokens, fp32, Xavier weights rescaled to
spectral norm 0.5 (seed 0), Zipf(1.1) token ids (seed 1), Picard max 20 / tol 1e-4, no Anderson.

A step is one full forward over the batch with inputs resident in HBM: embedding gather +
W_in signal, the device-resident Picard solve (per-token exit), the selective carrier scan,
the LM head (logits for every position) and the greedy arg-max.  K steps are timed between
two device synchronisations; value = B*T*K / elapsed (tokens/s).

Also reported: the roofline of the dominant kernel (from a profiled forward with HIP events
on the kernel's own stream), per-stage figures, the Picard iteration statistics, and the
same-run CPU baseline (the C oracle, OpenMP over tokens on this host, bounded sample).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "forward tokens/sec at d_r=512,h_slots=8,ctx=256,B=32; HBM GB/s & MFMA % of peak"
PEAK_HBM_GBS = 8000.0
# MI355X published dense MFMA peaks (TFLOP/s).  The split-precision GEMMs execute 3 16-bit
# products per fp32 product, so their algorithmic (fp32-equivalent) ceiling is the 16-bit
# peak / 3; bf16 single-product GEMMs are priced at the full bf16 peak.
GEMM_MODES = {
    "f16x3": dict(flag=0, peak=2500.0 / 3, basis="fp16 dense MFMA 2500 TFLOP/s / 3 products per fp32 multiply"),
    "bf16x3": dict(flag=1 << 7, peak=2500.0 / 3, basis="bf16 dense MFMA 2500 TFLOP/s / 3 products per fp32 multiply"),
    "fp32": dict(flag=1 << 6, peak=157.3, basis="fp32 MFMA 157.3 TFLOP/s"),
    "bf16": dict(flag=1 << 8, peak=2500.0, basis="bf16 dense MFMA 2500 TFLOP/s"),
}
MFMA_STAGES = ("signal_gemm", "qkv_gemm", "wo_gemm", "lmhead_gemm", "readout_gemm")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def host_info(threads: int) -> dict:
    """nproc, the CPU model and the thread count used (one GPU's share of the host is 16 cores on
    these boxes, whatever nproc reports, so the oracle runs at most 16 threads)."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = None
    return dict(nproc=os.cpu_count(), affinity=affinity, cpu_model=model, threads=threads,
                threads_basis="min(nproc, 16): one GPU's share of the box's cores")


def config_metric(name: str, mc, B: int, T: int) -> str:
    """The metric string of a configuration: the headline metric for NS, an own name otherwise."""
    if name == "NS":
        return METRIC
    if name == "C4":
        return (f"C4 long-context carrier stress: forward tokens/sec and carrier-scan HBM GB/s at "
                f"d_r={mc.d},h_slots={mc.H},ctx={T},B={B}")
    return f"{name} forward tokens/sec at d_r={mc.d},h_slots={mc.H},ctx={T},B={B} (not the headline metric)"


def config_data(name: str, mc, tokens: str) -> str:
    ids = "Zipf(1.1) token ids" if tokens == "zipf" else "uniform token ids"
    gates = ("; decay bases 0.999..0.01 across channels, gate logits N(0,1) through the model's projection"
             if name == "C4" else "")
    return f"synthetic (seeded Xavier weights at spectral norm {mc.sigma}, {ids}{gates})"


def cpu_baseline(mc, w, toks, seconds: float):
    """The C oracle (a port of the reference's CPU forward) timed on whole sequences of the same
    workload: one sequence calibrates, then as many sequences as fill about `seconds`."""
    from oracle import pyoracle
    pyoracle.build()
    threads = max(1, min(os.cpu_count() or 1, 16))
    o = pyoracle.Oracle(mc, w).prepared()
    B, T = toks.shape
    t0 = time.perf_counter()
    o.forward(toks[:1].copy(), nthreads=threads)
    t1 = time.perf_counter() - t0
    nseq = int(max(1, min(B, seconds / max(t1, 1e-6))))
    t0 = time.perf_counter()
    o.forward(toks[:nseq].copy(), nthreads=threads)
    t2 = time.perf_counter() - t0
    n = nseq * T
    return dict(value=round(n / t2, 2), unit="tokens/s", cores=threads, kind="port",
                sample=(f"{nseq} of the {B} sequences ({n} tokens) of the same workload, same weights "
                        f"and token ids: solve + LM-head logits + arg-max + carrier scan, "
                        f"{threads} OpenMP threads over tokens, {t2:.1f} s"),
                seconds=round(t2, 2), host=host_info(threads))


def cpu_baseline_memory(mc, w, toks, seconds: float):
    """The C oracle's memory-coupled forward (sequential over positions, OpenMP over sequences)
    timed on a prefix of as many sequences as there are threads: one short calibration run,
    then a prefix length that fills about `seconds`."""
    from oracle import pyoracle
    pyoracle.build()
    threads = max(1, min(os.cpu_count() or 1, 16))
    o = pyoracle.Oracle(mc, w)
    B, T = toks.shape
    nseq = min(B, threads)
    t_cal = min(T, 8)
    t0 = time.perf_counter()
    o.forward_memory(toks[:nseq, :t_cal].copy(), nthreads=threads)
    t1 = time.perf_counter() - t0
    tp = int(max(1, min(T, t_cal * seconds / max(t1, 1e-6))))
    t0 = time.perf_counter()
    o.forward_memory(toks[:nseq, :tp].copy(), nthreads=threads)
    t2 = time.perf_counter() - t0
    n = nseq * tp
    return dict(value=round(n / t2, 2), unit="tokens/s", cores=threads, kind="port",
                sample=(f"the first {tp} of {T} positions of {nseq} of the {B} sequences ({n} tokens) of the "
                        f"same workload, same weights and token ids: memory-coupled solve + carrier + "
                        f"LM-head logits + arg-max, {threads} OpenMP threads over sequences, {t2:.1f} s"),
                seconds=round(t2, 2), host=host_info(threads))


def bench_embed(args, be, mc, w, toks, dev, torch) -> int:
    """embed_context for every position of the NS batch (window = ctx = T): the input pipeline's
    GPU part.  HBM-bound: compulsory bytes are the token ids, one embedding row read and one
    query row written per position."""
    B, T = toks.shape
    ctx = T
    stream = torch.cuda.Stream(dev)
    torch.cuda.set_stream(stream)
    be.set_stream(stream.cuda_stream)
    tok_d = torch.from_numpy(toks).to(dev)
    out = torch.empty((B, T, mc.d), dtype=torch.float32, device=dev)
    for _ in range(args.warmup):
        be.embed_context_async(tok_d, ctx, out)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for _ in range(args.steps):
        be.embed_context_async(tok_d, ctx, out)
    ev1.record(stream)
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / args.steps
    tok_s = B * T / (ms / 1e3)
    byts = B * T * (4 + 8 * mc.d)
    gbs = byts / ms / 1e6
    log(f"embed_context: {ms * 1e3:.1f} us per call, {tok_s:,.0f} positions/s, {gbs:.0f} GB/s algorithmic")
    cpu = None
    if not args.no_cpu:
        from oracle import pyoracle
        pyoracle.build()
        n = max(1, min(B, int(args.cpu_seconds)))
        t0 = time.perf_counter()
        pyoracle.embed_context(w["embed"], toks[:1], ctx)
        t1 = time.perf_counter() - t0
        n = int(max(1, min(B, args.cpu_seconds / max(t1, 1e-6))))
        t0 = time.perf_counter()
        pyoracle.embed_context(w["embed"], toks[:n], ctx)
        t2 = time.perf_counter() - t0
        cpu = dict(value=round(n * T / t2, 1), unit="positions/s", cores=1, kind="port",
                   sample=f"{n} of the {B} sequences ({n * T} positions), one thread, {t2:.1f} s")
    line = {
        "metric": f"embed_context positions/sec at d_r={mc.d},ctx={ctx},B={B}", "value": round(tok_s, 1),
        "unit": "positions/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32 (f64 prefix sums)", "data": "synthetic (closed-form embedding table, Zipf(1.1) token ids)",
        "config": {"workload": f"{args.config}-embed: embed_context of the window ending at every position, "
                               f"B={B} T={T} ctx={ctx} d_r={mc.d} vocab={mc.V}", "mode": "embed",
                   "global_batch": B, "seq_len": T, "parallelism": "none (1 GPU)"},
        "roofline": dict(kernel="k_ctx_chunks + k_ctx_window", bound="hbm", achieved=round(gbs, 1),
                         peak=PEAK_HBM_GBS, unit="GB/s", frac=round(gbs / PEAK_HBM_GBS, 4), traffic=None,
                         basis="token ids + one embedding row read + one query row written per position",
                         bytes_per_call=byts),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def bench_adjoint(args, be, mc, w, toks, dev, torch) -> int:
    """The clean adjoint backward for the NS forward's 8192 tokens: adj_iters Picard steps on the
    adjoint state plus the source gradient.  HBM-bound: the first step reads signal and h* and
    writes pre and v; every further step reads pre and v and writes v (d floats per row each, plus
    the token's dL/dpool row); the source gradient reads pre and v."""
    import numpy as np
    B, T = toks.shape
    n = B * T
    stream = torch.cuda.Stream(dev)
    torch.cuda.set_stream(stream)
    be.set_stream(stream.cuda_stream)
    tok_d = torch.from_numpy(toks).to(dev)
    h = torch.empty((B, T, mc.H, mc.d), dtype=torch.float32, device=dev)
    be.forward_async(tok_d, outputs=dict(h_star=h))
    dl = torch.from_numpy(np.random.default_rng(3).standard_normal((B, T, mc.d)).astype(np.float32)).to(dev)
    v = torch.empty((B, T, mc.H, mc.d), dtype=torch.float32, device=dev)
    src = torch.empty((B, T, mc.d), dtype=torch.float32, device=dev)
    K = args.adj_iters
    for _ in range(args.warmup):
        be.adjoint_async(n, dl, K, mc.beta, v, src)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for _ in range(args.steps):
        be.adjoint_async(n, dl, K, mc.beta, v, src)
    ev1.record(stream)
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / args.steps
    tok_s = n / (ms / 1e3)
    rows = n * mc.H
    # first step: read signal, h*, dl; write pre, v.  each further step: read pre, v, dl; write v.
    # source gradient: read pre, v; write src.  (K = 0: the preparation alone, v_0 written.)
    first = rows * mc.d * 4 + n * mc.d
    byts = 4 * (first + max(K - 1, 0) * (rows * mc.d * 3 + n * mc.d) + rows * mc.d * 2 + n * mc.d)
    gbs = byts / ms / 1e6
    log(f"adjoint ({K} steps): {ms * 1e3:.1f} us per call, {tok_s:,.0f} tokens/s, {gbs:.0f} GB/s algorithmic")
    cpu = None
    if not args.no_cpu:
        from oracle import pyoracle
        pyoracle.build()
        o = pyoracle.Oracle(mc, w)
        hs = h.cpu().numpy().reshape(n, mc.H, mc.d)
        ns = max(1, min(n, 512))
        sig = np.stack([o.signal(w["embed"][t]) for t in toks.reshape(-1)[:ns]])
        dls = dl.cpu().numpy().reshape(n, mc.d)[:ns]
        t0 = time.perf_counter()
        o.adjoint(sig, hs[:ns], dls, K)
        t1 = time.perf_counter() - t0
        cpu = dict(value=round(ns / t1, 1), unit="tokens/s", cores=1, kind="port",
                   sample=f"the first {ns} of the {n} tokens, {K} steps + source gradient, one thread, {t1:.2f} s")
    line = {
        "metric": f"adjoint backward tokens/sec at d_r={mc.d},h_slots={mc.H},B={B},ctx={T}", "value": round(tok_s, 1),
        "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (NS weights and tokens; dL/dpool ~ N(0,1))",
        "config": {"workload": f"{args.config}-adjoint: clean adjoint Picard, {K} steps + source gradient, "
                               f"B={B} T={T} d_r={mc.d} h_slots={mc.H}", "mode": "adjoint",
                   "global_batch": B, "seq_len": T, "parallelism": "none (1 GPU)"},
        "roofline": dict(kernel="k_adj_prep + k_adj_step x iters + k_adj_source", bound="hbm",
                         achieved=round(gbs, 1), peak=PEAK_HBM_GBS, unit="GB/s", frac=round(gbs / PEAK_HBM_GBS, 4),
                         traffic=None, bytes_per_call=byts),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def bench_decode(args, be, mc, w, toks, dev, torch) -> int:
    """Greedy decode (``Trainer::generate`` with greedy sampling, trainer.rs:4219-4431): n_new
    tokens after the B x T prompt, each one position solved with generate's 10 fixed Picard
    steps from embed_context(context, ctx_len), its logits and arg-max.  One position per
    sequence makes every GEMM a weight stream (B rows against the per-slot d x d matrices and
    W_lm), so a step is bound by the weight bytes it reads; the roofline names the stage with
    the most device time in one profiled step and its algorithmic bytes (weights as their hi and
    lo halves, 4 bytes per weight, plus activations)."""
    import dataclasses
    import numpy as np
    from aideen_amd import synth
    B, T = toks.shape
    n_new, ctx_len = args.n_new, T
    smp = None
    if args.sample:
        t_, p_, k_, pen_ = (float(v) for v in args.sample.split(","))
        smp = dict(temperature=t_, top_p=p_, top_k=int(k_), repetition_penalty=pen_)
        # fixed 24-bit draws, as rng.gen::<f32>() makes them
        uni = (np.random.default_rng(7).integers(0, 1 << 24, size=(B, n_new)) * 2.0 ** -24).astype(np.float32)

    def run():
        if smp:
            return be.decode_sample(toks, n_new, ctx_len, uniforms=uni, **smp)
        return be.decode_greedy(toks, n_new, ctx_len)

    stream = torch.cuda.Stream(dev)
    torch.cuda.set_stream(stream)
    be.set_stream(stream.cuda_stream)
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        out = run()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = ev0.elapsed_time(ev1) / args.steps
    tok_s = B * n_new / (ms / 1e3)
    log(f"decode {n_new} tokens x B={B}: {ms:.3f} ms per call on the stream ({wall * 1e3 / args.steps:.3f} ms wall)"
        f" -> {ms * 1e3 / n_new:.1f} us per token, {tok_s:,.0f} tokens/s")

    # one decode step as a device forward: the query row (the prompt's embed_context at its last
    # position), 10 Picard steps without early exit, the arg-max of the position's logits
    q = be.embed_context(toks, ctx_len)[:, -1:, :]
    q_d = torch.from_numpy(np.ascontiguousarray(q)).to(dev)
    am = torch.empty((B, 1), dtype=torch.int32, device=dev)
    be.forward_async(s_in=q_d, outputs=dict(argmax=am), max_iters=10, eps=0.0)
    prof = be.profile_forward(s_in=q_d, outputs=dict(argmax=am), max_iters=10, eps=0.0)
    st = prof["stages"]
    dom = max(st, key=lambda n: st[n]["ms"])
    gbs = st[dom]["bytes"] / st[dom]["ms"] / 1e6
    step_bytes = sum(s["bytes"] for s in st.values())
    stages = {n: dict(ms=round(s["ms"], 4), launches=s["launches"],
                      gbs=round(s["bytes"] / s["ms"] / 1e6, 1) if s["ms"] > 0 else None) for n, s in st.items()}
    log(f"profiled step: {prof['total_ms'] * 1e3:.1f} us; dominant {dom} {st[dom]['ms'] * 1e3:.1f} us "
        f"({st[dom]['launches']} launches, {gbs:.0f} GB/s)")

    cpu = None
    if not args.no_cpu:
        from oracle import pyoracle
        pyoracle.build()
        o = pyoracle.Oracle(dataclasses.replace(mc, max_iters=10, eps=0.0), w)

        def oracle_decode(nn):
            if smp:
                return o.decode_sample(toks, nn, ctx_len, smp["temperature"], smp["top_p"], smp["top_k"],
                                       smp["repetition_penalty"], uni[:, :nn], nthreads=1)
            return o.decode_greedy(toks, nn, ctx_len, nthreads=1), None

        t0 = time.perf_counter()
        ref1, _ = oracle_decode(1)
        t1 = time.perf_counter() - t0
        nn = int(max(1, min(n_new, args.cpu_seconds / max(t1, 1e-6))))
        t0 = time.perf_counter()
        ref, cond = oracle_decode(nn)
        t2 = time.perf_counter() - t0
        same = np.array_equal(ref[:, :1], ref1) and np.array_equal(ref, out[:, :nn])
        if not same and cond is not None:
            # a sampled sequence may part from the oracle's only on a draw within rounding of a boundary
            same = np.array_equal(ref[:, :1], ref1)
            for b in range(B):
                diff = np.flatnonzero(ref[b] != out[b, :nn])
                same = same and (diff.size == 0 or cond[b, diff[0]] < 1.0)
        if not same:
            raise SystemExit("decode: the GPU tokens differ from the C oracle's")
        cpu = dict(value=round(B * nn / t2, 2), unit="tokens/s", cores=1, kind="port",
                   sample=(f"the first {nn} of the {n_new} decoded tokens of the same prompt and weights "
                           f"(one sequence: the oracle's decode runs sequences in parallel, so one thread), "
                           f"{t2:.1f} s; tokens identical to the GPU's"),
                   seconds=round(t2, 2), host=host_info(1))
    kind = "greedy" if not smp else "sampled (T={temperature}, top_p={top_p}, top_k={top_k}, penalty={repetition_penalty})".format(**smp)
    line = {
        "metric": f"{'greedy' if not smp else 'sampled'} decode tokens/sec at d_r={mc.d},h_slots={mc.H},vocab={mc.V},B={B},prompt={T}",
        "value": round(tok_s, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": config_data(args.config, mc, synth.PRESETS[args.config]["tokens"]),
        "config": {"workload": (f"{args.config}-decode: {n_new} {kind} tokens after a {B}x{T} prompt, ctx_len "
                                f"{ctx_len}, 10 Picard steps per token (no early exit), d_r={mc.d} "
                                f"h_slots={mc.H} vocab={mc.V}; one step = one call of {n_new} tokens"),
                   "mode": "decode", "global_batch": B, "seq_len": T, "n_new": n_new,
                   "parallelism": "none (1 GPU)"},
        "roofline": dict(kernel=dom, bound="hbm", achieved=round(gbs, 1), peak=PEAK_HBM_GBS, unit="GB/s",
                         frac=round(gbs / PEAK_HBM_GBS, 4), traffic=None,
                         basis="algorithmic bytes of one profiled decode step: weights read once per launch "
                               "(hi + lo halves) + activation rows; weights may be served from the MALL",
                         launches=st[dom]["launches"], avg_launch_ms=round(st[dom]["ms"] / st[dom]["launches"], 5),
                         bytes_per_launch=st[dom]["bytes"] / st[dom]["launches"]),
        "cpu_baseline": cpu,
        "step_profile": {"total_ms": round(prof["total_ms"], 4), "bytes": step_bytes,
                         "gbs": round(step_bytes / prof["total_ms"] / 1e6, 1), "stages": stages},
    }
    print(json.dumps(line), flush=True)
    return 0


SIMDS, CLOCK_GHZ = 1024, 2.4  # MI355X: 256 CUs x 4 SIMDs; the peak-rate clock


def scan_compute_bound(mc, B, T, ms):
    """The carrier scan's compute floor beside its HBM fraction.  Which form runs follows the
    library's rule (the matrix form where the per-step form would need time chunks: fewer than 512
    workgroups of 256 channels, and a decay that keeps 16-step products normal).  Per-step form
    (k_scan_fused): one thread per (sequence, slot, channel), 290 SIMD cycles per wave and step
    counted in the compiled 16-state instance (31 state and output FMAs and 25 other VALU
    instructions at 4 cycles, 4.3 transcendental ones at 16), i.e. about 8 n + 165 for an n-state
    instance (n = 1, 8, 16, 32; the others extrapolated), so floor = waves x T x cycles / SIMDs.
    Matrix form (k_scan_ssd): per 16 channels and 16 steps 24 v_mfma_f32_16x16x4f32 of 32 cycles
    (16 states; 36 with 32), so floor = waves x T/16 x MFMA cycles / SIMDs.  At the 2.4 GHz peak
    clock; frac = floor / measured."""
    nch, wgs = 1, B * mc.H * ((mc.d + 255) // 256)
    while wgs * nch < 512 and T // (nch * 2) >= 64:
        nch *= 2
    ssd = nch > 1 and mc.N <= 32 and mc.r <= 64 and mc.d % 16 == 0
    if ssd:
        waves = B * mc.H * (mc.d // 16)
        per = (24 if mc.N <= 16 else 36) * 32
        cyc = waves * ((T + 15) // 16) * per / SIMDS
        kind, basis = "mfma", "fp32 MFMA cycles of the chunked matrix form (v_mfma_f32_16x16x4f32, 32 cycles each)"
    else:
        waves = B * mc.H * ((mc.d + 63) // 64)
        n_inst = 16 if mc.N == 16 else 1 if mc.N == 1 else 32 if mc.N > 8 else 8
        per = 290 if n_inst == 16 else 8 * n_inst + 165
        cyc = waves * T * per / SIMDS
        kind, basis = "valu", (f"VALU issue cycles of the per-step form ({per} per wave and step: counted in the compiled "
                               f"16-state instance" + ("" if n_inst == 16 else ", extrapolated to this state count") + ")")
    floor_ms = cyc / (CLOCK_GHZ * 1e6)
    return dict(form="matrix" if ssd else "per-step", bound=kind, floor_ms=round(floor_ms, 4),
                frac=round(floor_ms / ms, 4), basis=basis + "; floor at 2.4 GHz over 1024 SIMDs")


def stream_calib(dev, mib: int, reps: int = 20) -> dict:
    """o = a + b * c over four arrays of `mib` MiB each (three reads and one write per element, as
    in the attention and update kernels), timed with events over `reps` launches after warm-up."""
    import torch
    n = mib << 18
    a, b, c = (torch.full((n,), 1.0 + q, dtype=torch.float32, device=dev) for q in range(3))
    o = torch.empty_like(a)
    for _ in range(3):
        torch.addcmul(a, b, c, out=o)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        torch.addcmul(a, b, c, out=o)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    gbs = 4.0 * n * 4 / (us * 1e-6) / 1e9
    del a, b, c, o
    return dict(pattern="3 reads + 1 write (torch.addcmul)", mib_per_array=mib, us=round(us, 1),
                gbs=round(gbs, 1), frac=round(gbs / PEAK_HBM_GBS, 4))


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="NS")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="also run one plain device copy of this size (calibrates HBM byte counters)")
    ap.add_argument("--stream-mib", type=int, default=0,
                    help="also time a three-read-one-write pass (torch.addcmul) over four arrays of this "
                         "size: the practical HBM rate of the attention's and update's access pattern "
                         "(reported as stream_calib; 128 MiB arrays exceed the memory-side cache together)")
    ap.add_argument("--mode", choices=["forward", "memory", "embed", "adjoint", "decode"], default="forward",
                    help="forward: the canonical (token-parallel) forward, the headline metric; memory: "
                         "the memory-coupled forward (positions in order, history context and carrier "
                         "state between them) on the same shape with a one-dimensional carrier state; "
                         "embed: embed_context queries for every position (window = ctx); adjoint: the "
                         "clean adjoint Picard backward of the NS forward; decode: greedy decode of "
                         "--n-new tokens after the configuration's B x T prompt (C2 is its shape)")
    ap.add_argument("--n-new", type=int, default=64, help="decode: tokens generated per call")
    ap.add_argument("--sample", default="",
                    help="decode: LmHead::sample instead of greedy, as 'temperature,top_p,top_k,penalty' "
                         "(the reference binaries use 0.8,0.9,40,1.1), with fixed seeded draws")
    ap.add_argument("--adj-iters", type=int, default=2,
                    help="adjoint steps (ArchitectureConfig::adj_iters defaults to 2)")
    ap.add_argument("--eps", type=float, default=None, help="override the Picard tolerance")
    ap.add_argument("--gemm", choices=list(GEMM_MODES), default="f16x3",
                    help="GEMM arithmetic (f16x3 / bf16x3 / fp32 are fp32-accurate; bf16 is the "
                         "reduced-precision bf16-input variant)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(one MI355X per box); run with --gpus 1", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from aideen_amd import synth
    from aideen_amd.backend import GpuDeqBackend

    import dataclasses
    p = synth.PRESETS[args.config]
    gm = GEMM_MODES[args.gemm]
    mc = dataclasses.replace(p["model"], flags=p["model"].flags | gm["flag"])
    memory = args.mode == "memory"
    if memory:  # the fixed-history mode's carrier: one state per (slot, dim), constant decay
        mc = dataclasses.replace(mc, N=1, flags=(mc.flags & ~synth.F_SCAN_SELECTIVE) | synth.F_MEMORY)
    if args.eps is not None:
        mc = dataclasses.replace(mc, eps=args.eps)
    B, T = p["B"], p["T"]
    log(f"config {args.config} ({args.mode}): d={mc.d} H={mc.H} V={mc.V} N={mc.N} B={B} T={T} eps={mc.eps}")
    w = synth.preset_weights(args.config, mc, seed=0)
    if memory:
        w = dict(w)
        w.update(synth.make_hist_weights(mc, seed=0))
    toks = synth.make_tokens(p["tokens"], B, T, mc.V, seed=1)

    dev = torch.device("cuda:0")
    be = GpuDeqBackend(mc, B, T)
    be.upload_weights(w)
    if args.mode == "embed":
        return bench_embed(args, be, mc, w, toks, dev, torch)
    if args.mode == "adjoint":
        return bench_adjoint(args, be, mc, w, toks, dev, torch)
    if args.mode == "decode":
        return bench_decode(args, be, mc, w, toks, dev, torch)
    # a dedicated (default-priority) stream: the library's kernels and the timing events share it
    stream = torch.cuda.Stream(dev)
    torch.cuda.set_stream(stream)
    be.set_stream(stream.cuda_stream)
    assert stream.cuda_stream != 0
    tok_d = torch.from_numpy(toks).to(dev)
    outs = dict(
        h_star=torch.empty((B, T, mc.H, mc.d), dtype=torch.float32, device=dev),
        iters=torch.empty((B, T), dtype=torch.int32, device=dev),
        logits=torch.empty((B, T, mc.V), dtype=torch.float32, device=dev),
        argmax=torch.empty((B, T), dtype=torch.int32, device=dev),
        scan_y=torch.empty((B, T, mc.H, mc.d), dtype=torch.float32, device=dev),
        scan_state=torch.empty((B, mc.H, mc.d, mc.N), dtype=torch.float32, device=dev),
    )

    if args.copy_mib:
        src = torch.ones(args.copy_mib << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    for _ in range(args.warmup):
        be.forward_async(tok_d, outputs=outs)
    torch.cuda.synchronize()
    be.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        be.forward_async(tok_d, outputs=outs)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    be.synchronize()
    gpu_ms = ev0.elapsed_time(ev1)
    ms_per_step = gpu_ms / args.steps
    tok_s = B * T * args.steps / (gpu_ms / 1e3)
    log(f"{args.steps} steps: {gpu_ms:.2f} ms on the stream ({wall * 1e3:.2f} ms wall) "
        f"-> {ms_per_step:.3f} ms/step, {tok_s:,.0f} tokens/s")

    iters = outs["iters"].cpu().numpy()
    prof = be.profile_forward(tok_d, outputs=outs)
    stages = {}
    for name, s in prof["stages"].items():
        e = dict(ms=round(s["ms"], 4), launches=s["launches"])
        if s["ms"] > 0:
            if s["flops"] > 0:
                e["tflops"] = round(s["flops"] / s["ms"] / 1e9, 2)
            if s["bytes"] > 0:
                e["gbs"] = round(s["bytes"] / s["ms"] / 1e6, 1)
        stages[name] = e
    dom = max((n for n in prof["stages"] if n in MFMA_STAGES), key=lambda n: prof["stages"][n]["ms"])
    ds = prof["stages"][dom]
    traffic = None
    tf_path = os.path.join(ROOT, "profiles", f"{dom}_{args.config}{'_memory' if memory else ''}_{args.gemm}_traffic.json")
    if os.path.exists(tf_path):
        traffic = json.load(open(tf_path)).get("bytes_per_launch")
    tflops = ds["flops"] / ds["ms"] / 1e9
    if memory:
        # one position of every sequence per launch (B rows): 2*B flops per 4-byte weight, far
        # below the f16x3 ridge (peak / HBM bandwidth), so the weight stream bounds the kernel
        gbs = ds["bytes"] / ds["ms"] / 1e6
        roofline = dict(kernel=dom, bound="hbm", achieved=round(gbs, 1), peak=PEAK_HBM_GBS, unit="GB/s",
                        frac=round(gbs / PEAK_HBM_GBS, 4), traffic=traffic,
                        basis="algorithmic bytes: fp32-equivalent weights (hi + lo halves) + A rows + C rows",
                        gemm=args.gemm, launches=ds["launches"], avg_launch_ms=round(ds["ms"] / ds["launches"], 4),
                        bytes_per_launch=ds["bytes"] / ds["launches"],
                        mfma_tflops=round(tflops, 2), mfma_frac=round(tflops / gm["peak"], 4))
    else:
        roofline = dict(kernel=dom, bound="mfma", achieved=round(tflops, 2), peak=round(gm["peak"], 1),
                        unit="TFLOP/s", frac=round(tflops / gm["peak"], 4), traffic=traffic,
                        peak_basis=gm["basis"], gemm=args.gemm,
                        launches=ds["launches"], avg_launch_ms=round(ds["ms"] / ds["launches"], 4),
                        flops_per_launch=ds["flops"] / ds["launches"])
    hbm = {}
    for n in ("attn", "update", "scan", "argmax", "pool", "hist_ctx", "temporal"):
        if n in prof["stages"] and prof["stages"][n]["ms"] > 0:
            s = prof["stages"][n]
            g = s["bytes"] / s["ms"] / 1e6
            hbm[n] = dict(gbs=round(g, 1), frac=round(g / PEAK_HBM_GBS, 4))
    if "scan" in hbm and not memory:
        hbm["scan"]["compute_bound"] = scan_compute_bound(mc, B, T, prof["stages"]["scan"]["ms"])

    cpu = None
    if not args.no_cpu:
        log("cpu baseline ...")
        cpu = (cpu_baseline_memory if memory else cpu_baseline)(mc, w, toks, args.cpu_seconds)
        log(f"cpu baseline {cpu['value']} tokens/s on {cpu['cores']} threads")

    line = {
        "metric": (config_metric(args.config, mc, B, T) if not memory else
                   f"memory-coupled forward tokens/sec at d_r={mc.d},h_slots={mc.H},ctx={T},B={B}"),
        "value": round(tok_s, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32" if args.gemm != "bf16" else "bf16-in/f32-acc",
        "data": config_data(args.config, mc, p["tokens"]),
        "config": {"workload": (f"{args.config}: DEQ forward d_r={mc.d} h_slots={mc.H} vocab={mc.V} "
                                f"d_state={mc.N} B={B} ctx={T}, Picard max {mc.max_iters} tol {mc.eps}, "
                                f"anderson m={mc.anderson_m}; logits for all positions + arg-max + scan; "
                                f"GEMM {args.gemm}") if not memory else
                               (f"{args.config}-memory: memory-coupled DEQ forward d_r={mc.d} h_slots={mc.H} "
                                f"vocab={mc.V} B={B} ctx={T} (positions in order, B tokens per solve), "
                                f"history context + carrier state d_state=1, Picard max {mc.max_iters} tol "
                                f"{mc.eps}; logits for all positions + arg-max; GEMM {args.gemm}"),
                   "mode": args.mode,
                   "global_batch": B, "seq_len": T, "parallelism": "none (1 GPU)"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "picard": {"mean_iters": round(float(iters.mean()), 3), "max_iters": int(iters.max()),
                   "hist": np.bincount(iters.ravel(), minlength=mc.max_iters + 1).tolist(),
                   "active_per_iter": prof["active"]},
        "hbm_kernels": hbm,
        "stages": stages,
        "profiled_forward_ms": round(prof["total_ms"], 3),
    }
    if args.stream_mib:
        line["stream_calib"] = stream_calib(dev, args.stream_mib)
    if args.config == "C4" and "scan" in hbm:  # the configuration's own figure: the carrier scan
        sc = prof["stages"]["scan"]
        line["scan"] = dict(gbs=hbm["scan"]["gbs"], frac=hbm["scan"]["frac"], ms=round(sc["ms"], 4),
                            bytes=sc["bytes"], basis="compulsory bytes: read h* and the carrier record, write y",
                            compute_bound=hbm["scan"]["compute_bound"])
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
