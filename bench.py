"""Benchmark of the quantized MoE hot path on one MI355X: Q4_K MoE-layer us/token + HBM GB/s (decode), TFLOPS at a 2k-token prefill.

Headline (value): config 1, Q4_K decode at batch 1 through 48 stacked MoE layers (hidden 2048, 512 experts x FF 512,
top-10 + shared; each layer's weights seeded independently, 0.908 GB a layer resident in HBM), one token per step.
The layers are chained as an engine chains them: x_{l+1} = x_l + MoE_l(rmsnorm(x_l)).  A step is one HIP-graph replay
of sfnx_moe_decode over the 48 layers (three launches a layer).  value = achieved algorithmic HBM GB/s: per
token-layer the router's fp32 rows plus the 11 experts' Q4_K bytes (23,666,688 B), over the measured step time.

Also in the JSON line: us/token-layer; each decode kernel's time from HIP events on the launch stream (eager, one
layer at a time) and the dominant one's roofline; the prompt path (config 3: 2048 tokens, Zipf-skewed routing); the
CPU baseline (the oracle on config 0, on the host's cores) with the GPU's parity against it for that token.

Configs 2 (a 96-row verify window through the whole layer) and 4 (Q8_0 experts: decode through 24 stacked layers and
a 4096-token prompt chunk) are reported beside it, and the other expert types the reference decodes (Q5_K, Q4_0,
Q5_1: decode through 12 stacked layers, a 2048-token prompt chunk).

python bench.py [--gpus 1] [--steps K] [--warmup W] [--layers 48] [--no-prefill] [--no-window] [--no-cpu] [--no-extra]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
F16_MFMA_PEAK_TFLOPS = 2500.0
INT8_MFMA_PEAK_TOPS = 5000.0
ZIPF_S, ZIPF_ALPHA, ZIPF_SEED = 1.1, 0.125, 7   # config 3: logits[:, e] += ALPHA * -S ln(rank_e), max rows/expert ~200


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-window", action="store_true", help="skip the 16-row decode window")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-extra", action="store_true", help="skip configs 2 and 4 (verify window, Q8_0)")
    ap.add_argument("--q8-layers", type=int, default=24)
    ap.add_argument("--type-layers", type=int, default=12, help="stacked layers for the Q5_K / Q4_0 / Q5_1 decode lines")
    ap.add_argument("--trace-summary", metavar="CSV",
                    help="only summarise a rocprofv3 kernel trace (run_kernel_trace.csv) of the decode-only bench "
                         "(--no-prefill --no-window --no-extra): each decode kernel's average duration over the timed "
                         "graph replays and over the clocked eager passes, in the lines bench.py reads back from profiles/")
    ap.add_argument("--copy-calib", action="store_true",
                    help="only copy 1 GiB device-to-device 3 times: the known-size kernel that scales rocprofv3's "
                         "FETCH_SIZE / WRITE_SIZE to bytes")
    return ap.parse_args()


def expert_bytes(s, moe):
    return 2 * s.ff * moe.row_bytes(s.wtype, s.H) + s.H * moe.row_bytes(s.dn_type, s.ff)


def shared_bytes(s, moe):
    """the shared expert's weight bytes: dense Q8_0 matrices (sh_q8s), else one more expert of the routed types"""
    if s.sh_q8s:
        return 2 * s.ff * moe.row_bytes(moe.Q8_0, s.H) + s.H * moe.row_bytes(moe.Q8_0, s.ff)
    return expert_bytes(s, moe)


def main():
    args = parse()
    if args.trace_summary:
        return trace_summary(args.trace_summary, args.layers)
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: every GPU box here has one, and no multi-GPU path is "
                                   "built (the path would shard by experts or by FF slices; this bench measures one GPU's share)", "n_gpus": args.gpus}))
        return 2
    import torch

    if args.copy_calib:
        a = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calib_bytes_per_copy": a.numel() * 4}), flush=True)
        return 0
    from sfnx_amd import moe

    torch.cuda.set_device(0)
    dev = "cuda"
    s = moe.LayerShape(H=2048, E=512, K=10, ff=512, wtype=moe.Q4_K, shared=True)
    NL = args.layers
    t0 = time.time()
    layers = [moe.MoeLayer.synthetic(s, seed=1000 + l) for l in range(NL)]
    torch.cuda.synchronize()
    log(f"generated {NL} layers in {time.time() - t0:.1f}s")

    # ------------------------------------------------------------------ decode, config 1
    T = 1
    x0 = torch.empty((T, s.H), dtype=torch.float32, device=dev)
    moe.synth_normal(x0, 4242, 1.0)
    x = x0.clone()
    f = moe.FusedDecode(layers, T)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        f(x)   # warm: loads every kernel's code object
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        x.copy_(x0)
        f(x)
    for _ in range(args.warmup):
        g.replay()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(args.steps):
        g.replay()
    ev1.record()
    torch.cuda.synchronize()
    ms_step = ev0.elapsed_time(ev1) / args.steps
    nj = int(f.piece("njobs", torch.int32, (2,))[0])
    assert nj == s.K + 1, nj   # 10 distinct routed experts + the shared one in the last layer
    assert torch.isfinite(x).all()
    eb = expert_bytes(s, moe)
    bytes_tl = (s.E + 1) * s.H * 4 + (s.K + 1) * eb
    us_tl = ms_step * 1000 / NL
    gbs = bytes_tl * NL / (ms_step * 1e-3) / 1e9
    log(f"decode: {ms_step:.3f} ms/step, {us_tl:.2f} us/token-layer, {gbs:.0f} GB/s")

    # ------------------------------------------------------------------ each kernel's own duration
    # The library's kernel clock launches each decode kernel with a start/stop event pair on the launch stream that
    # the runtime stamps at that dispatch's begin and end (hipExtLaunchKernel), so a duration excludes launch gaps
    # and agrees with rocprofv3's kernel trace.  One eager pass over the 48 layers, 3 repetitions.
    names = ["k_dec_router", "k_dec_experts", "k_dec_down"]
    alg = [(s.E + 1) * s.H * 4, (s.K + 1) * 2 * s.ff * moe.row_bytes(s.wtype, s.H),
           (s.K + 1) * s.H * moe.row_bytes(s.dn_type, s.ff)]
    reps = 3
    tot = [0.0, 0.0, 0.0]
    moe.kernel_clock(True)
    try:
        for _ in range(reps):
            x.copy_(x0)
            for l in range(NL):
                f(x, layer0=l, n_layers=1)
                for i, v in enumerate(moe.kernel_clock_read()):
                    tot[i] += v
    finally:
        moe.kernel_clock(False)
    avg_us = {names[i]: tot[i] / (reps * NL) for i in range(3)}
    dom = max(range(3), key=lambda i: tot[i])
    ach = alg[dom] / (avg_us[names[dom]] * 1e-6) / 1e9
    traffic = measured_traffic(names[dom])
    log("per-kernel avg us (dispatch-stamped events): " + ", ".join(f"{n} {v:.2f}" for n, v in avg_us.items()))

    out = {
        "metric": "Q4_K MoE-layer µs/token + HBM GB/s (decode); TFLOPS at 2k-token prefill",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k x q8_1 (int8 dot4), fp32 accumulate",
        "data": "synthetic: seeded Irwin-Hall(12) normals, weights N(0,0.02) quantized by the library's Q4_K quantizer",
        "config": {"workload": "config 1: Q4_K decode, batch 1, 48 stacked MoE layers", "hidden": s.H, "experts": s.E,
                   "ff": s.ff, "topk": s.K, "shared_expert": True, "layers": NL, "tokens_per_step": T,
                   "parallelism": "none (1 GPU, every expert resident in HBM)"},
        "us_per_token_layer": round(us_tl, 3),
        "us_per_token": round(ms_step * 1000, 2),
        "bytes_per_token_layer": bytes_tl,
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "kernel_avg_us": {n: round(v, 3) for n, v in avg_us.items()},
        "roofline": {"kernel": names[dom], "bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "algorithmic_bytes_per_launch": alg[dom]},
    }
    # The same kernel's average from the committed rocprofv3 trace of the decode-only bench, taken on this build (its
    # sources' hash recorded with it): over the timed graph replays, the regime the step time measures, and over the
    # clocked eager passes.  When it describes this build, roofline.frac and achieved are the graph average's, the
    # event clock's figure beside them; otherwise the event clock's, and the profile is reported as stale.
    src = source_hash()
    out["build_source"] = src
    rp = rocprof_avg(names[dom])
    if rp is not None:
        eager_us, graph_us, prof_src = rp
        fresh = prof_src == src
        out["roofline"]["rocprof"] = {"source": "profiles/kernel_stats_decode48_q4k.md", "profile_build": prof_src,
                                      "matches_build": fresh, "eager_avg_us": eager_us, "graph_avg_us": graph_us,
                                      "frac_eager": round(alg[dom] / (eager_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                                      "frac_graph": round(alg[dom] / (graph_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        out["roofline"]["frac_event"] = round(ach / HBM_PEAK_GBS, 4)
        out["roofline"]["achieved_event"] = round(ach, 1)
        if fresh:
            ach = alg[dom] / (graph_us * 1e-6) / 1e9
            out["roofline"]["achieved"] = round(ach, 1)
            out["roofline"]["frac"] = round(ach / HBM_PEAK_GBS, 4)
            out["roofline"]["timing"] = "rocprofv3 graph-replay average of this build (profiles/)"
        else:
            out["roofline"]["timing"] = "dispatch-stamped events (eager); the committed profile is of another build"
    tr_src = traffic_source()
    if traffic is not None and tr_src != src:
        out["roofline"]["traffic_stale"] = {"bytes": traffic, "profile_build": tr_src}
        out["roofline"]["traffic"] = None
    cb = copy_bandwidth(torch)
    out["hbm_copy_gbs"] = cb
    out["hbm_frac_of_copy"] = round(gbs / cb, 4)
    out["roofline"]["frac_of_copy"] = round(ach / cb, 4)
    if not args.no_window:
        out["decode_window16"] = bench_window16(layers, s, moe, torch, args.steps)
    if not args.no_prefill:
        out["prefill"] = bench_prefill(layers[0], s, moe, torch)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(layers[0], s, moe, torch, x0, args.cpu_seconds)
    if not args.no_extra:
        out["verify_window"] = bench_window(layers[0], s, moe, torch)
        out["q8_0"] = bench_q8_0(moe, torch, args.q8_layers, args.steps, args.warmup)
        out["other_types"] = bench_other_types(moe, torch, args.type_layers, args.steps, args.warmup)
        out["q8s_shared"] = bench_q8s_shared(moe, torch, args.type_layers, args.steps, args.warmup)
        out["hc_read"] = bench_hc_read(moe, torch)
        log(f"q8s shared: decode {out['q8s_shared']['decode_us_per_token_layer']} us/token-layer")
    print(json.dumps(out), flush=True)
    return 0


def copy_bandwidth(torch, nbytes=1 << 30, reps=10):
    """the HBM bandwidth a plain device copy achieves on this GPU (torch's copy kernel, 1 GiB to 1 GiB): bytes read
    plus bytes written over the time, the best of reps copies"""
    a = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        b.copy_(a)
        e1.record()
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) * 1e-3)
    del a, b
    torch.cuda.empty_cache()
    return round(2 * nbytes / best / 1e9, 1)


DECODE_KERNELS = {"k_dec_router": "k_dec_router", "k_dec_experts1": "k_dec_experts", "k_dec_down1": "k_dec_down"}
CLOCK_REPS = 3   # the eager passes bench.py clocks each decode kernel over, after the timed graph replays


def source_hash():
    """a short hash of the library's sources (sfnx_amd/csrc, the headers): names the build a committed profile was
    taken on, so the bench can tell whether it describes the build it runs"""
    import hashlib
    h = hashlib.sha256()
    files = sorted(list((ROOT / "sfnx_amd" / "csrc").glob("*")) + list((ROOT / "include").glob("*.h")))
    for f in files:
        if f.is_file():
            h.update(f.name.encode())
            h.update(f.read_bytes())
    return h.hexdigest()[:12]


def trace_summary(path, NL):
    """rocprofv3's per-dispatch kernel trace of the decode-only bench, split by regime: the clocked eager passes are each
    decode kernel's last CLOCK_REPS x NL dispatches (they run after the timed loop), the rest are graph replays (plus
    the warm pass).  Prints `rocprof <kernel> eager_avg_us E graph_avg_us G n_eager NE n_graph NG` lines, the build's
    source hash, and, over the graph replays, the period of the router's dispatches (one a layer: the traced time a
    layer takes) and how far each dispatch's start stamp precedes the previous decode dispatch's end stamp."""
    import csv
    durs, seq = {}, []
    with open(path) as f:
        for r in csv.DictReader(f):
            name = DECODE_KERNELS.get(r["Kernel_Name"].split("(")[0])
            if name:
                se = (int(r["Start_Timestamp"]), int(r["End_Timestamp"]))
                durs.setdefault(name, []).append(se)
                seq.append((se[0], se[1], name))
    ne = CLOCK_REPS * NL
    print(f"rocprof-source {source_hash()}")
    for name, v in sorted(durs.items()):
        v.sort()
        d = [(e - s) / 1e3 for s, e in v]
        eager, graph = d[-ne:], d[:-ne]
        print(f"rocprof {name} eager_avg_us {sum(eager) / len(eager):.3f} graph_avg_us {sum(graph) / max(1, len(graph)):.3f} "
              f"n_eager {len(eager)} n_graph {len(graph)}")
    seq.sort()
    g = seq[: len(seq) - 3 * ne]   # the graph replays and the warm pass, in dispatch order
    starts = [s for s, e, n in g if n == "k_dec_router"]
    per = [(b - a) / 1e3 for a, b in zip(starts, starts[1:]) if (b - a) < 100e3]   # within a replay (no host gap)
    ov = [(e0 - s1) / 1e3 for (s0, e0, _), (s1, e1, _) in zip(g, g[1:]) if s1 - e0 < 100e3]
    if per and ov:
        print(f"rocprof-graph layer_period_us {sum(per) / len(per):.3f} start_before_prev_end_us {sum(ov) / len(ov):.3f} "
              f"n {len(per)}")
    return 0


def rocprof_avg(kernel):
    """the committed rocprofv3 averages of a decode kernel (profiles/kernel_stats_decode48_q4k.md, lines written by
    bench.py --trace-summary): (eager_avg_us, graph_avg_us, source hash of the profiled build) or None"""
    p = ROOT / "profiles" / "kernel_stats_decode48_q4k.md"
    if not p.exists():
        return None
    src, got = None, None
    for line in p.read_text().splitlines():
        f = line.split()
        if len(f) == 2 and f[0] == "rocprof-source":
            src = f[1]
        if len(f) >= 6 and f[0] == "rocprof" and f[1] == kernel:
            got = float(f[3]), float(f[5])
    return None if got is None else (got[0], got[1], src)


def traffic_source():
    """the source hash of the build profiles/traffic.txt was measured on (its `source <hash>` line), or None"""
    p = ROOT / "profiles" / "traffic.txt"
    if not p.exists():
        return None
    for line in p.read_text().splitlines():
        f = line.split()
        if len(f) == 2 and f[0] == "source":
            return f[1]
    return None


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` on this workload, from the rocprofv3 FETCH_SIZE / WRITE_SIZE passes recorded
    in profiles/traffic.txt (each counter scaled by what it reads for a copy of known size), or None"""
    p = ROOT / "profiles" / "traffic.txt"
    if not p.exists():
        return None
    for line in p.read_text().splitlines():
        f = line.split()
        if len(f) == 4 and f[0] == "traffic" and f[1] == kernel:
            return int(float(f[2]) + float(f[3]))
    return None


def zipf_bias(E):
    import numpy as np
    rank = np.random.default_rng(ZIPF_SEED).permutation(E) + 1
    return (ZIPF_ALPHA * -ZIPF_S * np.log(rank)).astype(np.float32)


def bench_prefill(L, s, moe, torch, C=2048, reps=20):
    """config 3: 2048 tokens through layer 0, a seeded Zipf(1.1) bias on the routed logits; the routed + shared experts
    on the matrix cores (f16 MFMA, the reference's default prompt arithmetic) and on the int8 dot kernels (q8_1)"""
    dev = "cuda"
    x = torch.empty((C, s.H), dtype=torch.float32, device=dev)
    moe.synth_normal(x, 777, 1.0)
    xn = torch.empty_like(x)
    moe.residual_rmsnorm(x, None, xn)
    y = torch.empty_like(x)
    b = moe.PrefillBuffers(s, C)
    bias = torch.from_numpy(zipf_bias(s.E)).to(dev)
    moe.prefill_route(L, xn, b, bias)
    moe.quantize_q8_1(xn, b.xq)
    moe.to_f16(xn, b.xh)
    torch.cuda.synchronize()
    cnt = b.cnt.cpu()
    calls = {
        "mma_gate_up": lambda: moe.moe_gate_up_mma(L.gu_w, L.gu_stride, s.wtype, s.H, 2 * s.ff, b.jobs_gu, b.njobs, b.cap,
                                                   b.xh, b.gu),
        "swiglu_h16": lambda: moe.swiglu_h16(b.gu, b.h16, s.ff),
        "mma_gate_up_swiglu": lambda: moe.moe_gate_up_swiglu_mma(L.gu_w, L.gu_stride, s.wtype, s.H, s.ff, b.jobs_gu,
                                                                b.njobs, b.cap, b.xh, b.h16),
        "mma_down": lambda: moe.moe_down_mma(L.dn_w, L.dn_stride, s.dn_type, s.ff, s.H, b.jobs_dn, b.njobs, b.cap, b.h16,
                                             b.part),
        "q8_gate_up": lambda: moe.moe_gate_up_big(L.gu_w, L.gu_stride, s.wtype, s.H, 2 * s.ff, b.jobs_gu, b.njobs, b.cap,
                                                  b.xq, b.gu),
        "q8_down": lambda: moe.moe_down_big(L.dn_w, L.dn_stride, s.dn_type, s.ff, s.H, b.jobs_dn, b.njobs, b.cap, b.gu, b.part),
    }
    us = {}
    for name, c in calls.items():
        us[name] = median_us(torch, c, reps)
    # the whole layer as the prompt path runs it: router logits, the skew's bias, top-k and the job permutation, f16
    # activations, gate|up + SwiGLU, down, the combine
    us["layer"] = median_us(torch, lambda: moe.prefill_layer_mma(L, xn, y, b, bias), reps)
    # the same calls as the mean of a back-to-back series (the previous timing method; the clock management moves a
    # series more than single calls), beside the medians so the two methods can be compared
    mean = {n: round(time_us(torch, calls[n], reps), 1) for n in ("mma_gate_up_swiglu", "mma_down")}
    mean["layer"] = round(time_us(torch, lambda: moe.prefill_layer_mma(L, xn, y, b, bias), reps), 1)
    P = C * s.K
    flops = 2 * (P + C) * (2 * s.ff * s.H + s.H * s.ff)   # 2 per multiply-add, routed + shared pairs
    touched = int((cnt > 0).sum()) + 1
    wbytes = touched * expert_bytes(s, moe)
    # the prompt path as the layer runs it: gate|up with SwiGLU fused into its epilogue, then down
    t_mma = (us["mma_gate_up_swiglu"] + us["mma_down"]) * 1e-6
    t_q8 = (us["q8_gate_up"] + us["q8_down"]) * 1e-6
    return {"workload": "config 3: 2048 tokens, Zipf(1.1)-skewed routing (max rows/expert ~200), Q4_K experts + shared",
            "us": {k: round(v, 1) for k, v in us.items()}, "us_back_to_back_mean": mean,
            "tflops": round(flops / t_mma / 1e12, 1), "f16_mfma_peak_frac": round(flops / t_mma / 1e12 / F16_MFMA_PEAK_TFLOPS, 4),
            "int8_peak_frac_equiv": round(flops / t_mma / 1e12 / INT8_MFMA_PEAK_TOPS, 4),
            "weight_gbs": round(wbytes / t_mma / 1e9, 1), "hbm_frac": round(wbytes / t_mma / 1e9 / HBM_PEAK_GBS, 4),
            "q8_dot_tops": round(flops / t_q8 / 1e12, 2),
            "layer_us": round(us["layer"], 1), "layer_tflops": round(flops / (us["layer"] * 1e-6) / 1e12, 1),
            "layer_hbm_frac": round(wbytes / (us["layer"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "experts_touched": touched, "max_rows_per_expert": int(cnt.max()), "flops": flops, "weight_bytes": wbytes}


def graph_us(torch, fn, reps):
    """µs per call of fn replayed from a HIP graph (10 calls a graph), so the host's launch rate is not what is timed;
    eager timing when fn cannot be captured"""
    fn()
    torch.cuda.synchronize()
    try:
        g = torch.cuda.CUDAGraph()
        st = torch.cuda.Stream()
        st.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(st):
            fn()
        torch.cuda.current_stream().wait_stream(st)
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            for _ in range(10):
                fn()
    except Exception:
        torch.cuda.synchronize()
        return time_us(torch, fn, reps)
    return time_us(torch, g.replay, reps) / 10


def median_us(torch, fn, reps):
    """the median of reps individually timed calls of fn (events around each call, the stream drained between them):
    the GPU's clock management moves a back-to-back series of the prompt-path kernels by up to ~30% (one series of 60
    gate|up calls ran 204-272 us), and the median is the steady figure"""
    fn()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1) * 1e3)
    ts.sort()
    return ts[len(ts) // 2]


def time_us(torch, fn, reps):
    fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps * 1e3


def bench_window16(layers, s, moe, torch, steps):
    """a 16-row decode window (a speculative verify window's rows, the reference's MAXT) through the same stacked
    layers on the fused decode, in a graph: µs per window-layer; the touched experts' bytes counted from the routing of
    the last layer (each read once a window)"""
    T = 16
    x0 = torch.empty((T, s.H), dtype=torch.float32, device="cuda")
    moe.synth_normal(x0, 4545, 1.0)
    x = x0.clone()
    f = moe.FusedDecode(layers, T)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        f(x)
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        x.copy_(x0)
        f(x)
    ms = time_us(torch, g.replay, max(steps // 5, 5)) / 1e3
    assert torch.isfinite(x).all()
    touched = int(f.piece("njobs", torch.int32, (2,))[0])   # distinct experts of the last layer's window + shared
    nbytes = (s.E + 1) * s.H * 4 + touched * expert_bytes(s, moe)
    us_l = ms * 1000 / len(layers)
    return {"workload": f"16-row decode window through {len(layers)} stacked Q4_K layers (fused decode, graph)",
            "us_per_window_layer": round(us_l, 2), "us_per_token_layer": round(us_l / T, 3),
            "experts_touched_last_layer": touched, "bytes_per_window_layer": nbytes,
            "gbs": round(nbytes / (us_l * 1e-6) / 1e9, 1)}


def bench_window(L, s, moe, torch, C=96, reps=20):
    """config 2: a verify window of 6 sequences x 16 draft rows = 96 rows through layer 0 (N(0,1) activations, no
    skew): the whole layer on the prompt path (router, top-k, permutation, gate|up + SwiGLU, down, combine)"""
    x = torch.empty((C, s.H), dtype=torch.float32, device="cuda")
    moe.synth_normal(x, 779, 1.0)
    y = torch.empty_like(x)
    b = moe.PrefillBuffers(s, C)
    us = median_us(torch, lambda: moe.prefill_layer_mma(L, x, y, b), reps)
    touched = int((b.cnt.cpu() > 0).sum()) + 1
    nbytes = touched * expert_bytes(s, moe) + (s.E + 1) * s.H * 4
    return {"workload": "config 2: 96 rows (6 x 16), one Q4_K layer, whole layer on the prompt path", "us": round(us, 1),
            "us_per_row": round(us / C, 2), "experts_touched": touched, "bytes": nbytes,
            "gbs": round(nbytes / (us * 1e-6) / 1e9, 1), "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def bench_type(moe, torch, wtype, NL, steps, warmup, C, seed0, sh_q8s=False):
    """one expert type at the bench's layer shapes: decode at batch 1 through NL stacked layers (the fused path in a
    graph, as config 1) and a C-token prompt chunk through layer 0 (experts on the matrix cores, Zipf-skewed routing).
    sh_q8s: the shared expert as dense Q8_0 matrices in the reference's q8s sums."""
    s = moe.LayerShape(H=2048, E=512, K=10, ff=512, wtype=wtype, shared=True, sh_q8s=sh_q8s)
    layers = [moe.MoeLayer.synthetic(s, seed=seed0 + l) for l in range(NL)]
    x0 = torch.empty((1, s.H), dtype=torch.float32, device="cuda")
    moe.synth_normal(x0, 4343, 1.0)
    x = x0.clone()
    f = moe.FusedDecode(layers, 1)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        f(x)
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        x.copy_(x0)
        f(x)
    ms = time_us(torch, g.replay, max(steps, 5)) / 1e3
    assert torch.isfinite(x).all()
    bytes_tl = (s.E + 1) * s.H * 4 + s.K * expert_bytes(s, moe) + shared_bytes(s, moe)
    gbs = bytes_tl * NL / (ms * 1e-3) / 1e9
    L = layers[0]
    xp = torch.empty((C, s.H), dtype=torch.float32, device="cuda")
    moe.synth_normal(xp, 780, 1.0)
    xn = torch.empty_like(xp)
    moe.residual_rmsnorm(xp, None, xn)
    b = moe.PrefillBuffers(s, C)
    moe.prefill_route(L, xn, b, torch.from_numpy(zipf_bias(s.E)).cuda())
    moe.to_f16(xn, b.xh)
    t_gu = median_us(torch, lambda: moe.moe_gate_up_swiglu_mma(L.gu_w, L.gu_stride, s.wtype, s.H, s.ff, b.jobs_gu, b.njobs,
                                                             b.cap, b.xh, b.h16), 11)
    t_dn = median_us(torch, lambda: moe.moe_down_mma(L.dn_w, L.dn_stride, s.dn_type, s.ff, s.H, b.jobs_dn, b.njobs, b.cap,
                                                   b.h16, b.part), 11)
    t_sh = graph_us(torch, lambda: moe.prefill_shared(L, b), 5) if sh_q8s else 0.0
    flops = 2 * (C * s.K + C) * 3 * s.ff * s.H
    touched = int((b.cnt.cpu() > 0).sum())
    wbytes = touched * expert_bytes(s, moe) + shared_bytes(s, moe)
    t = (t_gu + t_dn + t_sh) * 1e-6
    del layers, L, b
    torch.cuda.empty_cache()
    return {"decode_layers": NL, "decode_us_per_token_layer": round(ms * 1000 / NL, 3), "decode_gbs": round(gbs, 1),
            "decode_hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_token_layer": bytes_tl, "prefill_tokens": C,
            "prefill_us": {"mma_gate_up_swiglu": round(t_gu, 1), "mma_down": round(t_dn, 1),
                           **({"shared_q8s": round(t_sh, 1)} if sh_q8s else {})},
            "prefill_tflops": round(flops / t / 1e12, 1), "prefill_weight_gbs": round(wbytes / t / 1e9, 1),
            "prefill_hbm_frac": round(wbytes / t / 1e9 / HBM_PEAK_GBS, 4)}


def bench_q8_0(moe, torch, NL, steps, warmup):
    """config 4: the same layer shapes with Q8_0 experts: decode at batch 1 through NL stacked layers and a 4096-token
    prompt chunk through layer 0"""
    r = bench_type(moe, torch, moe.Q8_0, NL, steps, warmup, 4096, 5000)
    r["workload"] = f"config 4: Q8_0 experts; decode batch 1 through {NL} stacked layers; 4096-token prompt chunk"
    return r


def bench_q8s_shared(moe, torch, NL, steps, warmup):
    """config 1's layer shape with the shared expert as the reference's models carry it (dense Q8_0, q8s sums;
    src/model.cpp:807-809, src/engine.cu:936-945): decode through NL stacked layers, a 2048-token prompt chunk"""
    r = bench_type(moe, torch, moe.Q4_K, NL, steps, warmup, 2048, 9000, sh_q8s=True)
    r["workload"] = f"Q4_K experts + dense Q8_0 shared expert; decode batch 1 through {NL} stacked layers; 2048-token chunk"
    return r


def bench_hc_read(moe, torch, reps=20):
    """the hyper-connection read that produces the MoE input (src/hc.cuh), at the reference model's shape (N 2560,
    4 streams, rank 320; src/model.hpp:39): one read with the last half's output folded in, 20 reads a HIP graph;
    bytes: both Q8S matrices, the bf16 inject rows, w_norm, R read and written, bo, mixed and its q8_1"""
    N, HC, LR = 2560, 4, 320
    D = HC * N
    g = torch.Generator(device="cuda").manual_seed(77)
    q = lambda r, c: torch.randint(-127, 128, (r, c), dtype=torch.int8, device="cuda", generator=g)
    sc = lambda r, c: (torch.rand((r, c), device="cuda", generator=g) * 3e-4 + 1.5e-4).half().view(torch.int16)
    h = moe.HcRead(N, HC, LR, 1 + 0.1 * torch.randn(D, device="cuda", generator=g), q(LR, D), sc(LR, D // 32),
                   q(D, LR), sc(D, LR // 32), (0.02 * torch.randn((HC, D), device="cuda", generator=g)).bfloat16().view(torch.int16))
    out = {"workload": "hc read (src/hc.cuh) at N 2560, 4 streams, rank 320, with the fold; HIP-graph replays"}
    for T in (1, 4, 16):
        R0 = torch.randn((T, D), device="cuda", generator=g)
        R = R0.clone()
        bo = torch.randn((T, N), device="cuda", generator=g)
        inj = torch.randn((T, HC), device="cuda", generator=g)
        mixed = torch.empty((T, N), device="cuda")
        xq = torch.empty(T * (N // 32) * 36, dtype=torch.uint8, device="cuda")
        injo = torch.empty((T, HC), device="cuda")
        st = torch.cuda.Stream()
        st.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(st):
            h(R, mixed, xq, bo, inj, injo)
        torch.cuda.current_stream().wait_stream(st)
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):   # 20 reads a graph, so the graph's launch is not what is timed
            for _ in range(20):
                h(R, mixed, xq, bo, inj, injo)
        us = time_us(torch, gr.replay, reps) / 20
        assert torch.isfinite(mixed).all()
        nbytes = 2 * (LR * D + LR * D // 32 * 2) + HC * D * 2 + D * 4 + T * (2 * D * 4 + 2 * N * 4 + N // 32 * 36)
        out[f"T{T}"] = {"us": round(us, 2), "bytes": nbytes, "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                        "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    log(f"hc read: {out}")
    return out


def bench_other_types(moe, torch, NL, steps, warmup):
    """the other expert types the reference decodes (Q5_K, Q4_0, Q5_1) at the same shapes: decode through NL stacked
    layers, a 2048-token prompt chunk (not among the benchmark configurations; reported beside them)"""
    out = {}
    for name, t, seed in (("q5_k", moe.Q5_K, 6000), ("q4_0", moe.Q4_0, 7000), ("q5_1", moe.Q5_1, 8000)):
        out[name] = bench_type(moe, torch, t, NL, steps, warmup, 2048, seed)
        log(f"{name}: decode {out[name]['decode_us_per_token_layer']} us/token-layer, prefill {out[name]['prefill_us']}")
    return out


def cpu_baseline(L, s, moe, torch, x0, seconds):
    """the oracle (the reference's arithmetic restated in C) on config 0: one token through layer 0 on the host's
    cores, against the GPU's output for the same token"""
    import numpy as np

    from oracle import oracle as orc
    E1 = s.E + 1
    gu_g = torch.empty_like(L.gu_w)
    dn_g = torch.empty_like(L.dn_w)
    moe.store_unpack(s.wtype, L.gu_w, gu_g, E1, 2 * s.ff, s.H)
    moe.store_unpack(s.dn_type, L.dn_w, dn_g, E1, s.H, s.ff)
    xn = torch.empty_like(x0)
    moe.residual_rmsnorm(x0.clone(), None, xn)
    y = torch.empty_like(x0)
    b = moe.DecodeBuffers(s, 1)
    moe.decode_layer(L, xn, y, b)
    torch.cuda.synchronize()
    host = orc.LayerWeights(L.W.cpu().numpy(), gu_g.cpu().numpy(), dn_g.cpu().numpy(), s.wtype, s.H, s.E, s.K, s.ff, True,
                            dn_type=s.dn_type)
    x = xn.cpu().numpy()
    # every core this process may run on (the affinity mask), and beside it the box's stated CPU share for one GPU
    # (OMP_NUM_THREADS, 16 here): the faster of the two is the baseline, both are recorded
    nproc = os.cpu_count() or 1
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else nproc
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    counts = sorted({c for c in (avail, share) if c > 0})
    runs = {}
    for threads in counts:
        us1, _ = orc.time_layer_decode(host, x, threads, 3, 0)   # one short run to size the sample
        reps = max(5, min(200, int(seconds / len(counts) * 1e6 / max(us1, 1.0) / 2)))
        runs[threads] = (orc.time_layer_decode(host, x, threads, reps, 1 << 30)[0], reps)
    threads = min(runs, key=lambda c: runs[c][0])
    us, reps = runs[threads]
    oy, _, oi, _, _, _ = orc.layer_decode(host, x, threads)
    err = float(np.max(np.abs(y.cpu().numpy() - oy)) / np.max(np.abs(oy)))
    bytes_tl = E1 * s.H * 4 + (s.K + 1) * expert_bytes(s, moe)
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k = k.strip()
            if k in ("model name", "cpu family", "model", "stepping", "cpu MHz") and k not in info:
                info[k] = v.strip()
    except OSError:
        pass
    cpu = f"{info.get('model name', 'unknown')} (family {info.get('cpu family', '?')}, model {info.get('model', '?')}, " \
          f"stepping {info.get('stepping', '?')})"
    return {"value": round(us, 1), "unit": "us/token-layer", "cores": threads, "kind": "port",
            "sample": f"config 0: one token through one layer (layer 0 of the bench), median of {reps} runs, "
                      f"a 1 GiB sweep between runs",
            "nproc": nproc, "cores_available": avail, "omp_num_threads_env": share,
            "us_by_threads": {str(c): round(v[0], 1) for c, v in runs.items()},
            "gbs": round(bytes_tl / (us * 1e-6) / 1e9, 2), "cpu_model": cpu,
            "gpu_vs_cpu_max_rel_err": err, "gpu_vs_cpu_topi_equal": bool(np.array_equal(b.topi.cpu().numpy(), oi))}


if __name__ == "__main__":
    sys.exit(main())
