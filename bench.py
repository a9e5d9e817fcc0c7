#!/usr/bin/env python3
"""bench.py -- the MoE expert-FFN hot path of moe-680m on one MI355X.

Metric: "MoE-FFN decode HBM GB/s (% of peak) @M=1; prefill tok/s @M=512
(% MFMA)".  One step = one token (M=1) through the 40-layer MoE-FFN stack of config 2:
per layer router softmax/top-8 (renormalised, BASELINE's convention) over seeded logits,
RMSNorm + the 9-expert IQ4_XS FFN + weighted combine + residual.  All 40 x 257 experts
(17.2 GB) are resident in HBM and every step routes differently, so weights stream from
HBM.  `value` is algorithmic bytes (602,316,800 per token) / wall time of the timed steps
(HIP graphs of 8 tokens; the HIP-event time is logged beside it).  The same line carries
config 0 (one layer, M = 1, the per-layer drop-in call moe_ffn_route; also routed from the
activations through moe_router_gemv_topk), config 1 prefill (M = 512, Zipf(1.1) router:
tok/s and the MFMA fraction, f16 operands; the f16 and bf16 dense peaks are the same
2.5 PFLOP/s), config 3 (one layer at M = 2, 4, 8: GB/s of the distinct experts selected)
and config 4 (M = 4096: MFMA fraction).  Per-layer and prefill steps are replayed several
per graph.

    python bench.py [--steps K] [--warmup W]      # one JSON line on stdout
    python bench.py --only config0 ...            # one leg, eager launches (for rocprofv3)
"""
import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))

H, I, E, LAYERS = 2048, 512, 256, 40
MATRIX_BYTES = H * I // 256 * 136                            # 557,056
EXPERT_BYTES = 3 * MATRIX_BYTES                              # 1,671,168
TOKEN_IO_BYTES = H * 4 + E * 4 + H * 4                       # x, logits, y of one token
DECODE_BYTES_PER_LAYER = 9 * EXPERT_BYTES + TOKEN_IO_BYTES   # 15,057,920
DECODE_BYTES_PER_TOKEN = LAYERS * DECODE_BYTES_PER_LAYER     # 602,316,800
# decode gate/up launch of one M=1 layer: the 9 experts' W1 and W3, x and the logits
DECODE_GATE_UP_BYTES = 9 * 2 * MATRIX_BYTES + H * 4 + E * 4  # 10,035,200
ROUTER_BYTES = E * H // 256 * 136                            # 278,528 (the gate matrix)
PREFILL_M = 512
PREFILL_FLOPS = 2 * (9 * PREFILL_M) * 3 * I * H             # 28,991,029,248
HBM_PEAK_GBS = 8000.0
F16_PEAK_TFLOPS = 2500.0  # dense f16 MFMA peak (the bf16 figure is the same)
# HBM bytes per decode-stack launch measured by rocprofv3 (FETCH_SIZE and WRITE_SIZE runs,
# calibrated on a plain copy); the summary and its commands are in this file:
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "decode_stack_config2.md")
LEGS = ("decode", "decode_routed", "config0", "prefill", "config3", "config4")
# config 2 routed from the activations: the 40 gate matrices are read too (IQ4_XS [256][2048])
DECODE_ROUTED_BYTES_PER_TOKEN = DECODE_BYTES_PER_TOKEN + LAYERS * (E * H // 256 * 136)
DTYPE = ("int8x2+f32: activations as two int8 planes (v_dot4_i32_i8 against the int8 IQ4_XS codebook, "
         "f32 scales and accumulation) in gate/up; f32 FMA in down and combine")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def load_pkg():
    sys.path.insert(0, ROOT)
    import __graft_entry__
    return __graft_entry__.load()


def capture(torch, fn):
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


# untimed replays before the timed replay of every leg but the headline (which honours --warmup)
SETTLE_MS = 20.0


def timed_graphs(torch, step, n, warm, per_graph, settle_ms=0.0):
    """Steps warm..n-1 replayed from graphs of per_graph steps after `warm` eager steps and
    one untimed replay of every graph (a graph's first launch pays its one-time upload, ~0.1 ms
    here, which is not a cost of the steps); with settle_ms, the graphs are replayed, untimed,
    for that long first (the shader clock ramps up under sustained load: config 3 at M = 8
    went 41.9 -> 37.5 us per step over a dozen back-to-back timings).  Returns (wall us per
    step, event us per step)."""
    for s in range(warm):
        step(s)
    torch.cuda.synchronize()
    groups = [list(range(b, min(b + per_graph, n))) for b in range(warm, n, per_graph)]
    graphs = [capture(torch, lambda g=g: [step(s) for s in g]) for g in groups]
    for g in graphs:
        g.replay()
    torch.cuda.synchronize()
    t_settle = time.perf_counter()
    while (time.perf_counter() - t_settle) * 1e3 < settle_ms:
        for g in graphs:
            g.replay()
        torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for g in graphs:
        g.replay()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    k = n - warm
    return wall * 1e6 / k, ev0.elapsed_time(ev1) * 1e3 / k


def kernel_times(ctx, fn, capacity=4096):
    ctx.timing_enable(capacity)
    fn()
    kt = ctx.timing_read()
    ctx.timing_enable(0)
    return {k: {"launches": n, "avg_us": round(ms * 1e3 / n, 3)} for k, (n, ms) in kt.items()}


def cpu_baseline(pkg, layer_dev, seconds):
    """The oracle's f32 port (C, OpenMP over each expert's output rows, all host threads) on
    decode M=1 token-layers of the config 0/2 workload, one resident layer, fresh routing per
    token, for about `seconds`; and the oracle's router + bucket fill at M = 512 and 4096."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    host = oracle.PackedLayer(layer_dev.cpu().numpy(), H, I, E)
    n_tok = 256
    x = oracle.gen_normal(pkg.seed_for(0, 0, pkg.TAG_X), 0, n_tok * H).reshape(n_tok, H)
    logits = oracle.gen_logits(pkg.seed_for(0, 0, pkg.TAG_L), n_tok, E)
    done, t0 = 0, time.perf_counter()
    while True:
        t = done % n_tok
        ids, w = oracle.router_topk(logits[t:t + 1], oracle.W_RENORM)
        x[t:t + 1] = oracle.moe_ffn_f32(host, x[t:t + 1], ids, w, 1.0, oracle.RMSNORM | oracle.ACCUMULATE,
                                        y=x[t:t + 1])
        done += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    gbs = done * DECODE_BYTES_PER_LAYER / el / 1e9
    rb = {}
    for M, kind, par, hot in ((512, 1, 1.1, 0.0), (4096, 2, 0.05, 1000.0)):
        lg = oracle.gen_logits(pkg.seed_for(1 if M == 512 else 4, 0, pkg.TAG_L), M, E, kind, par, hot)
        reps, t1 = 0, time.perf_counter()
        while reps < 3 or time.perf_counter() - t1 < 0.5:
            ids, w = oracle.router_topk(lg, oracle.W_RENORM)
            oracle.bucket_fill(ids, w, E)
            reps += 1
        rb[f"M{M}_ms"] = round((time.perf_counter() - t1) * 1e3 / reps, 3)
    return {"value": round(gbs, 4), "unit": "GB/s", "cores": oracle.num_threads(), "kind": "port",
            "sample": f"{done} decode token-layers (M=1, router + RMSNorm + 9-expert FFN + residual, "
                      f"RENORM) of one resident layer in {el:.1f} s: the oracle's f32 port "
                      f"(orc_moe_ffn_f32), OpenMP over output rows on {oracle.num_threads()} threads; "
                      f"host {platform.processor() or platform.machine()}, nproc {os.cpu_count()}",
            "router_bucket_fill": {**rb, "what": "oracle router top-8 + bucket fill (single thread), "
                                                 "config 1 and config 4 logits"}}


def profiled_traffic():
    """traffic_bytes_per_launch from the committed rocprofv3 summary, or None."""
    try:
        with open(TRAFFIC_PROFILE) as fh:
            for line in fh:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


# ---------------------------------------------------------------- decode stack timeline

# Events of one (workgroup, layer) record, in moe_stack_trace's order (k_stack.hip).
EV = {"start": 0, "x": 1, "routed": 2, "a": 3, "hpoll": 4, "h": 5, "b": 6, "pub": 7, "gather": 8,
      "xpub": 9, "xpoll": 10}
TRACE_EV = 16
# (name, from event, to event) of a layer's phases, all on one workgroup
PHASES = (("route (activation routing)", "x", "routed"), ("phase A", "x", "a"),
          ("phase A (after routing)", "routed", "a"), ("h exchange to B2", "a", "h"),
          ("phase B", "h", "b"), ("B3 + partial publish", "b", "pub"),
          ("cross-XCD partial gather", "pub", "gather"), ("reduce + x publish", "gather", "xpub"))


def stack_timeline(torch, pkg, ctx, routers, n_tok, routed):
    """Per-phase timeline of moe_decode_stack from the trace build (MOE680M_TRACE=1): n_tok
    tokens through the 40 layers (seeded logits, or routed from the activations); returns the
    per-phase medians over workgroups, averaged over layers 1..38 and the tokens."""
    import numpy as np
    nb = H // 8
    buf = torch.zeros(nb * LAYERS * TRACE_EV, dtype=torch.int64, device="cuda")
    x = pkg.gen_normal(H, pkg.seed_for(2, 0, pkg.TAG_X))
    logits = pkg.gen_logits(n_tok * LAYERS, E, pkg.seed_for(2, 0, pkg.TAG_L)).view(n_tok, LAYERS, E)
    if routed:
        for l in range(LAYERS):
            ctx.bind_router(l, routers[l])
    ctx.decode_stack(0, x, None if routed else logits[0], y=x, n_layers=LAYERS)  # warm
    torch.cuda.synchronize()
    ctx.stack_trace(buf)
    rows = []
    for t in range(n_tok):
        buf.zero_()
        ctx.decode_stack(0, x, None if routed else logits[t], y=x, n_layers=LAYERS)
        torch.cuda.synchronize()
        rows.append(buf.view(nb, LAYERS, TRACE_EV).cpu().numpy().astype(np.float64) * 10.0)  # 100 MHz -> ns
    ctx.stack_trace(None)
    assert ctx.device_flags() == 0
    if routed:
        for l in range(LAYERS):
            ctx.bind_router(l, None)
    ph = {name: [] for name, _, _ in PHASES}
    layer_ns, kernel_ns = [], []
    for tr in rows:
        t0 = tr[:, 0, EV["start"]].min()
        kernel_ns.append(tr[:, LAYERS - 1, EV["xpub"]].max() - t0)
        xs = tr[:, :, EV["x"]].max(axis=0)   # x of layer l in LDS on the last workgroup
        layer_ns += list(np.diff(xs)[1:-1])
        for name, a, b in PHASES:
            if name.startswith("route") or name.endswith("(after routing)"):
                if not routed:
                    continue
            elif name == "phase A" and routed:
                continue
            d = tr[:, 1:LAYERS - 1, EV[b]] - tr[:, 1:LAYERS - 1, EV[a]]
            ph[name].append(float(np.median(d)))
    out = {name: round(float(np.mean(v)) / 1e3, 3) for name, v in ph.items() if v}
    return {"tokens": n_tok, "routed_from_activations": routed,
            "kernel_us": round(float(np.mean(kernel_ns)) / 1e3, 2),
            "layer_us_median": round(float(np.median(layer_ns)) / 1e3, 3),
            "layer_us_mean": round(float(np.mean(layer_ns)) / 1e3, 3),
            "phase_us_median_over_workgroups": out,
            "what": "s_memrealtime stamps (100 MHz) by lane 0 of the named wave of every workgroup; a layer = "
                    "the time between the last workgroup's x of consecutive layers; phases are medians over "
                    "the 256 workgroups, averaged over layers 1..38"}


# ---------------------------------------------------------------- legs

def leg_decode(torch, pkg, ctx, K, W, eager, nl=LAYERS):
    """Config 2: one token through the 40 layers per moe_decode_stack launch (nl < 40 layers
    only in the eager runs profiled by rocprofv3, to split the traffic per launch into the
    per-layer part and the fixed part)."""
    dev = torch.device("cuda:0")
    nsteps = W + K
    logits = pkg.gen_logits(nsteps * LAYERS, E, pkg.seed_for(2, 0, pkg.TAG_L)).view(nsteps, LAYERS, E)
    x = pkg.gen_normal(H, pkg.seed_for(2, 0, pkg.TAG_X))
    ids = torch.empty((LAYERS, 9), dtype=torch.uint16, device=dev)
    wts = torch.empty((LAYERS, 9), dtype=torch.float32, device=dev)

    def token(s):
        ctx.decode_stack(0, x, logits[s][:nl], y=x, ids=ids, w=wts, rmsnorm=True)

    token(0)
    torch.cuda.synchronize()
    assert ctx.device_flags() == 0, "decode stack raised a device flag"
    assert eager or nl == LAYERS, "the timed decode leg runs all 40 layers"
    if eager:
        for s in range(nsteps):
            token(s)
        torch.cuda.synchronize()
        return None
    # Graphs of 8 consecutive tokens: in a serving loop the stack launch sits inside the
    # model's per-token graph, so the host-to-GPU gap between two separately launched graphs
    # is not a cost of this path.  The one-graph-per-token rate is logged beside it.
    us, us_ev = timed_graphs(torch, token, nsteps, W, 8)  # the headline: W eager tokens only
    gbs = DECODE_BYTES_PER_TOKEN / (us * 1e-6) / 1e9
    log(f"decode: {us:.1f} us/token ({us_ev:.1f} us by events; graphs of 8 tokens), "
        f"{gbs:.1f} GB/s = {100 * gbs / HBM_PEAK_GBS:.1f}% of HBM peak")
    assert torch.isfinite(x).all(), "decode chain produced non-finite values"
    assert ctx.device_flags() == 0, "decode stack raised a device flag"
    _, us_one = timed_graphs(torch, token, nsteps, W, 1, SETTLE_MS)
    log(f"decode, one graph per token: {us_one:.1f} us/token")
    kern = kernel_times(ctx, lambda: [token(s) for s in range(W, min(nsteps, W + 8))], 64)
    log(f"decode kernels: {kern}")
    return {"us": us, "gbs": gbs, "us_one_graph": us_one, "kern": kern}


def leg_decode_routed(torch, pkg, ctx, routers, K, W, eager):
    """Config 2 as a forward pass: every layer routed from its own RMSNorm'd input by its
    IQ4_XS gate matrix inside the one stack launch (moe_bind_router + MOE_STACK_ROUTE_GEMV)."""
    dev = torch.device("cuda:0")
    for l in range(LAYERS):
        ctx.bind_router(l, routers[l])
    nsteps = W + K
    x = pkg.gen_normal(H, pkg.seed_for(2, 0, pkg.TAG_X) + 1)
    ids = torch.empty((LAYERS, 9), dtype=torch.uint16, device=dev)
    wts = torch.empty((LAYERS, 9), dtype=torch.float32, device=dev)

    def token(s):
        ctx.decode_stack(0, x, y=x, ids=ids, w=wts, rmsnorm=True, n_layers=LAYERS)

    token(0)
    torch.cuda.synchronize()
    assert ctx.device_flags() == 0, "decode stack raised a device flag"
    if eager:
        for s in range(nsteps):
            token(s)
        torch.cuda.synchronize()
        return None
    us, us_ev = timed_graphs(torch, token, nsteps, W, 8, SETTLE_MS)
    gbs = DECODE_ROUTED_BYTES_PER_TOKEN / (us * 1e-6) / 1e9
    assert torch.isfinite(x).all() and ctx.device_flags() == 0
    kern = kernel_times(ctx, lambda: [token(s) for s in range(W, min(nsteps, W + 8))], 64)
    log(f"decode routed from activations: {us:.1f} us/token ({us_ev:.1f} by events), {gbs:.1f} GB/s = "
        f"{100 * gbs / HBM_PEAK_GBS:.1f}% of HBM peak; kernels {kern}")
    for l in range(LAYERS):
        ctx.bind_router(l, None)
    return {"workload": "config 2 as a forward pass: each of the 40 layers routed inside the stack launch "
                        "from its own RMSNorm'd input by an IQ4_XS [256][2048] gate matrix "
                        "(moe_bind_router, MOE_STACK_ROUTE_GEMV); graphs of 8 tokens",
            "us_per_token": round(us, 2), "bytes_per_token": DECODE_ROUTED_BYTES_PER_TOKEN,
            "gbs": round(gbs, 1), "hbm_peak_frac": round(gbs / HBM_PEAK_GBS, 4), "kernels": kern}


def leg_config0(torch, pkg, ctx, routers, eager):
    """Config 0: one layer, M = 1 -- moe_ffn_route (routing inside the decode launch); and the
    activation-routed variant: moe_router_gemv_topk for the logits only, then moe_ffn_route.
    Layers cycle over the 40 resident ones, so the selected experts come from HBM."""
    dev = torch.device("cuda:0")
    n, warm = 8 + 160, 8
    x0 = pkg.gen_normal(H, pkg.seed_for(0, 0, pkg.TAG_X)).view(1, H)
    y0 = torch.empty_like(x0)
    l0 = pkg.gen_logits(n, E, pkg.seed_for(0, 0, pkg.TAG_L)).view(n, 1, E)
    i0 = torch.empty((n, 1, 9), dtype=torch.uint16, device=dev)
    w0 = torch.empty((n, 1, 9), dtype=torch.float32, device=dev)
    g0 = torch.empty((n, 1, E), dtype=torch.float32, device=dev)

    def step(s):
        ctx.ffn_route(s % LAYERS, x0, l0[s], y=y0, ids=i0[s], w=w0[s], rmsnorm=True)

    def step_gemv(s):
        lg, _, _ = ctx.router_gemv_topk(routers[s % LAYERS], x0, rmsnorm=True, logits=g0[s], want_ids=False)
        ctx.ffn_route(s % LAYERS, x0, lg, y=y0, ids=i0[s], w=w0[s], rmsnorm=True)

    step(0)
    step_gemv(0)
    torch.cuda.synchronize()
    if eager:
        for s in range(n):
            step(s)
        for s in range(n):
            step_gemv(s)
        torch.cuda.synchronize()
        return None
    us, us_ev = timed_graphs(torch, step, n, warm, 8, SETTLE_MS)
    gbs = DECODE_BYTES_PER_LAYER / (us * 1e-6) / 1e9
    us_g, _ = timed_graphs(torch, step_gemv, n, warm, 8, SETTLE_MS)
    gbs_g = (DECODE_BYTES_PER_LAYER + ROUTER_BYTES) / (us_g * 1e-6) / 1e9
    kern = kernel_times(ctx, lambda: [step(s) for s in range(warm, warm + 64)], 256)
    kern_g = kernel_times(ctx, lambda: [step_gemv(s) for s in range(warm, warm + 64)], 512)
    gu = kern["decode_gate_up"]["avg_us"]
    gu_gbs = DECODE_GATE_UP_BYTES / (gu * 1e-6) / 1e9
    log(f"config 0: {us:.2f} us/step ({us_ev:.2f} by events), {gbs:.0f} GB/s = "
        f"{100 * gbs / HBM_PEAK_GBS:.1f}% of HBM peak; activation-routed {us_g:.2f} us/step; "
        f"kernels {kern} / {kern_g}")
    return {"workload": "config 0: one layer, M=1, N(0,1) x and logits, RMSNorm, top-8 renormalised + "
                        "shared; moe_ffn_route per step (routing inside the decode launch), steps "
                        "cycling the 40 resident layers, graphs of 8 steps",
            "us_per_step": round(us, 3), "bytes_per_step": DECODE_BYTES_PER_LAYER, "gbs": round(gbs, 1),
            "hbm_peak_frac": round(gbs / HBM_PEAK_GBS, 4),
            "roofline": {"bound": "hbm", "kernel": "decode_gate_up", "achieved": round(gu_gbs, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
                         "bytes_per_launch": DECODE_GATE_UP_BYTES, "avg_us": gu},
            "kernels": kern,
            "activation_routed": {"what": "moe_router_gemv_topk for the logits only (x . Wg over an IQ4_XS "
                                          "[256][2048] gate matrix per layer) + moe_ffn_route (the top-8 "
                                          "inside the decode launch)",
                                  "us_per_step": round(us_g, 3), "gbs": round(gbs_g, 1),
                                  "bytes_per_step": DECODE_BYTES_PER_LAYER + ROUTER_BYTES, "kernels": kern_g}}


def leg_prefill(torch, pkg, ctx, PK, eager):
    """Config 1: M = 512, Zipf(1.1)-biased logits, moe_ffn_route (router + FFN) per step."""
    dev = torch.device("cuda:0")
    pw, pn = 3, 3 + PK
    xp = pkg.gen_normal(PREFILL_M * H, pkg.seed_for(1, 0, pkg.TAG_X)).view(PREFILL_M, H)
    yp = torch.empty_like(xp)
    plog = pkg.gen_logits(pn * PREFILL_M, E, pkg.seed_for(1, 0, pkg.TAG_L), 1, 1.1).view(pn, PREFILL_M, E)
    pids = torch.empty((pn, PREFILL_M, 9), dtype=torch.uint16, device=dev)
    pwt = torch.empty((pn, PREFILL_M, 9), dtype=torch.float32, device=dev)

    def prefill(s):
        # moe_ffn_route: the routing runs inside the first prefill launch
        ctx.ffn_route(s % LAYERS, xp, plog[s], y=yp, ids=pids[s], w=pwt[s])

    prefill(0)
    torch.cuda.synchronize()
    if eager:
        for s in range(pn):
            prefill(s)
        torch.cuda.synchronize()
        return None
    us, _ = timed_graphs(torch, prefill, pn, pw, 5, SETTLE_MS)
    p_ms = us * 1e-3
    tflops = PREFILL_FLOPS / (us * 1e-6) / 1e12
    active = [int(torch.unique(pids[s].view(-1).to(torch.int32)).numel()) for s in range(pw, pn)]
    log(f"prefill M={PREFILL_M}: {us:.1f} us/step, {PREFILL_M / (us * 1e-6):.0f} tok/s, "
        f"{tflops:.1f} TFLOP/s = {100 * tflops / F16_PEAK_TFLOPS:.2f}% of the f16 MFMA peak; "
        f"active experts {min(active)}-{max(active)}")
    pkern = kernel_times(ctx, lambda: [prefill(s) for s in range(pw, min(pn, pw + 8))], 8 * 64)
    log(f"prefill kernels: {pkern}")
    pgu_us = pkern["prefill_gate_up"]["avg_us"]
    pgu_tflops = (PREFILL_FLOPS * 2 / 3) / (pgu_us * 1e-6) / 1e12  # gate/up: 2/3 of the FLOPs
    return {"workload": "config 1: M=512, Zipf(1.1) router bias, one layer per step "
                        "(cycling the 40 resident layers); moe_ffn_route per step (routing inside the "
                        "bucket-fill launch)",
            "dtype": "f16 MFMA (operands scaled by exact powers of two), f32 accumulate",
            "ms_per_step": round(p_ms, 5), "tok_per_s": round(PREFILL_M / (us * 1e-6), 1),
            "tflops": round(tflops, 2), "mfma_frac": round(tflops / F16_PEAK_TFLOPS, 4),
            "active_experts": [min(active), max(active)],
            "roofline": {"bound": "mfma", "kernel": "prefill_gate_up", "achieved": round(pgu_tflops, 2),
                         "peak": F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(pgu_tflops / F16_PEAK_TFLOPS, 4), "avg_us": pgu_us},
            "kernels": pkern}


def leg_config3(torch, pkg, ctx, eager):
    """Config 3: one layer, M = 2, 4, 8 with independent x and logits per token."""
    dev = torch.device("cuda:0")
    c3 = {}
    for Mv in (2, 4, 8):
        n3 = 3 + 30
        x3 = pkg.gen_normal(Mv * H, pkg.seed_for(3, Mv, pkg.TAG_X)).view(Mv, H)
        y3 = torch.empty_like(x3)
        l3 = pkg.gen_logits(n3 * Mv, E, pkg.seed_for(3, Mv, pkg.TAG_L)).view(n3, Mv, E)
        i3 = torch.empty((n3, Mv, 9), dtype=torch.uint16, device=dev)
        w3 = torch.empty((n3, Mv, 9), dtype=torch.float32, device=dev)

        def step3(s, x3=x3, y3=y3, l3=l3, i3=i3, w3=w3):
            ctx.ffn_route(s % LAYERS, x3, l3[s], y=y3, ids=i3[s], w=w3[s])

        step3(0)
        torch.cuda.synchronize()
        if eager:
            for s in range(n3):
                step3(s)
            torch.cuda.synchronize()
            continue
        us3, _ = timed_graphs(torch, step3, n3, 3, 5, SETTLE_MS)
        nexp = [int(torch.unique(i3[s].view(-1).to(torch.int32)).numel()) for s in range(3, n3)]
        b3 = sum(nexp) / len(nexp) * EXPERT_BYTES + Mv * TOKEN_IO_BYTES
        gbs3 = b3 / (us3 * 1e-6) / 1e9
        c3[f"M{Mv}"] = {"us_per_step": round(us3, 2), "distinct_experts": round(sum(nexp) / len(nexp), 1),
                        "bytes_per_step": int(b3), "gbs": round(gbs3, 1),
                        "hbm_peak_frac": round(gbs3 / HBM_PEAK_GBS, 4)}
        log(f"config 3, M={Mv}: {us3:.1f} us/step (moe_ffn_route), {gbs3:.0f} GB/s = "
            f"{100 * gbs3 / HBM_PEAK_GBS:.1f}% of HBM peak; {c3[f'M{Mv}']['distinct_experts']} experts")
    if eager:
        return None
    return {"workload": "config 3: one layer, M in {2, 4, 8}, independent N(0,1) x and logits per token; "
                        "moe_ffn_route per step, graph replays",
            "dtype": "int8x2+f32: activations and, in the down product, h as two int8 planes per 32 "
                     "elements (v_dot4_i32_i8 against the int8 IQ4_XS codebook), f32 scales and accumulation",
            **c3}


def leg_config4(torch, pkg, layer0, eager):
    """Config 4: M = 4096, N(0,1) logits with 5% of tokens forced onto one hot expert."""
    dev = torch.device("cuda:0")
    M4 = 4096
    ctx4 = pkg.Context(H, I, E, 1, M4, pkg.W_RENORM)
    ctx4.bind_packed(0, layer0)
    n4 = 2 + 6
    x4 = pkg.gen_normal(M4 * H, pkg.seed_for(4, 0, pkg.TAG_X)).view(M4, H)
    y4 = torch.empty_like(x4)
    l4 = pkg.gen_logits(n4 * M4, E, pkg.seed_for(4, 0, pkg.TAG_L), 2, 0.05, 1000.0).view(n4, M4, E)
    i4 = torch.empty((n4, M4, 9), dtype=torch.uint16, device=dev)
    w4 = torch.empty((n4, M4, 9), dtype=torch.float32, device=dev)

    def step4(s):
        ctx4.ffn_route(0, x4, l4[s], y=y4, ids=i4[s], w=w4[s])

    step4(0)
    torch.cuda.synchronize()
    if eager:
        for s in range(n4):
            step4(s)
        torch.cuda.synchronize()
        ctx4.close()
        return None
    us4, _ = timed_graphs(torch, step4, n4, 2, 1, SETTLE_MS)
    kern4 = kernel_times(ctx4, lambda: [step4(s) for s in range(2, n4)], 256)
    ctx4.close()
    fl4 = 2 * (9 * M4) * 3 * I * H
    tf4 = fl4 / (us4 * 1e-6) / 1e12
    log(f"config 4, M={M4}: {us4:.1f} us/step, {M4 / (us4 * 1e-6):.0f} tok/s, {tf4:.1f} TFLOP/s = "
        f"{100 * tf4 / F16_PEAK_TFLOPS:.2f}% of the f16 MFMA peak; kernels {kern4}")
    return {"workload": "config 4: one layer, M=4096, N(0,1) logits with 5% of tokens forced onto one hot "
                        "expert; moe_ffn_route per step (routing inside the first launch)",
            "us_per_step": round(us4, 1), "tok_per_s": round(M4 / (us4 * 1e-6), 1),
            "tflops": round(tf4, 2), "mfma_frac": round(tf4 / F16_PEAK_TFLOPS, 4), "kernels": kern4}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=40)  # ~10 ms of eager tokens: the clock ramps up
    ap.add_argument("--prefill-steps", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra-configs", action="store_true",
                    help="skip the config 0, 3 and 4 legs")
    ap.add_argument("--only", choices=LEGS,
                    help="run this leg alone with eager launches (no graphs, no JSON line): "
                         "the program profiled by rocprofv3")
    ap.add_argument("--stack-timeline", type=int, default=0, metavar="TOKENS",
                    help="print the decode stack's per-phase timeline over this many tokens (seeded and "
                         "activation-routed) from the trace build libmoe680m_trace.so, and nothing else")
    ap.add_argument("--stack-layers", type=int, default=LAYERS, metavar="N",
                    help="with --only decode: layers per moe_decode_stack launch (1..40; the timed "
                         "bench always runs 40)")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="run a plain device copy of this size first (scales PMC byte counters)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        log("bench.py measures one GPU only: this build has no multi-GPU path "
            "(the sharding design is in DESIGN.md); run with --gpus 1")
        sys.exit(2)

    if args.stack_timeline:
        os.environ["MOE680M_TRACE"] = "1"   # the package then loads libmoe680m_trace.so
    import torch
    pkg = load_pkg()
    torch.cuda.set_device(0)
    dev = torch.device("cuda:0")
    props = torch.cuda.get_device_properties(0)
    log(f"device: {props.name}, {props.multi_processor_count} CUs")

    if args.copy_calibration_mib:
        n = args.copy_calibration_mib << 20
        src = torch.ones(n // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration copy: {n} bytes read, {n} bytes written")
        del src, dst

    K, W = args.steps, args.warmup
    ctx = pkg.Context(H, I, E, LAYERS, PREFILL_M, pkg.W_RENORM)
    t0 = time.perf_counter()
    layer0 = None
    for l in range(LAYERS):
        buf = pkg.gen_layer(H, I, E, pkg.seed_for(2, l, pkg.TAG_W))
        ctx.bind_packed(l, buf)  # the library keeps its own copy
        if l == 0:
            layer0 = buf
    routers = [pkg.gen_iq4xs(E * H // 256, pkg.seed_for(2, l, pkg.TAG_W ^ 0x100)) for l in range(LAYERS)]
    torch.cuda.synchronize()
    log(f"generated {LAYERS} layers x {E + 1} experts ({LAYERS * (E + 1) * EXPERT_BYTES / 1e9:.2f} GB) "
        f"in {time.perf_counter() - t0:.2f} s")

    if args.stack_timeline:
        for routed in (False, True):
            tl = stack_timeline(torch, pkg, ctx, routers, args.stack_timeline, routed)
            log(f"stack timeline: {tl}")
            print(json.dumps(tl), flush=True)
        ctx.close()
        return

    if args.only:
        eager = True
        {"decode": lambda: leg_decode(torch, pkg, ctx, K, W, eager, args.stack_layers),
         "decode_routed": lambda: leg_decode_routed(torch, pkg, ctx, routers, K, W, eager),
         "config0": lambda: leg_config0(torch, pkg, ctx, routers, eager),
         "prefill": lambda: leg_prefill(torch, pkg, ctx, args.prefill_steps, eager),
         "config3": lambda: leg_config3(torch, pkg, ctx, eager),
         "config4": lambda: leg_config4(torch, pkg, layer0, eager)}[args.only]()
        log(f"leg {args.only}: done")
        ctx.close()
        return

    dec = leg_decode(torch, pkg, ctx, K, W, False)
    kern = dec["kern"]
    stack_us = kern["decode_stack"]["avg_us"]
    stack_gbs = DECODE_BYTES_PER_TOKEN / (stack_us * 1e-6) / 1e9
    extra = {}
    if not args.no_extra_configs:
        extra["decode_routed"] = leg_decode_routed(torch, pkg, ctx, routers, K, W, False)
        extra["config0"] = leg_config0(torch, pkg, ctx, routers, False)
    prefill = leg_prefill(torch, pkg, ctx, args.prefill_steps, False)
    if not args.no_extra_configs:
        extra["config3"] = leg_config3(torch, pkg, ctx, False)
        extra["config4"] = leg_config4(torch, pkg, layer0, False)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(pkg, layer0, args.cpu_seconds)
        cpu["router_bucket_fill"]["gpu_bucket_fill_us"] = {
            "M512": prefill["kernels"].get("bucket_fill", {}).get("avg_us"),
            "M4096": extra.get("config4", {}).get("kernels", {}).get("bucket_fill", {}).get("avg_us")}
        log(f"cpu baseline: {cpu}")

    ms_step = dec["us"] * 1e-3
    out = {
        "metric": "MoE-FFN decode HBM GB/s (% of peak) @M=1; prefill tok/s @M=512 (% MFMA)",
        "value": round(dec["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE,
        "data": "synthetic (seeded IQ4_XS weights, N(0,1) activations and router logits; "
                "random-init, no checkpoint)",
        "config": {"workload": "config 2: 40-layer MoE-FFN decode stack, M=1 token/step, "
                               "hidden 2048, 256+1 experts (top-8 renormalised + shared), inter 512, "
                               "IQ4_XS, all 10,280 experts resident (17.19 GB)",
                   "bytes_per_step": DECODE_BYTES_PER_TOKEN, "tokens_per_step": 1,
                   "timing": "steps replayed from HIP graphs of 8 tokens each",
                   "us_per_step_one_graph_per_token": round(dec["us_one_graph"], 2)},
        "hbm_peak_frac": round(dec["gbs"] / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "kernel": "decode_stack", "achieved": round(stack_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(stack_gbs / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic(),
                     "traffic_source": "rocprofv3 FETCH_SIZE x2 + WRITE_SIZE x1 per launch, "
                                       "profiles/decode_stack_config2.md",
                     "bytes_per_launch": DECODE_BYTES_PER_TOKEN, "avg_us": stack_us},
        "kernels": kern,
        "prefill": prefill,
        **extra,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
