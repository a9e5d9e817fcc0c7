#!/usr/bin/env python3
"""bench.py -- the MoE expert-FFN hot path of moe-680m on one MI355X.

Metric: "MoE-FFN decode HBM GB/s (% of peak) @M=1; prefill tok/s @M=512
(% MFMA)".  One step = one token (M=1) through the 40-layer MoE-FFN stack of config 2:
per layer router softmax/top-8 over seeded logits, RMSNorm + the 9-expert IQ4_XS FFN +
weighted combine + residual.  All 40 x 257 experts (17.2 GB) are resident in HBM and
every step routes differently, so weights stream from HBM.  `value` is algorithmic bytes
(602,316,800 per token) / wall time of the timed steps (HIP graphs of 8 tokens; the HIP-event
time is logged beside it).  The prefill leg (config 1: M=512, Zipf(1.1)-biased router) is reported in the
same line, with tok/s and the MFMA fraction (f16 operands; the f16 and bf16 dense peaks are
the same 2.5 PFLOP/s), and so are config 3 (one layer at M = 2, 4, 8: GB/s of the distinct
experts selected) and config 4 (M = 4096: MFMA fraction); prefill and config 3 steps are
replayed five per graph.

    python bench.py [--steps K] [--warmup W]      # one JSON line on stdout
"""
import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))

H, I, E, LAYERS = 2048, 512, 256, 40
EXPERT_BYTES = 3 * (H * I // 256 * 136)                     # 1,671,168
DECODE_BYTES_PER_LAYER = 9 * EXPERT_BYTES + H * 4 + E * 4 + H * 4   # 15,057,920
DECODE_BYTES_PER_TOKEN = LAYERS * DECODE_BYTES_PER_LAYER     # 602,316,800
PREFILL_M = 512
PREFILL_FLOPS = 2 * (9 * PREFILL_M) * 3 * I * H             # 28,991,029,248
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0  # dense bf16 and f16 MFMA peak
# HBM bytes per decode-stack launch measured by rocprofv3 (FETCH_SIZE and WRITE_SIZE runs,
# calibrated on a plain copy); the summary and its commands are in this file:
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "decode_stack_config2.md")


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


def cpu_baseline(pkg, layer_dev, seconds):
    """The oracle (C, OpenMP) on the host: decode M=1 token-layers of the same workload,
    one resident layer, fresh routing per token, for about `seconds`."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    host = oracle.PackedLayer(layer_dev.cpu().numpy(), H, I, E)
    n_tok = 256
    x = oracle.gen_normal(pkg.seed_for(0, 0, pkg.TAG_X), 0, n_tok * H).reshape(n_tok, H)
    logits = oracle.gen_logits(pkg.seed_for(0, 0, pkg.TAG_L), n_tok, E)
    done, t0 = 0, time.perf_counter()
    while True:
        t = done % n_tok
        lg = oracle.router_topk(logits[t:t + 1], oracle.W_REF)
        oracle.moe_ffn(host, x[t:t + 1], lg[0], lg[1], 1.0 / 9, oracle.RMSNORM | oracle.ACCUMULATE,
                       y=x[t:t + 1])
        done += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    gbs = done * DECODE_BYTES_PER_LAYER / el / 1e9
    threads = min(oracle.num_threads(), 9)  # one OpenMP task per selected expert
    return {"value": round(gbs, 4), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{done} decode token-layers (M=1, router + RMSNorm + 9-expert FFN + "
                      f"residual) of one resident layer in {el:.1f} s; f64 oracle, OpenMP over "
                      f"the 9 experts; host {platform.processor() or platform.machine()}, "
                      f"nproc {os.cpu_count()}"}


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--prefill-steps", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra-configs", action="store_true",
                    help="skip the config 3 (M=2,4,8 single layer) and config 4 (M=4096) legs")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="run a plain device copy of this size first (scales PMC byte counters)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        log("bench.py measures one GPU only: this build has no multi-GPU path "
            "(the sharding design is in DESIGN.md); run with --gpus 1")
        sys.exit(2)

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
    ctx = pkg.Context(H, I, E, LAYERS, PREFILL_M, pkg.W_REF)
    t0 = time.perf_counter()
    layers = []
    for l in range(LAYERS):
        buf = pkg.gen_layer(H, I, E, pkg.seed_for(2, l, pkg.TAG_W))
        ctx.bind_packed(l, buf)
        layers.append(buf)
    torch.cuda.synchronize()
    log(f"generated {LAYERS} layers x {E + 1} experts ({LAYERS * (E + 1) * EXPERT_BYTES / 1e9:.2f} GB) "
        f"in {time.perf_counter() - t0:.2f} s")

    # ---------------------------------------------------------------- decode (config 2)
    # One step = one token through the 40 layers in one moe_decode_stack launch (routing
    # from that token's per-layer logits, RMSNorm + MoE + residual per layer).
    nsteps = W + K
    logits = pkg.gen_logits(nsteps * LAYERS, E, pkg.seed_for(2, 0, pkg.TAG_L)).view(nsteps, LAYERS, E)
    x = pkg.gen_normal(H, pkg.seed_for(2, 0, pkg.TAG_X))
    ids = torch.empty((LAYERS, 9), dtype=torch.uint16, device=dev)
    wts = torch.empty((LAYERS, 9), dtype=torch.float32, device=dev)

    def token(s):
        ctx.decode_stack(0, x, logits[s], y=x, ids=ids, w=wts, rmsnorm=True)

    token(0)  # eager first pass (also checks the call path before capture)
    torch.cuda.synchronize()
    assert ctx.device_flags() == 0, "decode stack raised a device flag"
    # The timed tokens are replayed from graphs of up to TOKENS_PER_GRAPH consecutive tokens:
    # in a serving loop the stack launch sits inside the model's per-token graph, so the
    # host-to-GPU gap between two separately launched graphs (~15 us here) is not a cost of
    # this path.  The one-graph-per-token rate is logged beside it.
    TOKENS_PER_GRAPH = 8
    groups = [list(range(s, min(s + TOKENS_PER_GRAPH, nsteps))) for s in range(W, nsteps, TOKENS_PER_GRAPH)]
    graphs = [capture(torch, lambda g=g: [token(s) for s in g]) for g in groups]
    for s in range(W):
        token(s)
    graphs[0].replay()  # first replay of an instantiated graph carries one-time setup
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for g in graphs:
        g.replay()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / K
    decode_gbs = DECODE_BYTES_PER_TOKEN / (ms_step * 1e-3) / 1e9
    log(f"decode: {ms_step * 1e3:.1f} us/token ({ev0.elapsed_time(ev1) * 1e3 / K:.1f} us by events; "
        f"graphs of {TOKENS_PER_GRAPH} tokens), "
        f"{decode_gbs:.1f} GB/s = {100 * decode_gbs / HBM_PEAK_GBS:.1f}% of HBM peak")
    assert torch.isfinite(x).all(), "decode chain produced non-finite values"
    assert ctx.device_flags() == 0, "decode stack raised a device flag"
    del graphs
    graphs = [capture(torch, lambda s=s: token(s)) for s in range(W, nsteps)]
    torch.cuda.synchronize()
    ev0.record()
    for g in graphs:
        g.replay()
    ev1.record()
    torch.cuda.synchronize()
    per_token_graph_us = ev0.elapsed_time(ev1) * 1e3 / K
    log(f"decode, one graph per token: {per_token_graph_us:.1f} us/token")
    del graphs

    # per-kernel HIP-event timing of the same token steps, launched eagerly
    ctx.timing_enable(64)
    for s in range(W, min(nsteps, W + 8)):
        token(s)
    kt = ctx.timing_read()
    ctx.timing_enable(0)
    kern = {k: {"launches": n, "avg_us": round(ms * 1e3 / n, 3)} for k, (n, ms) in kt.items()}
    stack_us = kern["decode_stack"]["avg_us"]
    stack_gbs = DECODE_BYTES_PER_TOKEN / (stack_us * 1e-6) / 1e9
    log(f"decode kernels: {kern}")

    # the per-layer entry points (router + moe_ffn), for reference
    xl = x.clone().view(1, H)
    ctx.timing_enable(8 * LAYERS * 4)
    for s in range(W, min(nsteps, W + 2)):
        for l in range(LAYERS):
            ctx.router_topk(logits[s, l:l + 1], ids[l:l + 1], wts[l:l + 1])
            ctx.ffn(l, xl, ids[l:l + 1], wts[l:l + 1], y=xl, accumulate=True, rmsnorm=True)
    lkt = ctx.timing_read()
    ctx.timing_enable(0)
    layer_kern = {k: {"launches": n, "avg_us": round(ms * 1e3 / n, 3)} for k, (n, ms) in lkt.items()}
    log(f"per-layer path kernels: {layer_kern}")

    # ---------------------------------------------------------------- prefill (config 1)
    PK = args.prefill_steps
    pw = 3
    pn = pw + PK
    xp = pkg.gen_normal(PREFILL_M * H, pkg.seed_for(1, 0, pkg.TAG_X)).view(PREFILL_M, H)
    yp = torch.empty_like(xp)
    plog = pkg.gen_logits(pn * PREFILL_M, E, pkg.seed_for(1, 0, pkg.TAG_L), 1, 1.1).view(pn, PREFILL_M, E)
    pids = torch.empty((pn, PREFILL_M, 9), dtype=torch.uint16, device=dev)
    pw_ = torch.empty((pn, PREFILL_M, 9), dtype=torch.float32, device=dev)

    def prefill(s):
        ctx.router_topk(plog[s], pids[s], pw_[s])
        ctx.ffn(s % LAYERS, xp, pids[s], pw_[s], y=yp)

    prefill(0)
    torch.cuda.synchronize()
    # warm-up steps one per graph, timed steps five per graph (so the host's launch rate does
    # not show in a step), wall time bracketed by synchronisation like the decode leg
    PG = 5
    pgraphs = [capture(torch, lambda s=s: prefill(s)) for s in range(pw)]
    pgraphs += [capture(torch, lambda b=b: [prefill(s) for s in range(b, min(b + PG, pn))])
                for b in range(pw, pn, PG)]
    for g in pgraphs[:pw]:
        g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for g in pgraphs[pw:]:
        g.replay()
    torch.cuda.synchronize()
    p_ms = (time.perf_counter() - t0) * 1e3 / PK
    p_tflops = PREFILL_FLOPS / (p_ms * 1e-3) / 1e12
    active = [int(torch.unique(pids[s].view(-1).to(torch.int32)).numel()) for s in range(pw, pn)]
    log(f"prefill M={PREFILL_M}: {p_ms * 1e3:.1f} us/step, {PREFILL_M / (p_ms * 1e-3):.0f} tok/s, "
        f"{p_tflops:.1f} TFLOP/s = {100 * p_tflops / BF16_PEAK_TFLOPS:.2f}% of the f16/bf16 MFMA peak; "
        f"active experts {min(active)}-{max(active)}")
    del pgraphs
    ctx.timing_enable(8 * 64)
    for s in range(pw, min(pn, pw + 8)):
        prefill(s)
    pkt = ctx.timing_read()
    ctx.timing_enable(0)
    pkern = {k: {"launches": n, "avg_us": round(ms * 1e3 / n, 3)} for k, (n, ms) in pkt.items()}
    log(f"prefill kernels: {pkern}")
    # dominant prefill kernel: gate/up carries 2/3 of the FLOPs
    pgu_us = pkern["prefill_gate_up"]["avg_us"]
    pgu_tflops = (PREFILL_FLOPS * 2 / 3) / (pgu_us * 1e-6) / 1e12

    # ---------------------------------------------------------------- configs 3 and 4
    extra = {}
    if not args.no_extra_configs:
        # config 3: one layer, M = 2, 4, 8 tokens with independent activations and logits;
        # algorithmic bytes = the distinct experts the step selects + the tokens' x, logits, y
        c3 = {}
        for Mv in (2, 4, 8):
            n3 = 3 + 30
            x3 = pkg.gen_normal(Mv * H, pkg.seed_for(3, Mv, pkg.TAG_X)).view(Mv, H)
            y3 = torch.empty_like(x3)
            l3 = pkg.gen_logits(n3 * Mv, E, pkg.seed_for(3, Mv, pkg.TAG_L)).view(n3, Mv, E)
            i3 = torch.empty((n3, Mv, 9), dtype=torch.uint16, device=dev)
            w3 = torch.empty((n3, Mv, 9), dtype=torch.float32, device=dev)

            def step3(s, Mv=Mv, x3=x3, y3=y3, l3=l3, i3=i3, w3=w3):
                ctx.router_topk(l3[s], i3[s], w3[s])
                ctx.ffn(s % LAYERS, x3, i3[s], w3[s], y=y3)

            step3(0)
            torch.cuda.synchronize()
            # warm-up steps one per graph, timed steps PG per graph, as in the prefill leg
            g3 = [capture(torch, lambda s=s, f=step3: f(s)) for s in range(3)]
            g3 += [capture(torch, lambda b=b, f=step3: [f(s) for s in range(b, min(b + PG, n3))])
                   for b in range(3, n3, PG)]
            for g in g3[:3]:
                g.replay()
            torch.cuda.synchronize()
            ev0.record()
            for g in g3[3:]:
                g.replay()
            ev1.record()
            torch.cuda.synchronize()
            us3 = ev0.elapsed_time(ev1) * 1e3 / (n3 - 3)
            nexp = [int(torch.unique(i3[s].view(-1).to(torch.int32)).numel()) for s in range(3, n3)]
            b3 = sum(nexp) / len(nexp) * EXPERT_BYTES + Mv * (H * 4 + E * 4 + H * 4)
            gbs3 = b3 / (us3 * 1e-6) / 1e9
            c3[f"M{Mv}"] = {"us_per_step": round(us3, 2), "distinct_experts": round(sum(nexp) / len(nexp), 1),
                            "bytes_per_step": int(b3), "gbs": round(gbs3, 1),
                            "hbm_peak_frac": round(gbs3 / HBM_PEAK_GBS, 4)}
            log(f"config 3, M={Mv}: {us3:.1f} us/step (router + moe_ffn), {gbs3:.0f} GB/s = "
                f"{100 * gbs3 / HBM_PEAK_GBS:.1f}% of HBM peak; {c3[f'M{Mv}']['distinct_experts']} experts")
            del g3
        extra["config3"] = {"workload": "config 3: one layer, M in {2, 4, 8}, independent N(0,1) x and "
                                        "logits per token; router + moe_ffn per step, graph replays",
                            **c3}
        # config 4: M = 4096, N(0,1) logits with 5% of the tokens forced onto one hot expert
        M4 = 4096
        ctx4 = pkg.Context(H, I, E, 1, M4, pkg.W_REF)
        ctx4.bind_packed(0, layers[0])
        n4 = 2 + 6
        x4 = pkg.gen_normal(M4 * H, pkg.seed_for(4, 0, pkg.TAG_X)).view(M4, H)
        y4 = torch.empty_like(x4)
        l4 = pkg.gen_logits(n4 * M4, E, pkg.seed_for(4, 0, pkg.TAG_L), 2, 0.05, 1000.0).view(n4, M4, E)
        i4 = torch.empty((n4, M4, 9), dtype=torch.uint16, device=dev)
        w4 = torch.empty((n4, M4, 9), dtype=torch.float32, device=dev)

        def step4(s):
            ctx4.router_topk(l4[s], i4[s], w4[s])
            ctx4.ffn(0, x4, i4[s], w4[s], y=y4)

        step4(0)
        torch.cuda.synchronize()
        g4 = [capture(torch, lambda s=s: step4(s)) for s in range(n4)]
        for s in range(2):
            g4[s].replay()
        torch.cuda.synchronize()
        ev0.record()
        for s in range(2, n4):
            g4[s].replay()
        ev1.record()
        torch.cuda.synchronize()
        us4 = ev0.elapsed_time(ev1) * 1e3 / (n4 - 2)
        fl4 = 2 * (9 * M4) * 3 * I * H
        tf4 = fl4 / (us4 * 1e-6) / 1e12
        log(f"config 4, M={M4}: {us4:.1f} us/step, {M4 / (us4 * 1e-6):.0f} tok/s, {tf4:.1f} TFLOP/s = "
            f"{100 * tf4 / BF16_PEAK_TFLOPS:.2f}% of the f16/bf16 MFMA peak")
        del g4
        ctx4.close()
        extra["config4"] = {"workload": "config 4: one layer, M=4096, N(0,1) logits with 5% of tokens "
                                        "forced onto one hot expert; router + moe_ffn per step",
                            "us_per_step": round(us4, 1), "tok_per_s": round(M4 / (us4 * 1e-6), 1),
                            "tflops": round(tf4, 2), "mfma_frac": round(tf4 / BF16_PEAK_TFLOPS, 4)}

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(pkg, layers[0], args.cpu_seconds)
        log(f"cpu baseline: {cpu}")

    out = {
        "metric": "MoE-FFN decode HBM GB/s (% of peak) @M=1; prefill tok/s @M=512 (% MFMA)",
        "value": round(decode_gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded IQ4_XS weights, N(0,1) activations and router logits; "
                "random-init, no checkpoint)",
        "config": {"workload": "config 2: 40-layer MoE-FFN decode stack, M=1 token/step, "
                               "hidden 2048, 256+1 experts (top-8 + shared), inter 512, IQ4_XS, "
                               "all 10,280 experts resident (17.19 GB)",
                   "bytes_per_step": DECODE_BYTES_PER_TOKEN, "tokens_per_step": 1,
                   "timing": "steps replayed from HIP graphs of 8 tokens each",
                   "us_per_step_one_graph_per_token": round(per_token_graph_us, 2)},
        "hbm_peak_frac": round(decode_gbs / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "kernel": "decode_stack", "achieved": round(stack_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(stack_gbs / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic(),
                     "traffic_source": "rocprofv3 FETCH_SIZE x2 + WRITE_SIZE x1 per launch, "
                                       "profiles/decode_stack_config2.md",
                     "bytes_per_launch": DECODE_BYTES_PER_TOKEN, "avg_us": stack_us},
        "kernels": kern,
        "per_layer_path_kernels": layer_kern,
        "prefill": {"workload": "config 1: M=512, Zipf(1.1) router bias, one layer per step "
                                "(cycling the 40 resident layers)",
                    "dtype": "f16 MFMA (operands scaled by exact powers of two), f32 accumulate",
                    "ms_per_step": round(p_ms, 5),
                    "tok_per_s": round(PREFILL_M / (p_ms * 1e-3), 1),
                    "tflops": round(p_tflops, 2), "mfma_frac": round(p_tflops / BF16_PEAK_TFLOPS, 4),
                    "active_experts": [min(active), max(active)],
                    "roofline": {"bound": "mfma", "kernel": "prefill_gate_up",
                                 "achieved": round(pgu_tflops, 2), "peak": BF16_PEAK_TFLOPS,
                                 "unit": "TFLOP/s", "frac": round(pgu_tflops / BF16_PEAK_TFLOPS, 4),
                                 "avg_us": pgu_us},
                    "kernels": pkern},
        **extra,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
