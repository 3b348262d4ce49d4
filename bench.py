#!/usr/bin/env python3
"""MoE-layer benchmark on one MI355X.

Default workload ("decode"): one bf16 token per step through one MoE layer
(hidden 2048, 512 experts top-10 + a sigmoid-gated shared expert, SwiGLU
intermediate 512, MLX affine 4-bit weights with group 64).  Consecutive
steps use different tokens and rotate over --layers resident layers so the
expert weights come from HBM, not from the 256 MB Infinity Cache.  Steps are
captured in a HIP graph (one node per kernel) and replayed.

Prints ONE JSON line: whole-job tokens/s, the roofline of the dominant
kernel (measured with HIP events on the stream it runs on), and the CPU
baseline (the oracle's C restatement of the reference C port, timed on this
host's cores on a bounded sample).
"""
import argparse
import importlib.util
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "qwen3.8-flash-next_amd")

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense bf16 MFMA
# symbol of the one-token gate/up launch (top-k inside) that hidden 2048 and
# 512 experts select (64 lanes per weight row, one chunk per lane, 8 experts
# per lane in the top-k), by activation type
GATEUP_SYMBOL = {True: "k_gateup_dec<64, 1, 2, true, 8>", False: "k_gateup_dec<64, 1, 2, false, 8>"}
METRIC = "MoE-layer tokens/sec at decode+prefill, 1 MI355X; % HBM BW / % MFMA peak"


def load_pkg():
    spec = importlib.util.spec_from_file_location(
        "qmoe_amd", os.path.join(PKG_DIR, "__init__.py"), submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["qmoe_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def q4_matrix_bytes(rows, cols, g=64):
    """codes (4 bits/weight) + one bf16 scale and one bf16 bias per group"""
    return rows * cols // 2 + rows * (cols // g) * 4


def expert_bytes(w):
    return 2 * q4_matrix_bytes(w.moe_inter, w.hidden, w.group_size) + \
        q4_matrix_bytes(w.hidden, w.moe_inter, w.group_size)


class Setup:
    """resident layers + per-step token batches for one workload"""

    def __init__(self, pkg, torch, w, n_layers, n_steps, seed_base=1000):
        self.pkg, self.torch, self.w = pkg, torch, w
        self.L = n_layers
        self.ctx = pkg.MoeContext.for_workload(w, n_layers=n_layers, max_tokens=w.n_tokens)
        self.bias = []
        sys.path.insert(0, ROOT)
        for layer in range(n_layers):
            rb = None
            if w.zipf_s > 0:
                rb = zipf_bias_host(w.n_experts, w.zipf_s, w.zipf_scale, w.seed * 1000003 + layer)
            self.ctx.synth_layer(layer, w.seed, with_norm=w.rms_norm, router_bias=rb)
        dt = torch.bfloat16 if w.x_bf16 else torch.float32
        kind = 0 if w.x_bf16 else 1
        self.x = []
        for i in range(n_steps):
            t = torch.empty((w.n_tokens, w.hidden), dtype=dt, device="cuda")
            pkg.synth_fill(t, kind, seed_base + i, 0, pkg.TAGS["X"], stddev=1.0)
            self.x.append(t)
        self.out = [torch.empty((w.n_tokens, w.hidden), dtype=torch.float32, device="cuda")
                    for _ in range(n_steps)]
        torch.cuda.synchronize()


def zipf_bias_host(E, s, scale, seed):
    """Zipf(s) router bias b_e = scale * ln p_{pi(e)} -- same definition as
    the oracle's orc_zipf_bias, restated here so the product path does not
    import the oracle"""
    import numpy as np

    def mix64(z):
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9 & 0xFFFFFFFFFFFFFFFF
        z = (z ^ (z >> 27)) * 0x94D049BB133111EB & 0xFFFFFFFFFFFFFFFF
        return z ^ (z >> 31)

    G = 0x9E3779B97F4A7C15
    key = mix64(seed ^ 0x5A17F00D)
    perm = list(range(E))
    for i in range(E - 1, 0, -1):
        j = mix64((key + (i + 1) * G) & 0xFFFFFFFFFFFFFFFF) % (i + 1)
        perm[i], perm[j] = perm[j], perm[i]
    r = np.arange(1, E + 1, dtype=np.float64)
    z = (r ** -s).sum()
    p = (np.array(perm, dtype=np.float64) + 1) ** -s / z
    return (scale * np.log(p)).astype(np.float32)


def capture(torch, fn):
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm the launch path outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def time_graph(torch, g, reps):
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1000.0  # seconds


def bench_layer(pkg, torch, w, n_layers, steps, warmup):
    """whole-layer steps: returns (seconds per step, setup)"""
    S = n_layers
    st = Setup(pkg, torch, w, n_layers, S)

    def run():
        for i in range(S):
            st.ctx.layer_forward(i % n_layers, st.x[i], out=st.out[i],
                                 residual=w.rms_norm)
    g = capture(torch, run)
    reps_w = max(1, math.ceil(warmup / S))
    time_graph(torch, g, reps_w)
    reps = max(1, math.ceil(steps / S))
    sec = time_graph(torch, g, reps)
    return sec / (reps * S), reps * S, reps_w * S, st


HC_COUNT, HC_LOWRANK = 4, 320  # the model's hyper connection (text_config hc_count, hc_lowrank)


def bench_hyper(pkg, torch, w, n_layers, steps, warmup):
    """whole hyper-connection layers: gated_residual, the MoE layer on the
    mixed rows and the inject update fused into the combine, on a resident
    hyper state [n, hc*hidden] updated in place; returns seconds per step"""
    ctx = pkg.MoeContext.for_workload(w, n_layers=n_layers, max_tokens=w.n_tokens)
    ctx.hc_enable(HC_COUNT, HC_LOWRANK)
    for layer in range(n_layers):
        rb = None
        if w.zipf_s > 0:
            rb = zipf_bias_host(w.n_experts, w.zipf_s, w.zipf_scale, w.seed * 1000003 + layer)
        ctx.synth_layer(layer, w.seed, router_bias=rb)
        ctx.hc_synth_layer(layer, w.seed)
    hyper = torch.empty((w.n_tokens, HC_COUNT * w.hidden), dtype=torch.float32, device="cuda")
    pkg.synth_fill(hyper, 1, 77, 0, pkg.TAGS["HYPER"], stddev=1.0)
    torch.cuda.synchronize()

    def run():
        for i in range(n_layers):
            ctx.hc_layer_forward(i, hyper, want_out=False)
    g = capture(torch, run)
    time_graph(torch, g, max(1, math.ceil(warmup / n_layers)))
    reps = max(1, math.ceil(steps / n_layers))
    sec = time_graph(torch, g, reps)
    ctx.close()
    return sec / (reps * n_layers), reps * n_layers


def bench_stream(pkg, torch, w, n_layers, slots, prefetch, steps, warmup):
    """decode with streamed experts: every layer's routed experts in pinned
    host memory, `slots` HBM expert slots per layer (ADAPTIVE policy,
    route-transition prefetch); one token through all layers per step.
    prefetch >= 0: run eagerly (each layer call reads its segment table on
    the host); prefetch -1: residency resolved on the GPU, the timed steps
    captured in one HIP graph and replayed once.  Returns seconds per layer
    call and the cache counters of the timed steps."""
    ctx = pkg.MoeContext.for_workload(w, n_layers=n_layers, max_tokens=w.n_tokens)
    ctx.stream_enable(slots, pkg.CACHE_ADAPTIVE, prefetch)
    for layer in range(n_layers):
        rb = None
        if w.zipf_s > 0:
            rb = zipf_bias_host(w.n_experts, w.zipf_s, w.zipf_scale, w.seed * 1000003 + layer)
        ctx.synth_layer(layer, w.seed, router_bias=rb)
    dt = torch.bfloat16 if w.x_bf16 else torch.float32
    xs = []
    for i in range(steps + warmup):
        t = torch.empty((w.n_tokens, w.hidden), dtype=dt, device="cuda")
        pkg.synth_fill(t, 0 if w.x_bf16 else 1, 5000 + i, 0, pkg.TAGS["X"], stddev=1.0)
        xs.append(t)
    out = torch.empty((w.n_tokens, w.hidden), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    for i in range(warmup):
        for layer in range(n_layers):
            ctx.layer_forward(layer, xs[i], out=out)
    torch.cuda.synchronize()

    def timed_steps():
        for i in range(warmup, warmup + steps):
            for layer in range(n_layers):
                ctx.layer_forward(layer, xs[i], out=out)

    g = None
    if prefetch < 0:
        # captured without a run first (the warmup steps warmed the launch
        # path), so the replay meets the cache the warmup left
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            timed_steps()
        torch.cuda.synchronize()
    s0 = ctx.stream_stats()
    t0 = time.perf_counter()
    if g is not None:
        g.replay()
    else:
        timed_steps()
    torch.cuda.synchronize()
    sec = time.perf_counter() - t0
    s1 = ctx.stream_stats()
    ctx.close()
    return sec / (steps * n_layers), {k: s1[k] - s0[k] for k in s1}


def bench_gateup(pkg, torch, st, reps_target=200):
    """dominant kernel of the one-token layer step: the launch that selects
    the top-k from the router logits and runs the grouped gate/up GEMV
    (qmoe_expert_gateup_topk, the launch qmoe_layer_forward makes for one
    token), one launch per resident layer with that layer's router logits;
    returns (avg seconds per launch, algorithmic bytes per launch averaged
    over the launches)"""
    w, ctx = st.w, st.ctx
    S = st.L
    logits, outs = [], []
    for i in range(S):
        r = ctx.router(i % st.L, st.x[i], want_logits=True)
        # [E+1]: the router logits, then a shared-gate logit (its value does
        # not change the work)
        logits.append(torch.cat([r["logits"][0], torch.zeros(1, device="cuda")]).contiguous())
        outs.append(ctx.expert_gateup_topk(i % st.L, st.x[i], logits[-1]))
    torch.cuda.synchronize()
    mb = q4_matrix_bytes(w.moe_inter, w.hidden, w.group_size)
    xbytes = w.hidden * (2 if w.x_bf16 else 4)
    algo = []
    for i in range(S):
        U = int(outs[i]["segments"][0].item())
        algo.append((U + 1) * 2 * mb + xbytes + (w.n_experts + 1) * 4 +
                    (w.top_k + 1) * w.moe_inter * 4)

    def run_raw():
        stream = torch.cuda.current_stream().cuda_stream
        for i in range(S):
            ctx.expert_gateup_topk_raw(i % st.L, st.x[i], logits[i], outs[i], stream)
    g = capture(torch, run_raw)
    time_graph(torch, g, 2)
    reps = max(1, math.ceil(reps_target / S))
    sec = time_graph(torch, g, reps)
    return sec / (reps * S), sum(algo) / len(algo)


def cpu_baseline(w, budget_s=12.0):
    """the oracle (C restatement of the reference C port's CPU path, q4
    weights resident, gemm_q4 for every expert) timed on this host"""
    sys.path.insert(0, ROOT)
    from oracle import oracle as orc
    import numpy as np
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
    t0 = time.time()
    rb = orc.zipf_bias(w.n_experts, w.zipf_s, w.zipf_scale, w.seed * 1000003) if w.zipf_s > 0 else None
    L = orc.Layer(w.hidden, w.n_experts, w.top_k, w.moe_inter, seed=w.seed, router_bias=rb,
                  with_norm=w.rms_norm, group_size=w.group_size)
    log(f"cpu baseline: host layer generated in {time.time() - t0:.1f}s")
    ntok_batch = w.n_tokens
    # sample: as many batches as fit the budget (at least 2)
    x = orc.gen_x(ntok_batch, w.hidden, 4242, bf16=w.x_bf16)
    one = L.time_forward(x, w.x_bf16, threads, warmup=1, iters=1)
    iters = max(2, min(50, int(budget_s / max(one, 1e-6))))
    med = L.time_forward(x, w.x_bf16, threads, warmup=1, iters=iters, residual=w.rms_norm)
    med1 = L.time_forward(x, w.x_bf16, 1, warmup=0, iters=max(1, min(3, int(4.0 / max(med * threads, 1e-6)))))
    return dict(value=ntok_batch / med, unit="tokens/s", cores=threads, kind="port",
                value_1thread=ntok_batch / med1,
                sample=f"{iters} runs of the {w.name} batch ({ntok_batch} token(s), one layer, "
                       f"H={w.hidden} E={w.n_experts} k={w.top_k} I={w.moe_inter}) through "
                       f"oracle/moe_oracle.c with q4-resident gemm_q4 experts; median; "
                       f"{threads} OpenMP threads (value_1thread: 1 thread)")


def copy_calibration(torch, mib):
    """a plain device copy of known size, run under rocprofv3 --pmc to
    calibrate FETCH_SIZE / WRITE_SIZE (bytes moved per dispatch are known)"""
    n = mib * 1024 * 1024 // 4
    a = torch.randn(n, device="cuda")
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(8):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": n * 4, "copy_bytes_written": n * 4, "copies": 8}),
          flush=True)


def measured_traffic(kernel_symbol, workload):
    """HBM traffic per launch of the roofline kernel, as measured by the two
    rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE) recorded in
    profiles/traffic.json, scaled by the copy-kernel calibration factors
    stored beside them; None when no measurement of this kernel/workload is
    recorded"""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    for r in rec.get("kernels", []):
        if r.get("kernel") == kernel_symbol and r.get("workload") == workload:
            return int(r["traffic_bytes_per_launch"])
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=480)
    ap.add_argument("--warmup", type=int, default=48)
    ap.add_argument("--workload", default="decode")
    ap.add_argument("--layers", type=int, default=48,
                    help="resident layers rotated over (defeats the Infinity Cache)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--extra", default="batched,prefill",
                    help="comma list of other workloads to time (secondary results)")
    ap.add_argument("--hyper", default="decode,batched,prefill",
                    help="comma list of workloads also timed as hyper-connection layers "
                         f"(hc {HC_COUNT}, rank {HC_LOWRANK}; secondary results)")
    ap.add_argument("--stream-device", default="16,64", metavar="LAYERS,SLOTS",
                    help="decode with streamed experts, residency resolved on the GPU, graph "
                         "replay ('' to skip)")
    ap.add_argument("--stream", default="16,64,16", metavar="LAYERS,SLOTS,PREFETCH",
                    help="also time Zipf decode with streamed experts (pinned host store, SLOTS "
                         "of 512 HBM expert slots per layer); empty: skip")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 8 plain copies of MIB MiB (counter calibration) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              f"(the MoE layer runs on a single MI355X here)", file=sys.stderr)
        sys.exit(2)

    import torch
    if args.copy_calibration > 0:
        copy_calibration(torch, args.copy_calibration)
        return
    pkg = load_pkg()
    dev = torch.cuda.get_device_name(0)
    log(f"device {dev}, library {pkg.version()}")
    w = pkg.WORKLOADS[args.workload]
    n_layers = max(1, min(args.layers, 48 if w.n_tokens <= 64 else 8))

    sec_step, steps, warm, st = bench_layer(pkg, torch, w, n_layers, args.steps, args.warmup)
    log(f"{w.name}: {sec_step * 1e6:.2f} us/step over {steps} steps, {n_layers} layers")
    roof = None
    if w.n_tokens == 1:
        k_sec, k_bytes = bench_gateup(pkg, torch, st)
        achieved = k_bytes / k_sec / 1e9
        log(f"gate/up kernel: {k_sec * 1e6:.2f} us/launch, {k_bytes / 1e6:.2f} MB -> {achieved:.0f} GB/s")
        roof = {
            "kernel": GATEUP_SYMBOL[w.x_bf16] + " (top-k + grouped gate/up GEMV + SiLU*up, one token)",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(GATEUP_SYMBOL[w.x_bf16], w.name),
            "avg_launch_us": round(k_sec * 1e6, 3),
            "algorithmic_bytes_per_launch": int(k_bytes),
        }
    value = w.n_tokens / sec_step
    layer_bytes = (10 + 1) * expert_bytes(w) + w.n_experts * w.hidden * 2 + w.hidden * 2

    extra = {}
    for name in [e for e in args.extra.split(",") if e and e != w.name]:
        we = pkg.WORKLOADS[name]
        st.ctx.close()
        del st
        torch.cuda.empty_cache()
        nl = 8 if we.n_tokens <= 64 else 2
        s_e, k_e, _, st = bench_layer(pkg, torch, we, nl, max(16, nl * 4), nl)
        extra[name] = dict(tokens_per_s=we.n_tokens / s_e, ms_per_step=s_e * 1e3,
                           tokens_per_step=we.n_tokens, layers_rotated=nl, steps=k_e)
        log(f"{name}: {s_e * 1e3:.3f} ms/step -> {we.n_tokens / s_e:.0f} tokens/s")
    st.ctx.close()
    del st
    torch.cuda.empty_cache()
    for name in [e for e in args.hyper.split(",") if e]:
        we = pkg.WORKLOADS[name]
        nl = 16 if we.n_tokens == 1 else (8 if we.n_tokens <= 64 else 2)
        s_h, k_h = bench_hyper(pkg, torch, we, nl, max(48, nl * 4), nl)
        extra[name + "+hyper"] = dict(tokens_per_s=we.n_tokens / s_h, ms_per_step=s_h * 1e3,
                                      tokens_per_step=we.n_tokens, layers_rotated=nl, steps=k_h,
                                      hc_count=HC_COUNT, hc_lowrank=HC_LOWRANK)
        log(f"{name}+hyper: {s_h * 1e3:.3f} ms/step -> {we.n_tokens / s_h:.0f} tokens/s")
        torch.cuda.empty_cache()
    if args.stream:
        nl, slots, pf = (int(v) for v in args.stream.split(","))
        we = pkg.Workload("decode-zipf", 2048, 512, 10, 512, 1, x_bf16=True, zipf_s=1.1)
        s_s, cs = bench_stream(pkg, torch, we, nl, slots, pf, steps=24, warmup=4)
        calls = cs["hits"] + cs["misses"]
        extra["decode+streamed"] = dict(
            tokens_per_s=1.0 / s_s, ms_per_layer_call=s_s * 1e3, layers=nl,
            slots_per_layer=slots, prefetch=pf, hit_rate=cs["hits"] / max(1, calls),
            host_to_hbm_bytes_per_layer_call=cs["bytes_in"] / (24 * nl),
            prefetched=cs["prefetched"], prefetch_hits=cs["prefetch_hits"],
            note="one token through one layer per call (tokens/s = layer calls/s), experts "
                 "streamed from pinned host memory over PCIe, eager (host reads each segment table)")
        log(f"decode+streamed: {s_s * 1e6:.1f} us per layer call, hit rate "
            f"{cs['hits'] / max(1, calls):.3f}, {cs['bytes_in'] / (24 * nl) / 1e6:.2f} MB in per call")
        torch.cuda.empty_cache()
    if args.stream_device:
        nl, slots = (int(v) for v in args.stream_device.split(","))
        we = pkg.Workload("decode-zipf", 2048, 512, 10, 512, 1, x_bf16=True, zipf_s=1.1)
        s_s, cs = bench_stream(pkg, torch, we, nl, slots, -1, steps=24, warmup=4)
        calls = cs["hits"] + cs["misses"]
        extra["decode+streamed-device"] = dict(
            tokens_per_s=1.0 / s_s, ms_per_layer_call=s_s * 1e3, layers=nl,
            slots_per_layer=slots, hit_rate=cs["hits"] / max(1, calls),
            host_to_hbm_bytes_per_layer_call=cs["bytes_in"] / (24 * nl),
            note="one token through one layer per call (tokens/s = layer calls/s), experts "
                 "streamed from pinned host memory over PCIe, residency resolved on the GPU, "
                 "no prefetch, timed steps replayed from one HIP graph")
        log(f"decode+streamed-device: {s_s * 1e6:.1f} us per layer call, hit rate "
            f"{cs['hits'] / max(1, calls):.3f}, {cs['bytes_in'] / (24 * nl) / 1e6:.2f} MB in per call")
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(w)
        log(f"cpu baseline: {cpu['value']:.1f} tokens/s with {cpu['cores']} threads, "
            f"{cpu['value_1thread']:.1f} with 1")

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm,
        "ms_per_step": round(sec_step * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"{w.name}: {w.n_tokens} token(s)/step through one MoE layer, "
                        f"hidden {w.hidden}, {w.n_experts} experts top-{w.top_k} + shared expert, "
                        f"SwiGLU intermediate {w.moe_inter}, q4 g{w.group_size} weights "
                        f"(bf16 scale/bias), {'bf16' if w.x_bf16 else 'f32'} activations, "
                        f"{n_layers} resident layers rotated",
            "tokens_per_step": w.n_tokens,
            "layer_algorithmic_bytes_per_token": layer_bytes if w.n_tokens == 1 else None,
            "layer_hbm_fraction": round(layer_bytes / sec_step / 1e9 / HBM_PEAK_GBS, 4)
            if w.n_tokens == 1 else None,
            "device": dev,
            "extra": extra,
        },
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
