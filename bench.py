#!/usr/bin/env python3
"""MoE-layer benchmark on one MI355X.

Default workload ("decode"): one bf16 token per step through one MoE layer
(hidden 2048, 512 experts top-10 + a sigmoid-gated shared expert, SwiGLU
intermediate 512, MLX affine 4-bit weights with group 64).  Consecutive
steps use different tokens and rotate over --layers resident layers so the
expert weights come from HBM, not from the 256 MB Infinity Cache.  The
--warmup steps run eagerly; the --steps timed steps are captured in one HIP
graph (one node per kernel), uploaded, and replayed once between two
synchronisations.

Prints ONE JSON line: whole-job tokens/s, the roofline of the dominant
kernel (measured with HIP events on the stream it runs on), the other
workloads (the tiny block, batched decode, prefill with its MFMA fraction,
48-layer decode) and the CPU baseline (the oracle's C restatement of the
reference C port, timed on this host's cores on bounded samples, in both
weight modes: warm fp32 experts and q4-resident experts).
"""
import argparse
import ctypes
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


def layer_token_bytes(w):
    """algorithmic bytes of one token through one layer: top-k routed experts
    + the shared expert, router [E,H] bf16, shared gate [H] bf16, the
    token's row in and out (2 x H x 2 B), and the RMSNorm weight (H x 2 B)
    when the layer has one: 21,573,632 B at hidden 2048 / 512 experts /
    top-10 / intermediate 512, 21,577,728 B with the norm"""
    return ((w.top_k + 1) * expert_bytes(w) + w.n_experts * w.hidden * 2 + w.hidden * 2 +
            4 * w.hidden + (2 * w.hidden if w.rms_norm else 0))


def step_bytes_batched(w, U):
    """algorithmic bytes of one batched step with U distinct routed experts:
    U x 1,769,472 + 4,395,008 B at 64 tokens of the decode shape (experts,
    shared expert, router and gate weights, 2 x H x 2 B per token)"""
    return (U + 1) * expert_bytes(w) + w.n_experts * w.hidden * 2 + w.hidden * 2 + \
        w.n_tokens * 4 * w.hidden


def prefill_flops(w):
    """(grouped GEMM: routed + shared experts, router) flops of one prefill step"""
    per_pair = 3 * 2 * w.hidden * w.moe_inter
    gemm = w.n_tokens * (w.top_k + 1) * per_pair
    router = w.n_tokens * 2 * w.hidden * w.n_experts
    return gemm, router


class Setup:
    """resident layers + per-step token batches for one workload"""

    def __init__(self, pkg, torch, w, n_layers, n_inputs, seed_base=1000, max_tokens=None):
        self.pkg, self.torch, self.w = pkg, torch, w
        self.L = n_layers
        self.ctx = pkg.MoeContext.for_workload(w, n_layers=n_layers,
                                               max_tokens=max_tokens or w.n_tokens)
        for layer in range(n_layers):
            rb = None
            if w.zipf_s > 0:
                rb = zipf_bias_host(w.n_experts, w.zipf_s, w.zipf_scale, w.seed * 1000003 + layer)
            self.ctx.synth_layer(layer, w.seed, with_norm=w.rms_norm, router_bias=rb)
        dt = torch.bfloat16 if w.x_bf16 else torch.float32
        kind = 0 if w.x_bf16 else 1
        self.x = []
        for i in range(n_inputs):
            t = torch.empty((w.n_tokens, w.hidden), dtype=dt, device="cuda")
            pkg.synth_fill(t, kind, seed_base + i, 0, pkg.TAGS["X"], stddev=1.0)
            self.x.append(t)
        self.out = [torch.empty((w.n_tokens, w.hidden), dtype=torch.float32, device="cuda")
                    for _ in range(n_inputs)]
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


_HIP = None


def hip():
    global _HIP
    if _HIP is None:
        _HIP = ctypes.CDLL("libamdhip64.so")
    return _HIP


def capture(torch, fn, warm=True):
    """fn's launches captured in one graph on a side stream; the graph is
    uploaded to the device so its first replay carries no set-up cost"""
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    if warm:
        with torch.cuda.stream(s):
            fn()  # warm the launch path outside capture
        torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        fn()
    torch.cuda.synchronize()
    try:
        rc = hip().hipGraphUpload(ctypes.c_void_p(g.raw_cuda_graph_exec()),
                                  ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if rc == 0:
            torch.cuda.synchronize()
    except (AttributeError, RuntimeError):
        pass
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


GRAPH_WARM_REPLAYS = 1  # untimed replays of the timed graph before its timed replay


def bench_layer(pkg, torch, w, n_layers, steps, warmup, n_inputs=None):
    """exactly `steps` timed whole-layer steps after `warmup` untimed eager
    ones; step i runs layer i % n_layers on input batch i % n_inputs.  The
    timed steps are one HIP graph, replayed GRAPH_WARM_REPLAYS times untimed
    (the first replay of a new graph carries ~45 us of one-time launch
    set-up on this runtime: 19.6 against 17.4 us per step over 20 decode
    steps, whatever the warm-up count), then timed over one replay.
    Returns (seconds per step, setup)."""
    X = n_inputs or max(1, min(max(steps, warmup), 64))
    st = Setup(pkg, torch, w, n_layers, X)

    def run(first, count):
        for i in range(first, first + count):
            st.ctx.layer_forward(i % n_layers, st.x[i % X], out=st.out[i % X], residual=w.rms_norm)

    run(0, warmup)
    torch.cuda.synchronize()
    g = capture(torch, lambda: run(warmup, steps), warm=warmup == 0)
    if GRAPH_WARM_REPLAYS:
        time_graph(torch, g, GRAPH_WARM_REPLAYS)
    sec = time_graph(torch, g, 1)
    return sec / steps, st


def distinct_experts(st, steps):
    """U (distinct routed experts) of each step, from an eager pass"""
    us = []
    torch = st.torch
    for i in range(min(steps, len(st.x))):
        st.ctx.layer_forward(i % st.L, st.x[i], out=st.out[i], residual=st.w.rms_norm)
        torch.cuda.synchronize()
        us.append(int(st.ctx.last_routing(st.w.n_tokens)["segments"][0].item()))
    return us


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
    X = len(st.x)
    logits, outs = [], []
    for i in range(S):
        r = ctx.router(i, st.x[i % X], want_logits=True)
        # [E+1]: the router logits, then a shared-gate logit (its value does
        # not change the work)
        logits.append(torch.cat([r["logits"][0], torch.zeros(1, device="cuda")]).contiguous())
        outs.append(ctx.expert_gateup_topk(i, st.x[i % X], logits[-1]))
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
            ctx.expert_gateup_topk_raw(i, st.x[i % X], logits[i], outs[i], stream)
    g = capture(torch, run_raw)
    time_graph(torch, g, 2)
    reps = max(1, math.ceil(reps_target / S))
    sec = time_graph(torch, g, reps)
    return sec / (reps * S), sum(algo) / len(algo)


def bench_prefill_stages(pkg, torch, st, reps=6):
    """the grouped expert GEMMs of the prefill layer, timed alone: the
    gate/up stage (activation packing + MFMA gate/up) and the down stage
    (MFMA down) of qmoe_expert_gateup / qmoe_expert_down on each resident
    layer's own routing; returns seconds per launch of each stage"""
    w, ctx = st.w, st.ctx
    n = w.n_tokens
    ds, hs, ys = [], [], []
    for layer in range(st.L):
        ctx.layer_forward(layer, st.x[layer], out=st.out[layer])
        torch.cuda.synchronize()
        r = ctx.last_routing(n)
        ds.append(dict(perm=r["perm"].clone(), segments=r["segments"].clone()))
        hs.append(torch.empty((n * w.top_k + n, w.moe_inter), dtype=torch.float32, device="cuda"))
    ys = torch.empty((n * w.top_k + n, w.hidden), dtype=torch.float32, device="cuda")
    for layer in range(st.L):
        ctx.expert_gateup(layer, st.x[layer], ds[layer], out=hs[layer])
    torch.cuda.synchronize()

    def gu():
        for layer in range(st.L):
            ctx.expert_gateup(layer, st.x[layer], ds[layer], out=hs[layer])

    def dn():
        for layer in range(st.L):
            ctx.expert_down(layer, hs[layer], n, ds[layer], out=ys)
    res = []
    for fn in (gu, dn):
        g = capture(torch, fn)
        time_graph(torch, g, 1)
        res.append(time_graph(torch, g, reps) / (reps * st.L))
    return res


DN_SHAPE = (2048, 16, 32, 128, 128, 4)  # hidden, key heads, value heads, dk, dv, conv taps


def dn_token_bytes(shape):
    """algorithmic HBM bytes of one token through one DeltaNet mixer: q4
    in_proj_qkv, in_proj_z, out_proj (codes + bf16 scale/bias per 64),
    bf16 in_proj_a/b and conv1d, the f32 vectors, the recurrent state read
    and written, the conv state read and written, x in and out"""
    d, hk, hv, dk, dv, kc = shape
    kd, vd = hk * dk, hv * dv
    cd = 2 * kd + vd
    q4 = lambda rows, cols: rows * cols // 2 + rows * (cols // 64) * 4
    w = q4(cd, d) + q4(vd, d) + q4(d, vd) + 2 * hv * d * 2 + cd * kc * 2 + (dv + 2 * hv) * 4
    state = 2 * (hv * dv * dk * 4) + 2 * ((kc - 1) * cd * 4)
    return w + state + 2 * d * 4


def bench_deltanet(pkg, torch, layers, steps, warmup):
    """one f32 token per step through one gated DeltaNet mixer of DN_SHAPE,
    layer i % layers on input i % 16 (states carried from step to step);
    random q4/bf16 weights (numpy), the same host arrays in every layer
    slot.  Returns seconds per token-layer."""
    import numpy as np
    d, hk, hv, dk, dv, kc = DN_SHAPE
    kd, vd = hk * dk, hv * dv
    cd = 2 * kd + vd
    rng = np.random.default_rng(0)
    bf = lambda n, std: ((rng.normal(0, std, n).astype(np.float32).view(np.uint32) + 0x8000) >> 16).astype(np.uint16)
    codes = lambda n: rng.integers(0, 2**32, n, dtype=np.uint32)
    host = dict(qkv_q=codes(cd * d // 8), qkv_s=bf(cd * d // 64, 0.02), qkv_b=bf(cd * d // 64, 0.01),
                z_q=codes(vd * d // 8), z_s=bf(vd * d // 64, 0.02), z_b=bf(vd * d // 64, 0.01),
                a_w=bf(hv * d, 0.02), b_w=bf(hv * d, 0.02),
                out_q=codes(d * vd // 8), out_s=bf(d * vd // 64, 0.02), out_b=bf(d * vd // 64, 0.01),
                conv_w=bf(cd * kc, 0.5), norm_w=(1 + rng.normal(0, 0.1, dv)).astype(np.float32),
                a_log=rng.normal(0, 1, hv).astype(np.float32), dt_bias=rng.normal(0, 1, hv).astype(np.float32))
    ctx = pkg.DeltaNetContext(d, hk, hv, dk, dv, kc, n_layers=layers, max_tokens=1)
    for layer in range(layers):
        ctx.upload_layer(layer, host)
    X = 16
    xs = [torch.randn((1, d), device="cuda") for _ in range(X)]
    outs = [torch.empty((1, d), device="cuda") for _ in range(X)]

    def run(first, count):
        for i in range(first, first + count):
            rc, msg = ctx.forward_raw(i % layers, xs[i % X].data_ptr(), 1, outs[i % X].data_ptr(),
                                      torch.cuda.current_stream().cuda_stream)
            if rc:
                raise RuntimeError(msg)

    run(0, warmup)
    torch.cuda.synchronize()
    g = capture(torch, lambda: run(warmup, steps), warm=False)
    sec = time_graph(torch, g, 1) / steps
    ctx.close()
    return sec


AT_SHAPE = (2048, 16, 2, 128, 4, 128, 2048, 4)  # hidden, heads, kv heads, head dim, indexer heads,
#                                                 indexer head dim, indexer budget, compress ratio
AT_CONTEXT = 4096  # cached tokens before the timed steps: past the budget, so the block mask runs


def at_token_bytes(shape, context):
    """algorithmic HBM bytes of one token through one attention mixer at
    `context` cached tokens with the block mask active: q4 q/k/v/o
    projections (codes + bf16 scale/bias per 64), the bf16 indexer matrix,
    every cached indexer key (pooled each step), the k and v rows of the
    kept blocks (budget) and of the token's own tail, the cache rows
    appended, x in and out"""
    d, h, kvh, hd, ih, ihd, budget, comp = shape
    q4 = lambda rows, cols: rows * cols // 2 + rows * (cols // 64) * 4
    w = q4(2 * h * hd, d) + 2 * q4(kvh * hd, d) + q4(d, h * hd) + (ih + 1) * ihd * d * 2
    kept = min(budget, context) + comp
    return w + context * ihd * 4 + 2 * kept * kvh * hd * 4 + (2 * kvh * hd + ihd) * 4 + 2 * d * 4


def bench_attention(pkg, torch, layers, steps, warmup, context=AT_CONTEXT):
    """one f32 token per step through one full-attention mixer of AT_SHAPE
    with its QSA indexer, layer i % layers, each layer's caches first filled
    with `context` tokens; random q4/bf16 weights (numpy), the same host
    arrays in every layer slot.  Returns seconds per token-layer."""
    import numpy as np
    d, h, kvh, hd, ih, ihd, budget, comp = AT_SHAPE
    rng = np.random.default_rng(1)
    bf = lambda n, std: ((rng.normal(0, std, n).astype(np.float32).view(np.uint32) + 0x8000) >> 16).astype(np.uint16)
    codes = lambda n: rng.integers(0, 2**32, n, dtype=np.uint32)
    q4 = lambda rows, cols: (codes(rows * cols // 8), bf(rows * cols // 64, 0.02), bf(rows * cols // 64, 0.01))
    host = {}
    for nm, (rows, cols) in (("q", (2 * h * hd, d)), ("k", (kvh * hd, d)), ("v", (kvh * hd, d)), ("o", (d, h * hd))):
        host[nm + "_q"], host[nm + "_s"], host[nm + "_b"] = q4(rows, cols)
    host["idx_w"] = bf((ih + 1) * ihd * d, 0.02)
    for nm, n in (("q_norm", hd), ("k_norm", hd), ("idx_q_norm", ihd), ("idx_k_norm", ihd)):
        host[nm] = (1 + rng.normal(0, 0.1, n)).astype(np.float32)
    chunk = 256
    cap = context + (warmup + steps) // layers + 2 * layers + chunk
    ctx = pkg.AttentionContext(d, h, kvh, hd, ih, ihd, budget, comp, kv_cap=cap, n_layers=layers,
                               max_tokens=chunk)
    xs = torch.randn((chunk, d), device="cuda") * 0.5
    for layer in range(layers):
        ctx.upload_layer(layer, host)
        for t0 in range(0, context, chunk):
            ctx.forward(layer, xs, t0)
    torch.cuda.synchronize()
    pos = [context] * layers
    X = 16
    xt = [torch.randn((1, d), device="cuda") for _ in range(X)]
    outs = [torch.empty((1, d), device="cuda") for _ in range(X)]

    def run(first, count):
        for i in range(first, first + count):
            layer = i % layers
            ctx.forward(layer, xt[i % X], pos[layer], out=outs[i % X])
            pos[layer] += 1

    run(0, warmup)
    torch.cuda.synchronize()
    g = capture(torch, lambda: run(warmup, steps), warm=False)
    sec = time_graph(torch, g, 1) / steps
    ctx.close()
    return sec


def hc_token_bytes(d, hc, R, inject):
    """algorithmic HBM bytes of one token through one hyper connection
    (gated_residual): the q4 down [R, hc*d] and up [hc*d, R] mix matrices,
    the f32 hc_norm, the bf16 inject matrix [hc, hc*d] when the connection
    has one, the hyper state read, the mixed row written and, with inject,
    the update's read and write of the hyper state"""
    q4 = lambda rows, cols: rows * cols // 2 + rows * (cols // 64) * 4
    b = q4(R, hc * d) + q4(hc * d, R) + hc * d * 4 + hc * d * 4 + d * 4
    if inject:
        b += hc * hc * d * 2 + 2 * hc * d * 4
    return b


STACK_LAYERS = 48  # the model's text stack: DeltaNet : attention = 3 : 1
STACK_CONTEXT = 4096  # cached tokens in each attention layer before the timed tokens


def stack_token_bytes(w, layers, context):
    """algorithmic HBM bytes of one token through the decoder stack: per
    layer the attention-block hyper connection, its mixer (DeltaNet or
    attention at `context` cached), the MLP hyper connection and the MoE
    layer on the f32 mixed row; then the final mixer"""
    types = [("attn" if (l + 1) % 4 == 0 else "dn") for l in range(layers)]
    moe = layer_token_bytes(w) + 2 * w.hidden  # f32 mixed row in instead of bf16
    total = 0
    for t in types:
        total += hc_token_bytes(w.hidden, HC_COUNT, HC_LOWRANK, True) * 2 + moe
        total += dn_token_bytes(DN_SHAPE) if t == "dn" else at_token_bytes(AT_SHAPE, context)
    return total + hc_token_bytes(w.hidden, HC_COUNT, HC_LOWRANK, False)


def bench_stack(pkg, torch, w, tokens, warmup, layers=STACK_LAYERS, context=STACK_CONTEXT):
    """one token per step through the decoder stack (qmoe.DecoderStack): 48
    layers, gated DeltaNet and full attention at 3 : 1, both hyper
    connections of every layer (hc 4, rank 320), the MoE layers of the
    decode workload (hidden 2048, 512 experts top-10, all resident), and the
    final mixer.  The attention layers' caches are first filled with
    `context` tokens (their mixer alone, random inputs); the DeltaNet
    states start empty.  `warmup` eager tokens, then `tokens` tokens
    captured in one HIP graph, replayed once untimed, then timed.  Random
    weights (device synthesis for the MoE and MLP hyper layers, numpy for
    the mixers and the attention-block hyper connections, the same host
    arrays in every slot).  Returns seconds per token."""
    import numpy as np
    types = pkg.decoder_layer_types(layers)
    d = w.hidden
    rng = np.random.default_rng(3)
    bf = lambda n, std: ((rng.normal(0, std, n).astype(np.float32).view(np.uint32) + 0x8000) >> 16).astype(np.uint16)
    codes = lambda n: rng.integers(0, 2**32, n, dtype=np.uint32)
    chunk = 256
    moe = pkg.MoeContext.for_workload(w, n_layers=layers, max_tokens=chunk)
    moe.hc_enable(HC_COUNT, HC_LOWRANK)
    for l in range(layers):
        moe.synth_layer(l, w.seed)
        moe.hc_synth_layer(l, w.seed)
    hcd = HC_COUNT * d
    ghost = dict(hc_norm=(1 + rng.normal(0, 0.1, hcd)).astype(np.float32),
                 down_q=codes(HC_LOWRANK * hcd // 8), down_s=bf(HC_LOWRANK * hcd // 64, 0.02),
                 down_b=bf(HC_LOWRANK * hcd // 64, 0.01), up_q=codes(hcd * HC_LOWRANK // 8),
                 up_s=bf(hcd * HC_LOWRANK // 64, 0.02), up_b=bf(hcd * HC_LOWRANK // 64, 0.01),
                 inject_w=bf(HC_COUNT * hcd, 0.02))
    gr = pkg.GatedResidualContext(d, HC_COUNT, HC_LOWRANK, n_slots=layers + 1, max_tokens=chunk)
    for l in range(layers):
        gr.upload_slot(l, ghost)
    gr.upload_slot(layers, {k: v for k, v in ghost.items() if k != "inject_w"})
    _, hk, hv, dk, dv, kc = DN_SHAPE
    kd, vd = hk * dk, hv * dv
    cd = 2 * kd + vd
    dnw = dict(qkv_q=codes(cd * d // 8), qkv_s=bf(cd * d // 64, 0.02), qkv_b=bf(cd * d // 64, 0.01),
               z_q=codes(vd * d // 8), z_s=bf(vd * d // 64, 0.02), z_b=bf(vd * d // 64, 0.01),
               a_w=bf(hv * d, 0.02), b_w=bf(hv * d, 0.02),
               out_q=codes(d * vd // 8), out_s=bf(d * vd // 64, 0.02), out_b=bf(d * vd // 64, 0.01),
               conv_w=bf(cd * kc, 0.5), norm_w=(1 + rng.normal(0, 0.1, dv)).astype(np.float32),
               a_log=rng.normal(0, 1, hv).astype(np.float32), dt_bias=rng.normal(0, 1, hv).astype(np.float32))
    dn = pkg.DeltaNetContext(d, hk, hv, dk, dv, kc, n_layers=layers, max_tokens=chunk)
    _, h, kvh, hd, ih, ihd, budget, comp = AT_SHAPE
    q4 = lambda rows, cols: (codes(rows * cols // 8), bf(rows * cols // 64, 0.02), bf(rows * cols // 64, 0.01))
    atw = {}
    for nm, (rows, cols) in (("q", (2 * h * hd, d)), ("k", (kvh * hd, d)), ("v", (kvh * hd, d)), ("o", (d, h * hd))):
        atw[nm + "_q"], atw[nm + "_s"], atw[nm + "_b"] = q4(rows, cols)
    atw["idx_w"] = bf((ih + 1) * ihd * d, 0.02)
    for nm, n in (("q_norm", hd), ("k_norm", hd), ("idx_q_norm", ihd), ("idx_k_norm", ihd)):
        atw[nm] = (1 + rng.normal(0, 0.1, n)).astype(np.float32)
    cap = context + warmup + tokens + chunk
    at = pkg.AttentionContext(d, h, kvh, hd, ih, ihd, budget, comp, kv_cap=cap, n_layers=layers,
                              max_tokens=chunk)
    xs = torch.randn((chunk, d), device="cuda") * 0.5
    for l, t in enumerate(types):
        if t == "dn":
            dn.upload_layer(l, dnw)
        else:
            at.upload_layer(l, atw)
            for t0 in range(0, context, chunk):
                at.forward(l, xs, t0)
    torch.cuda.synchronize()
    stack = pkg.DecoderStack(gr, moe, dn, at, types, 1)
    hyper = torch.empty((1, hcd), dtype=torch.float32, device="cuda")
    pkg.synth_fill(hyper, 1, 78, 0, pkg.TAGS["HYPER"], stddev=1.0)
    for i in range(warmup):
        stack.step(hyper, context + i)
    torch.cuda.synchronize()

    def run():
        for i in range(tokens):
            stack.step(hyper, context + warmup + i)
    g = capture(torch, run, warm=False)
    time_graph(torch, g, GRAPH_WARM_REPLAYS)
    sec = time_graph(torch, g, 1) / tokens
    ok = bool(torch.isfinite(stack.final).all().item())
    for c in (moe, gr, dn, at):
        c.close()
    if not ok:
        raise RuntimeError("decoder stack output is not finite")
    return sec


def bench_depth(pkg, torch, w, tokens, warmup):
    """48 stacked layers, one token: h <- h + MoE(RMSNorm(h)) layer after
    layer (f32 residual stream), captured as one graph per token; returns
    seconds per token"""
    L = w.n_layers
    ctx = pkg.MoeContext.for_workload(w, n_layers=L, max_tokens=1)
    for layer in range(L):
        rb = zipf_bias_host(w.n_experts, w.zipf_s, w.zipf_scale, w.seed * 1000003 + layer)
        ctx.synth_layer(layer, w.seed, with_norm=True, router_bias=rb)
    xs = []
    for i in range(tokens + warmup):
        t = torch.empty((1, w.hidden), dtype=torch.float32, device="cuda")
        pkg.synth_fill(t, 1, 7000 + i, 0, pkg.TAGS["X"], stddev=1.0)
        xs.append(t)
    h = [torch.empty((1, w.hidden), dtype=torch.float32, device="cuda") for _ in range(2)]
    torch.cuda.synchronize()

    def token(x):
        src = x
        for layer in range(L):
            dst = h[layer & 1]
            ctx.layer_forward(layer, src, out=dst, residual=True)
            src = dst

    for i in range(warmup):
        token(xs[i])
    torch.cuda.synchronize()
    g = capture(torch, lambda: [token(xs[i]) for i in range(warmup, warmup + tokens)],
                warm=warmup == 0)
    sec = time_graph(torch, g, 1)
    ctx.close()
    return sec / tokens


# ------------------------------------------------------------ CPU baseline

def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _timed_runs(make_fn, n_max, budget_s, runs=10, warm=3):
    """the median of `runs` timed runs after `warm` warm-ups; when
    runs + warm runs of n_max tokens would take longer than budget_s, the
    token sample shrinks to fit (never the run count).
    make_fn(n) -> fn(warmups, iters) returning the median seconds.  Returns
    (median, tokens per run, runs, warm-ups)."""
    n = n_max
    one = make_fn(n)(1, 1)  # a warm run: the first touches the weights
    per = budget_s / (runs + warm)
    if one > per and n > 1:
        n = max(1, int(n * per / one))
    return make_fn(n)(warm, runs), n, runs, warm


def cpu_baselines(pkg, names, threads, budget_s):
    """The oracle (the C restatement of the reference C port's path) on
    this host's cores, per workload, in both weight modes: (i) warm fp32
    experts (the steady state of the C port's expert cache, gemm_fp32 on
    dequantised weights) and (ii) q4-resident experts (gemm_q4 for every
    expert); all threads and one thread.  Layers are the workloads' seeded
    layers with only the routed experts generated (no other expert is
    touched).  Prefill runs on a token sample (stated); the 48-layer stack
    is q4 only (a warm fp32 cache of 48 layers does not fit host memory)."""
    import numpy as np
    sys.path.insert(0, ROOT)
    from oracle import oracle as orc
    res = {}
    for name in names:
        w = pkg.WORKLOADS[name]
        t0 = time.time()
        if name == "depth48":
            res[name] = cpu_depth(orc, w, threads, budget_s)
            log(f"cpu {name}: {res[name]['q4']['tokens_per_s_all']:.1f} tokens/s (q4, "
                f"{threads} threads) in {time.time() - t0:.1f}s")
            continue
        n_all = min(w.n_tokens, 256)
        n_one = min(w.n_tokens, 32)
        x = orc.gen_x(n_all, w.hidden, 4242, bf16=w.x_bf16)
        rb = (orc.zipf_bias(w.n_experts, w.zipf_s, w.zipf_scale, w.seed * 1000003)
              if w.zipf_s > 0 else None)
        Lr = orc.Layer(w.hidden, w.n_experts, w.top_k, w.moe_inter, seed=w.seed, router_bias=rb,
                       only_experts=[], group_size=w.group_size)
        ids = Lr.route(x, w.x_bf16)["idx"].reshape(-1)
        L = orc.Layer(w.hidden, w.n_experts, w.top_k, w.moe_inter, seed=w.seed, router_bias=rb,
                      only_experts=ids, group_size=w.group_size)
        warm = orc.Warm(L, ids, n_threads=threads)
        entry = dict(warm_fp32_bytes=warm.nbytes)
        for mode in ("warm_fp32", "q4"):
            row = {}
            for th, n_max in ((threads, n_all), (1, n_one)):
                def make_fn(n, th=th, mode=mode):
                    xs = np.ascontiguousarray(x[:n])
                    if mode == "warm_fp32":
                        return lambda wu, it: warm.time_forward(xs, w.x_bf16, th, wu, it)
                    return lambda wu, it: L.time_forward(xs, w.x_bf16, th, wu, it)
                med, n, iters, wu = _timed_runs(make_fn, n_max, budget_s)
                key = "all" if th > 1 else "1"
                row[f"tokens_per_s_{key}"] = n / med
                row[f"sample_tokens_{key}"] = n
                row[f"runs_{key}"] = iters
                row[f"warmups_{key}"] = wu
                if name == "prefill":
                    gemm, router = prefill_flops(w)
                    row[f"gflops_{key}"] = (gemm + router) / w.n_tokens * n / med / 1e9
                elif w.n_tokens <= 64:
                    row[f"gbs_{key}"] = layer_token_bytes(w) * n / med / 1e9 if n == 1 else None
            entry[mode] = row
        warm.close()
        res[name] = entry
        log(f"cpu {name}: warm fp32 {entry['warm_fp32']['tokens_per_s_all']:.1f} / q4 "
            f"{entry['q4']['tokens_per_s_all']:.1f} tokens/s ({threads} threads), "
            f"{entry['warm_fp32']['tokens_per_s_1']:.1f} / {entry['q4']['tokens_per_s_1']:.1f} "
            f"(1 thread) in {time.time() - t0:.1f}s")
    return res


def cpu_depth(orc, w, threads, budget_s, sample_layers=8):
    """one token through the stacked layers (RMSNorm + residual), q4
    experts: the first `sample_layers` layers of the stack run as a chain,
    their per-layer medians summed and scaled to the stack's depth (every
    layer has the same shape and routes the same number of experts)"""
    import numpy as np
    h = orc.gen_x(1, w.hidden, 4242, bf16=False)
    layers = []
    for layer in range(min(sample_layers, w.n_layers)):
        rb = orc.zipf_bias(w.n_experts, w.zipf_s, w.zipf_scale, w.seed * 1000003 + layer)
        Lr = orc.Layer(w.hidden, w.n_experts, w.top_k, w.moe_inter, seed=w.seed, layer=layer,
                       with_norm=True, router_bias=rb, only_experts=[])
        ids = Lr.route(h, False)["idx"].reshape(-1)
        L = orc.Layer(w.hidden, w.n_experts, w.top_k, w.moe_inter, seed=w.seed, layer=layer,
                      with_norm=True, router_bias=rb, only_experts=ids)
        layers.append((L, h))
        h = L.forward(h, False, residual=True, routed_mode=orc.ROUTED_Q4)["out"]
    out = {}
    per_layer = budget_s / len(layers)
    for th, key in ((threads, "all"), (1, "1")):
        tot = 0.0
        for L, hin in layers:
            med, _, _, _ = _timed_runs(lambda n, L=L, hin=hin: (lambda wu, it: L.time_forward(
                np.ascontiguousarray(hin), False, th, wu, it, residual=True)), 1, per_layer)
            tot += med
        tot *= w.n_layers / len(layers)
        out[f"tokens_per_s_{key}"] = 1.0 / tot
        out[f"gbs_{key}"] = layer_token_bytes(w) * w.n_layers / tot / 1e9
    return dict(q4=out, sample_tokens=1, sample_layers=len(layers),
                runs=10, warmups=3,
                note=f"one token through the first {len(layers)} of the {w.n_layers} layers as a "
                     f"chain, per-layer medians (10 runs after 3 warm-ups) summed and scaled to "
                     f"{w.n_layers} layers; only the routed experts of each layer generated")


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


def free(torch, *objs):
    for o in objs:
        if o is not None and hasattr(o, "ctx"):
            o.ctx.close()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=480)
    ap.add_argument("--warmup", type=int, default=48)
    ap.add_argument("--workload", default="decode")
    ap.add_argument("--layers", type=int, default=48,
                    help="resident layers rotated over (defeats the Infinity Cache)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=12.0,
                    help="at most this many seconds of CPU timing per (workload, mode, thread "
                         "count): past it the token sample shrinks, the 10 runs after 3 warm-ups stay")
    ap.add_argument("--cpu", default="tiny,decode,batched,prefill,depth48",
                    help="workloads timed on the CPU (the oracle)")
    ap.add_argument("--extra", default="tiny,batched,prefill,depth48",
                    help="comma list of other workloads to time (secondary results)")
    ap.add_argument("--deltanet", type=int, default=1,
                    help="also time the gated DeltaNet mixer at one token (0: skip)")
    ap.add_argument("--attention", type=int, default=1,
                    help=f"also time the full-attention mixer at one token, {AT_CONTEXT} cached (0: skip)")
    ap.add_argument("--hyper", default="decode,batched,prefill",
                    help="comma list of workloads also timed as hyper-connection layers "
                         f"(hc {HC_COUNT}, rank {HC_LOWRANK}; secondary results)")
    ap.add_argument("--stream-device", default="16,64", metavar="LAYERS,SLOTS",
                    help="decode with streamed experts, residency resolved on the GPU, graph "
                         "replay ('' to skip)")
    ap.add_argument("--stream", default="16,64,16", metavar="LAYERS,SLOTS,PREFETCH",
                    help="also time Zipf decode with streamed experts (pinned host store, SLOTS "
                         "of 512 HBM expert slots per layer); empty: skip")
    ap.add_argument("--stack", type=int, default=1,
                    help=f"also time one token through the {STACK_LAYERS}-layer decoder stack "
                         f"(DeltaNet : attention 3 : 1, hyper connections, final mixer; 0: skip)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 8 plain copies of MIB MiB (counter calibration) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              f"(the MoE layer runs on a single MI355X here)", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        print("--steps must be >= 1 and --warmup >= 0", file=sys.stderr)
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

    sec_step, st = bench_layer(pkg, torch, w, n_layers, args.steps, args.warmup)
    log(f"{w.name}: {sec_step * 1e6:.2f} us/step over {args.steps} steps "
        f"(+{args.warmup} warm-up), {n_layers} layers")
    roof = None
    if w.n_tokens == 1 and w.x_bf16 and not w.rms_norm:
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
    layer_bytes = layer_token_bytes(w)
    free(torch, st)
    del st

    extra = {}
    for name in [e for e in args.extra.split(",") if e and e != w.name]:
        we = pkg.WORKLOADS[name]
        if name == "depth48":
            s_t = bench_depth(pkg, torch, we, tokens=20, warmup=3)
            b = layer_token_bytes(we) * we.n_layers
            extra[name] = dict(us_per_token=s_t * 1e6, tokens_per_s=1.0 / s_t, layers=we.n_layers,
                               tokens=20, algorithmic_bytes_per_token=b,
                               hbm_fraction=round(b / s_t / 1e9 / HBM_PEAK_GBS, 4),
                               note="one f32 token through 48 stacked layers (RMSNorm, Zipf "
                                    "routing, residual), one HIP graph per 20 tokens")
            log(f"{name}: {s_t * 1e6:.1f} us/token -> {b / s_t / 1e9:.0f} GB/s")
            torch.cuda.empty_cache()
            continue
        nl = 1 if we.n_tokens <= 4 else (8 if we.n_tokens <= 64 else 2)
        steps_e = 64 if we.n_tokens <= 64 else 16
        s_e, st = bench_layer(pkg, torch, we, nl, steps_e, nl * 2, n_inputs=nl * 4)
        ent = dict(tokens_per_s=we.n_tokens / s_e, ms_per_step=s_e * 1e3,
                   tokens_per_step=we.n_tokens, layers_rotated=nl, steps=steps_e)
        if name == "batched":
            us = distinct_experts(st, nl * 4)
            b = sum(step_bytes_batched(we, u) for u in us) / len(us)
            ent.update(mean_distinct_experts=sum(us) / len(us), algorithmic_bytes_per_step=int(b),
                       hbm_fraction=round(b / s_e / 1e9 / HBM_PEAK_GBS, 4))
        if name == "prefill":
            t_gu, t_dn = bench_prefill_stages(pkg, torch, st)
            gemm, router = prefill_flops(we)
            ent.update(gateup_stage_us=t_gu * 1e6, down_stage_us=t_dn * 1e6,
                       grouped_gemm_flops=gemm,
                       grouped_gemm_mfma_fraction=round(gemm / (t_gu + t_dn) / 1e12 / BF16_PEAK_TFLOPS, 4),
                       layer_flops=gemm + router,
                       layer_mfma_fraction=round((gemm + router) / s_e / 1e12 / BF16_PEAK_TFLOPS, 4))
            log(f"prefill stages: gate/up {t_gu * 1e6:.1f} us, down {t_dn * 1e6:.1f} us -> "
                f"{gemm / (t_gu + t_dn) / 1e12:.0f} TFLOP/s")
        extra[name] = ent
        log(f"{name}: {s_e * 1e3:.4f} ms/step -> {we.n_tokens / s_e:.0f} tokens/s")
        free(torch, st)
        del st
    if args.stack:
        ws = pkg.WORKLOADS["decode"]
        s_s = bench_stack(pkg, torch, ws, 20, 4)
        b = stack_token_bytes(ws, STACK_LAYERS, STACK_CONTEXT)
        extra["decoder_stack"] = dict(
            us_per_token=s_s * 1e6, tokens_per_s=1.0 / s_s, layers=STACK_LAYERS,
            deltanet_layers=sum(1 for l in range(STACK_LAYERS) if (l + 1) % 4),
            attention_context=STACK_CONTEXT, tokens=20, algorithmic_bytes_per_token=b,
            hbm_fraction=round(b / s_s / 1e9 / HBM_PEAK_GBS, 4),
            note="one f32 hyper-state token through 48 decoder layers (attention-block hyper "
                 "connection, gated DeltaNet or QSA attention at 3 : 1, inject, MLP hyper connection "
                 "+ MoE layer + inject) and the final mixer, 20 tokens in one HIP graph")
        log(f"decoder stack: {s_s * 1e6:.1f} us/token -> {b / s_s / 1e9:.0f} GB/s")
        torch.cuda.empty_cache()
    if args.deltanet:
        nl = 16
        s_d = bench_deltanet(pkg, torch, nl, 256, 32)
        b = dn_token_bytes(DN_SHAPE)
        extra["deltanet"] = dict(
            us_per_token=s_d * 1e6, tokens_per_s=1.0 / s_d, layers_rotated=nl, steps=256,
            algorithmic_bytes_per_token=b, hbm_fraction=round(b / s_d / 1e9 / HBM_PEAK_GBS, 4),
            shape=dict(zip(("hidden", "key_heads", "value_heads", "k_head_dim", "v_head_dim",
                            "conv_kernel"), DN_SHAPE)),
            note="one f32 token through one gated DeltaNet mixer (projections, conv + delta-rule "
                 "recurrence with HBM-resident states, gated norm + out_proj), layers rotated, "
                 "one HIP graph")
        log(f"deltanet: {s_d * 1e6:.2f} us/token-layer -> {b / s_d / 1e9:.0f} GB/s")
        torch.cuda.empty_cache()
    if args.attention:
        nl = 16
        s_a = bench_attention(pkg, torch, nl, 256, 32)
        b = at_token_bytes(AT_SHAPE, AT_CONTEXT)
        extra["attention"] = dict(
            us_per_token=s_a * 1e6, tokens_per_s=1.0 / s_a, layers_rotated=nl, steps=256,
            context=AT_CONTEXT, algorithmic_bytes_per_token=b,
            hbm_fraction=round(b / s_a / 1e9 / HBM_PEAK_GBS, 4),
            shape=dict(zip(("hidden", "heads", "kv_heads", "head_dim", "idx_heads", "idx_head_dim",
                            "idx_budget", "idx_compress"), AT_SHAPE)),
            note="one f32 token through one full-attention mixer (q4 projections, per-head norm + "
                 "partial RoPE, indexer block selection, masked softmax over the cache, gate, "
                 "o_proj) at 4096 cached tokens, layers rotated, one HIP graph")
        log(f"attention: {s_a * 1e6:.2f} us/token-layer at {AT_CONTEXT} cached -> "
            f"{b / s_a / 1e9:.0f} GB/s")
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
        threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
        names = [c for c in args.cpu.split(",") if c]
        if w.name not in names:
            names.insert(0, w.name)
        per = cpu_baselines(pkg, names, threads, args.cpu_budget)
        head = per[w.name]
        mode = "warm_fp32" if "warm_fp32" in head else "q4"
        cpu = dict(value=round(head[mode]["tokens_per_s_all"], 2), unit="tokens/s", cores=threads,
                   kind="port", value_1thread=round(head[mode]["tokens_per_s_1"], 2),
                   cpu_model=cpu_model(),
                   sample=f"the {w.name} workload through oracle/moe_oracle.c (the C restatement of "
                          f"the reference C port's moe_forward) with warm fp32-dequantised routed "
                          f"experts (weight mode i, gemm_fp32), median of 10 runs after 3 warm-ups "
                          f"(the token sample per run shrunk to fit {args.cpu_budget:.0f} s, as "
                          f"per_config's sample_tokens_* give); {threads} OpenMP threads "
                          f"(value_1thread: 1 thread); per_config holds every workload in both weight "
                          f"modes (q4: gemm_q4 for every expert)",
                   per_config=per)
        log(f"cpu baseline: {cpu['value']:.1f} tokens/s with {threads} threads "
            f"({cpu['cpu_model']}), {cpu['value_1thread']:.1f} with 1")

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
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
            "timing": f"{args.warmup} eager warm-up steps, then the {args.steps} timed steps as one HIP "
                      f"graph: replayed {GRAPH_WARM_REPLAYS}x untimed (one-time graph launch set-up), "
                      f"then one timed replay between HIP events",
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
