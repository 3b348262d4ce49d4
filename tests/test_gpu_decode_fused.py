"""The one-token layer in one launch (router, shared and routed gate/up,
down and combine, with the logits and h handed over inside the launch
through tagged words) against the staged kernels on the same context:
outputs, hyper state and routing bit-identical.  The staged kernels (the default) are pinned to the oracle
by the parity tests.
Every case ends with qmoe_decode_status: no wait may have given up."""
import numpy as np
import pytest

from conftest import load_oracle, load_pkg

orc = load_oracle()

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def torch_dev(gpu):
    import torch
    return torch, gpu


def _routing(ctx):
    r = ctx.last_routing(1)
    return {k: v.cpu().numpy() for k, v in r.items() if k != "offsets"}


def _both(ctx, torch, fn):
    """fn() under the staged kernels, then under the one-launch path"""
    ctx.set_fused_decode(False)
    a = fn()
    torch.cuda.synchronize()
    ra = _routing(ctx)
    ctx.set_fused_decode(True)
    b = fn()
    torch.cuda.synchronize()
    rb = _routing(ctx)
    return a, b, ra, rb


def _assert_same(a, b, ra, rb, what):
    for t_a, t_b in zip(a, b):
        if t_a is None:
            continue
        ga, gb = t_a.cpu().numpy(), t_b.cpu().numpy()
        assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32)), \
            (what, int((ga != gb).sum()), float(np.abs(ga - gb).max()))
    for k in ("idx", "w", "shared_gate", "perm"):
        assert np.array_equal(ra[k], rb[k]), (what, k, ra[k], rb[k])
    U = int(ra["segments"][0])
    assert np.array_equal(ra["segments"][:1 + 3 * U], rb["segments"][:1 + 3 * U]), what


SHAPES = [
    # H, E, k, I: the decode workload, then the other template instances
    # (experts per lane 2, 4, 16; two chunks per lane at hidden 4096)
    (2048, 512, 10, 512),
    (2048, 128, 4, 512),
    (2048, 1024, 11, 512),
    (4096, 256, 6, 512),
    (4096, 64, 2, 512),
]


@pytest.mark.parametrize("H,E,k,I", SHAPES)
def test_one_launch_matches_staged(torch_dev, H, E, k, I):
    torch, dev = torch_dev
    pkg = load_pkg()
    say(f"case: one-launch vs staged one-token layer H={H} E={E} k={k} I={I}")
    rb = orc.zipf_bias(E, 1.1, 1.0, 77)
    with pkg.MoeContext(H, E, k, I, n_layers=2, max_tokens=1) as ctx:
        ctx.synth_layer(0, 3)
        ctx.synth_layer(1, 4, with_norm=True, router_bias=rb)
        for seed in range(6):
            layer = seed & 1
            bf16 = seed % 3 != 2
            residual = seed % 4 >= 2
            xh = orc.gen_x(1, H, 100 + seed, bf16=bf16)
            if bf16:
                x = torch.from_numpy(xh.view(np.int16)).to(dev).view(torch.bfloat16)
            else:
                x = torch.from_numpy(xh).to(dev)
            a, b, ra, rb_ = _both(ctx, torch,
                                  lambda: (ctx.layer_forward(layer, x, residual=residual),))
            _assert_same(a, b, ra, rb_, (H, E, k, I, seed))
            assert np.isfinite(a[0].cpu().numpy()).all()
        assert ctx.decode_status() == 0


def test_one_launch_refused_for_other_shapes(torch_dev):
    pkg = load_pkg()
    with pkg.MoeContext(256, 8, 2, 128, max_tokens=1) as ctx:
        ctx.set_fused_decode(False)
        with pytest.raises(pkg.QmoeError, match="does not take this shape"):
            ctx.set_fused_decode(True)
        assert ctx.decode_status() == 0


def test_one_launch_hyper(torch_dev):
    """the hyper connection's one-token layer: MoE output and the updated
    hyper state bit-identical"""
    torch, dev = torch_dev
    pkg = load_pkg()
    H, E, k, I, hc, R = 2048, 512, 10, 512, 4, 320
    say("case: one-launch vs staged, hyper connection (hc 4, R 320)")
    with pkg.MoeContext(H, E, k, I, n_layers=1, max_tokens=1) as ctx:
        ctx.synth_layer(0, 5, with_norm=False)
        ctx.hc_enable(hc, R)
        ctx.hc_synth_layer(0, 5)
        g = torch.Generator().manual_seed(9)
        for it in range(3):
            h0 = torch.randn((1, hc * H), generator=g).to(dev)

            def run():
                hy = h0.clone()
                out = ctx.hc_layer_forward(0, hy)
                return out, hy
            a, b, ra, rb = _both(ctx, torch, run)
            _assert_same(a, b, ra, rb, ("hyper", it))
        assert ctx.decode_status() == 0


def test_one_launch_long_chain_and_graph(torch_dev):
    """48 layers chained (the hand-off state is reused call after call),
    eager and as one captured HIP graph replayed three times: every replay
    equals the staged chain"""
    torch, dev = torch_dev
    pkg = load_pkg()
    w = pkg.WORKLOADS["depth48"]
    nl = 48
    say("case: 48-layer one-token chain, one-launch vs staged, eager and graph")
    with pkg.MoeContext.for_workload(w, n_layers=nl) as ctx:
        for layer in range(nl):
            rb = orc.zipf_bias(w.n_experts, w.zipf_s, w.zipf_scale, w.seed * 1000003 + layer)
            ctx.synth_layer(layer, w.seed, with_norm=True, router_bias=rb)
        h0 = torch.from_numpy(orc.gen_x(1, w.hidden, 5, bf16=False)).to(dev)
        bufs = [torch.empty_like(h0) for _ in range(2)]

        def chain():
            h = h0
            for layer in range(nl):
                o = bufs[layer & 1]
                ctx.layer_forward(layer, h, out=o, residual=True)
                h = o
            return h

        ctx.set_fused_decode(False)
        ref = chain().clone()
        torch.cuda.synchronize()
        ctx.set_fused_decode(True)
        got = chain().clone()
        torch.cuda.synchronize()
        assert torch.equal(ref, got)
        assert ctx.decode_status() == 0

        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            chain()  # warm-up on the capture stream
            torch.cuda.synchronize()
            with torch.cuda.graph(graph, stream=s):
                res = chain()
        torch.cuda.synchronize()
        for rep in range(3):
            bufs[0].fill_(0.0)
            bufs[1].fill_(0.0)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(res, ref), rep
        assert ctx.decode_status() == 0
        say("48-layer chain: one-launch == staged, eager and 3 graph replays")
