"""Expert streaming on the GPU (qmoe_stream_enable): routed experts in pinned
host memory, a few HBM slots per layer, the reference's cache policy
(c/src/cache.c) and route-transition prefetch (streaming.py:400-435).

Bar: the streamed layer runs the same kernels on the same weights, so its
outputs are bit-identical to the resident layer's on every call, whatever
the cache did (misses, evictions, prefetches); routing is unchanged; the
counters add up (every routed expert is a hit or a miss)."""
import numpy as np
import pytest

from ckpt_util import write_moe_layer
from conftest import load_oracle, load_pkg

orc = load_oracle()

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def torch_dev(gpu):
    import torch
    return torch, gpu


def _pair(pkg, H, E, k, I, L, max_tokens, slots, policy, prefetch, seed, zipf=0.0):
    """a resident and a streamed context holding the same synthetic layers"""
    res = pkg.MoeContext(H, E, k, I, n_layers=L, max_tokens=max_tokens)
    stm = pkg.MoeContext(H, E, k, I, n_layers=L, max_tokens=max_tokens)
    stm.stream_enable(slots, policy, prefetch)
    for layer in range(L):
        rb = orc.zipf_bias(E, zipf, 1.0, seed * 1000003 + layer) if zipf else None
        res.synth_layer(layer, seed, router_bias=rb)
        stm.synth_layer(layer, seed, router_bias=rb)
    return res, stm


def _run_sequence(torch, dev, res, stm, L, steps, n, H, bf16, seed, us=None):
    routed = 0
    for step in range(steps):
        x = orc.gen_x(n, H, seed + step, bf16=bf16)
        xt = (torch.from_numpy(x.view(np.int16)).to(dev).view(torch.bfloat16) if bf16
              else torch.from_numpy(x).to(dev))
        for layer in range(L):
            a = res.layer_forward(layer, xt)
            b = stm.layer_forward(layer, xt)
            torch.cuda.synchronize()
            ra, rb = res.last_routing(n), stm.last_routing(n)
            assert np.array_equal(ra["idx"].cpu().numpy(), rb["idx"].cpu().numpy())
            sa, sb = ra["segments"].cpu().numpy(), rb["segments"].cpu().numpy()
            u = int(sa[0])  # entries past the count are not written by the call
            assert np.array_equal(sa[:1 + 3 * u], sb[:1 + 3 * u])
            routed += u
            if us is not None:
                us.append(u)
            assert np.array_equal(a.cpu().numpy(), b.cpu().numpy()), (step, layer)
    return routed


@pytest.mark.parametrize("policy", [0, 1, 2])
def test_tiny_streamed_bit_identical(torch_dev, policy):
    torch, dev = torch_dev
    pkg = load_pkg()
    say(f"case: tiny layers streamed, 4 slots of 8 experts, policy {policy}, prefetch 2")
    res, stm = _pair(pkg, 256, 8, 2, 128, 3, 2, 4, policy, 2, seed=5)
    routed = _run_sequence(torch, dev, res, stm, 3, 12, 2, 256, False, seed=40)
    st = stm.stream_stats()
    say(f"stats {st}")
    assert st["hits"] + st["misses"] == routed
    assert st["misses"] > 0 and st["evictions"] > 0 and st["rejected"] == 0
    expert_bytes = 3 * (128 * 256 // 2 + 128 * (256 // 64) * 4)
    assert st["bytes_in"] == (st["misses"] + st["prefetched"]) * expert_bytes
    res.close()
    stm.close()


def test_decode_shape_streamed_with_prefetch(torch_dev):
    torch, dev = torch_dev
    pkg = load_pkg()
    say("case: decode-shape layers (E 512, top-10) streamed, 32 slots per layer, prefetch 16, Zipf routing")
    res, stm = _pair(pkg, 2048, 512, 10, 512, 3, 1, 32, 2, 16, seed=3, zipf=1.1)
    routed = _run_sequence(torch, dev, res, stm, 3, 10, 1, 2048, True, seed=90)
    st = stm.stream_stats()
    say(f"stats {st}")
    assert st["hits"] + st["misses"] == routed
    assert st["prefetched"] > 0 and st["hits"] > 0
    assert st["bytes_in"] == (st["misses"] + st["prefetched"]) * 1769472
    res.close()
    stm.close()


@pytest.mark.parametrize("prefetch,n", [(4, 1), (0, 70), (-1, 70)])
def test_odd_shape_streamed(torch_dev, prefetch, n):
    """hidden 768, 60 experts top-6, intermediate 320: streamed layers (host-
    and device-resolved) equal the resident ones bit for bit: one token with
    12 slots (evicting), and 70 tokens on the MFMA path with every expert's
    slot"""
    torch, dev = torch_dev
    pkg = load_pkg()
    slots = 12 if n == 1 else 60
    say(f"case: odd shape streamed, {slots} slots of 60 experts, prefetch {prefetch}, n={n}")
    res, stm = _pair(pkg, 768, 60, 6, 320, 2, n, slots, 2, prefetch, seed=8, zipf=1.1)
    _run_sequence(torch, dev, res, stm, 2, 6, n, 768, n == 1, seed=70)
    st = stm.stream_stats()
    say(f"stats {st}")
    assert st["hits"] + st["misses"] > 0
    res.close()
    stm.close()


@pytest.mark.parametrize("prefetch", [0, -1])
def test_batched_streamed_mfma_path(torch_dev, prefetch):
    """64 tokens route to up to 512 experts: every slot in use, segments
    remapped to slots on the MFMA path (host- and device-resolved)"""
    torch, dev = torch_dev
    pkg = load_pkg()
    say(f"case: decode-shape layer, 64 tokens, 512 slots (MFMA path over remapped segments), prefetch {prefetch}")
    res, stm = _pair(pkg, 2048, 512, 10, 512, 1, 64, 512, 0, prefetch, seed=8, zipf=1.1)
    _run_sequence(torch, dev, res, stm, 1, 3, 64, 2048, True, seed=7)
    res.close()
    stm.close()


@pytest.mark.parametrize("prefetch", [0, -1])
def test_streamed_checkpoint_and_hyper(torch_dev, tmp_path, prefetch):
    """a streamed context loaded from a checkpoint, run inside the hyper
    connection, equals the resident one (host- and device-resolved)"""
    torch, dev = torch_dev
    pkg = load_pkg()
    say(f"case: streamed tiny layer from a checkpoint, inside its hyper connection, prefetch {prefetch}")
    H, E, k, I = 256, 8, 2, 128
    L = orc.Layer(H, E, k, I, seed=2)
    write_moe_layer(str(tmp_path), L.arrays(), H, E, I, layer=0)
    hp = orc.Hyper(4, H, 128, seed=2)
    hyper = orc.gen_hyper(3, 4, H, seed=3)
    outs = []
    with pkg.Checkpoint(str(tmp_path)) as ck:
        for streamed in (False, True):
            with pkg.MoeContext(H, E, k, I, max_tokens=3) as ctx:
                if streamed:
                    ctx.stream_enable(6, 2, prefetch)
                ctx.upload_layer_st(0, ck, 0)
                ctx.hc_enable(4, 128)
                ctx.hc_upload_layer(0, hp.arrays())
                h = torch.from_numpy(hyper).to(dev)
                for _ in range(3):
                    ctx.hc_layer_forward(0, h, want_out=False)
                torch.cuda.synchronize()
                outs.append(h.cpu().numpy())
    assert np.array_equal(outs[0], outs[1])


def test_stream_errors(torch_dev):
    torch, dev = torch_dev
    pkg = load_pkg()
    say("case: expert streaming argument errors")
    with pkg.MoeContext(256, 8, 2, 128, max_tokens=2) as ctx:
        for slots, needle in ((3, "must be in [4, 8]"), (9, "must be in [4, 8]")):
            with pytest.raises(pkg.QmoeError, match=needle.replace("[", r"\[").replace("]", r"\]")):
                ctx.stream_enable(slots)
        with pytest.raises(pkg.QmoeError, match="not enabled"):
            ctx.stream_stats()
        ctx.stream_enable(4)
        ctx.stream_enable(4)  # same values: no-op
        ctx.synth_layer(0, 1)
        x = torch.zeros((1, 256), dtype=torch.float32, device=dev)
        with pytest.raises(pkg.QmoeError, match="not available with streamed experts"):
            ctx.expert_ffn(0, x, ctx.dispatch(ctx.router(0, x)["idx"]))
    with pkg.MoeContext(256, 8, 2, 128, max_tokens=2) as ctx:
        ctx.synth_layer(0, 1)
        with pytest.raises(pkg.QmoeError, match="must precede every layer upload"):
            ctx.stream_enable(4)


@pytest.mark.parametrize("policy", [0, 1, 2])
def test_device_resolved_matches_host_policy(torch_dev, policy):
    """prefetch -1: residency decided on the GPU.  Outputs bit-identical to
    the resident layer, and the hit/miss/eviction counts equal the host
    cache's (prefetch 0) on the same call sequence, which holds only if
    every victim is the one the host policy picks"""
    torch, dev = torch_dev
    pkg = load_pkg()
    say(f"case: tiny layers, device-resolved vs host-resolved residency, policy {policy}")
    res, dvc = _pair(pkg, 256, 8, 2, 128, 3, 2, 4, policy, -1, seed=5)
    routed = _run_sequence(torch, dev, res, dvc, 3, 12, 2, 256, False, seed=40)
    res.close()
    res, hst = _pair(pkg, 256, 8, 2, 128, 3, 2, 4, policy, 0, seed=5)
    _run_sequence(torch, dev, res, hst, 3, 12, 2, 256, False, seed=40)
    a, b = dvc.stream_stats(), hst.stream_stats()
    say(f"device {a} host {b}")
    assert a["hits"] + a["misses"] == routed
    for f in ("hits", "misses", "evictions", "rejected", "bytes_in"):
        assert a[f] == b[f], f
    assert a["evictions"] > 0 and a["prefetched"] == 0
    for c in (res, dvc, hst):
        c.close()


def test_device_resolved_decode_zipf(torch_dev):
    torch, dev = torch_dev
    pkg = load_pkg()
    say("case: decode-shape layers (E 512, top-10), 16 slots, device-resolved, Zipf routing")
    stats = []
    for prefetch in (-1, 0):
        res, stm = _pair(pkg, 2048, 512, 10, 512, 2, 1, 16, 2, prefetch, seed=3, zipf=1.1)
        _run_sequence(torch, dev, res, stm, 2, 12, 1, 2048, True, seed=90)
        stats.append(stm.stream_stats())
        res.close()
        stm.close()
    say(f"device {stats[0]} host {stats[1]}")
    for f in ("hits", "misses", "evictions", "rejected", "bytes_in"):
        assert stats[0][f] == stats[1][f], f


def test_device_resolved_graph_replay(torch_dev):
    """the device-resolved layer call captured once and replayed: each
    replay equals an eager resident call on the same input, while the
    residency state keeps changing inside the graph"""
    torch, dev = torch_dev
    pkg = load_pkg()
    say("case: device-resolved streamed layer captured in a graph, 6 replays")
    H, E, k, I, L = 256, 8, 2, 128, 2
    res, stm = _pair(pkg, H, E, k, I, L, 2, 4, 2, -1, seed=6)
    xs = [torch.from_numpy(orc.gen_x(2, H, 70 + i, bf16=False)).to(dev) for i in range(6)]
    x = xs[0].clone()
    outs = [torch.zeros((2, H), dtype=torch.float32, device=dev) for _ in range(L)]
    for layer in range(L):  # warm the slots eagerly once
        stm.layer_forward(layer, x, out=outs[layer])
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for layer in range(L):
            stm.layer_forward(layer, x, out=outs[layer])
    for i, xi in enumerate(xs):
        x.copy_(xi)
        g.replay()
        torch.cuda.synchronize()
        for layer in range(L):
            want = res.layer_forward(layer, xi)
            torch.cuda.synchronize()
            assert np.array_equal(outs[layer].cpu().numpy(), want.cpu().numpy()), (i, layer)
    st = stm.stream_stats()
    say(f"stats {st}")
    assert st["misses"] > 0 and st["rejected"] == 0
    res.close()
    stm.close()


def test_device_resolved_many_experts_evicting(torch_dev):
    """more than 256 routed experts in one call (the resolve kernel takes the
    hits before each miss in passes of 256 threads) while the slots still
    evict: device-resolved and host-resolved residency give the same counts,
    and both give the resident layer's bits"""
    torch, dev = torch_dev
    pkg = load_pkg()
    H, E, k, I, n, slots = 128, 1024, 10, 64, 32, 320
    say(f"case: E={E} top-{k}, {n} tokens per call, {slots} slots, device vs host residency")
    stats, routed, us = [], [], []
    for prefetch in (-1, 0):
        res, stm = _pair(pkg, H, E, k, I, 1, n, slots, 2, prefetch, seed=12)
        routed.append(_run_sequence(torch, dev, res, stm, 1, 6, n, H, False, seed=300, us=us))
        stats.append(stm.stream_stats())
        res.close()
        stm.close()
    say(f"device {stats[0]} host {stats[1]} routed {routed}")
    assert routed[0] == routed[1] and max(us) > 256
    for f in ("hits", "misses", "evictions", "rejected", "bytes_in"):
        assert stats[0][f] == stats[1][f], f
    assert stats[0]["evictions"] > 0 and stats[0]["hits"] > 0


def test_reupload_after_prefetch(torch_dev):
    """a layer re-uploaded right after a call that queued prefetch copies:
    the upload waits for the copies, the layer forgets its slots, and the
    next call gives the new weights' bits"""
    torch, dev = torch_dev
    pkg = load_pkg()
    H, E, k, I, L = 256, 8, 2, 128, 2
    say("case: re-upload of a streamed layer with prefetch copies in flight")
    res, stm = _pair(pkg, H, E, k, I, L, 2, 4, 2, 4, seed=21)
    xs = [torch.from_numpy(orc.gen_x(2, H, 500 + i, bf16=False)).to(dev) for i in range(4)]
    for x in xs:
        for layer in range(L):
            stm.layer_forward(layer, x)
    # no synchronisation: the last calls' prefetches may still be queued
    stm.synth_layer(0, 99)
    res.synth_layer(0, 99)
    for i, x in enumerate(xs):
        for layer in range(L):
            a = res.layer_forward(layer, x)
            b = stm.layer_forward(layer, x)
            torch.cuda.synchronize()
            assert np.array_equal(a.cpu().numpy(), b.cpu().numpy()), (i, layer)
    st = stm.stream_stats()
    say(f"stats {st}")
    assert st["prefetched"] > 0
    res.close()
    stm.close()
