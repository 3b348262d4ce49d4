"""The HIP gated DeltaNet mixer (qmoe_dn_*, through the C ABI) against the
oracle (oracle/dn_oracle.c, pinned by tests/test_oracle_dn.py).

Bar: per call, outputs within 2e-2 max-abs and 1e-3 relative L2 of the
oracle run on the same weights and inputs from the same states; the conv
and recurrent states after each call within 1e-4 relative L2.  One call
over n tokens equals n one-token calls bit for bit.
"""
import ctypes

import numpy as np
import pytest

from conftest import load_oracle, load_pkg

orc = load_oracle()

pytestmark = pytest.mark.gpu

MAX_ABS, REL_L2 = 2e-2, 1e-3


def say(msg):
    print(msg, flush=True)


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


_hip = None


def hip():
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
    return _hip


def d2h(ptr, shape):
    buf = np.empty(shape, np.float32)
    assert hip().hipMemcpy(ctypes.c_void_p(buf.ctypes.data), ctypes.c_void_p(ptr),
                           ctypes.c_size_t(buf.nbytes), 2) == 0
    return buf


def h2d(ptr, arr):
    arr = np.ascontiguousarray(arr, np.float32)
    assert hip().hipMemcpy(ctypes.c_void_p(ptr), ctypes.c_void_p(arr.ctypes.data),
                           ctypes.c_size_t(arr.nbytes), 1) == 0


@pytest.fixture(scope="module")
def torch_dev(gpu):
    import torch
    return torch, gpu


def read_states(ctx, layer):
    cp, rp = ctx.state_ptrs(layer)
    cshape, rshape = ctx.state_shapes()
    conv = d2h(cp, cshape) if cshape[0] > 0 else np.zeros(cshape, np.float32)
    return conv, d2h(rp, rshape)


def run_steps(torch, dev, shape, calls, seed=1, seed_state=False):
    """calls: token counts of the successive calls; every call compared"""
    d, hk, hv, dk, dv, kc = shape
    pkg = load_pkg()
    D = orc.DeltaNet(d, hk, hv, dk, dv, kc, seed=seed)
    cs, rs = D.new_state()
    ntot = sum(calls)
    x = orc.gen_dn_x(ntot, d, seed + 100)
    with pkg.DeltaNetContext(d, hk, hv, dk, dv, kc, n_layers=2, max_tokens=max(calls)) as ctx:
        ctx.upload_layer(1, D.arrays())
        if seed_state:
            rng = np.random.default_rng(seed)
            cs[:] = rng.normal(0, 2.0, cs.shape)
            rs[:] = rng.normal(0, 0.3, rs.shape)
            cp, rp = ctx.state_ptrs(1)
            if cs.size:
                h2d(cp, cs)
            h2d(rp, rs)
        t0 = 0
        for i, n in enumerate(calls):
            xi = x[t0:t0 + n]
            ref = D.forward(xi, cs, rs)
            got = ctx.forward(1, torch.from_numpy(xi).to(dev))
            torch.cuda.synchronize()
            g = got.cpu().numpy()
            err, r = float(np.abs(g - ref).max()), rel(g, ref)
            gc, gr = read_states(ctx, 1)
            rc, rr = rel(gc, cs) if cs.size else 0.0, rel(gr, rs)
            say(f"{shape} call {i} (n={n}): out max-abs {err:.2e} rel-L2 {r:.2e} "
                f"(|ref| max {np.abs(ref).max():.2f}); states rel {rc:.1e} / {rr:.1e}")
            assert err < MAX_ABS and r < REL_L2, (i, err, r)
            assert rc < 1e-4 and rr < 1e-4, (i, rc, rr)
            t0 += n


def test_tiny_decode_steps(torch_dev):
    torch, dev = torch_dev
    say("case: DeltaNet tiny (d 256, heads 2/4, dk 64, dv 64, conv 4), 6 one-token calls")
    run_steps(torch, dev, (256, 2, 4, 64, 64, 4), [1] * 6)


def test_model_shape_decode_and_chunk(torch_dev):
    """hidden 2048, 16 key / 32 value heads of 128, conv 4 (the Qwen3-Next
    family's linear-attention shape): three one-token calls, then 5 tokens
    in one call, then one more token"""
    torch, dev = torch_dev
    say("case: DeltaNet d 2048, heads 16/32, dk 128, dv 128, conv 4")
    run_steps(torch, dev, (2048, 16, 32, 128, 128, 4), [1, 1, 1, 5, 1], seed=2)


@pytest.mark.parametrize("shape", [(128, 1, 2, 32, 128, 3), (4096, 4, 8, 256, 64, 2),
                                   (512, 2, 2, 64, 128, 1), (1024, 8, 64, 128, 128, 4)])
def test_other_shapes_seeded_state(torch_dev, shape):
    torch, dev = torch_dev
    say(f"case: DeltaNet shape {shape}, seeded states")
    run_steps(torch, dev, shape, [1, 3, 1], seed=3, seed_state=True)


@pytest.mark.parametrize("shape", [(320, 1, 2, 32, 32, 7), (448, 3, 6, 64, 256, 5),
                                   (1536, 2, 4, 256, 512, 16), (640, 5, 5, 128, 1024, 2)])
def test_irregular_shapes(torch_dev, shape):
    """valid shapes off the usual ones: hidden 320 / 448 / 640 / 1536, odd
    head counts, value heads 1x to 2x the key heads, value dims 32 to 1024,
    conv kernels 2 to 16; one-token calls and chunks of 2, 9 and 17"""
    torch, dev = torch_dev
    say(f"case: DeltaNet irregular shape {shape}")
    run_steps(torch, dev, shape, [1, 2, 1, 9, 1, 17, 1], seed=5)


def test_tokens_at_once_equal_one_by_one(torch_dev):
    torch, dev = torch_dev
    pkg = load_pkg()
    shape = (2048, 16, 32, 128, 128, 4)
    say("case: DeltaNet 4 tokens in one call == 4 one-token calls (bit for bit)")
    D = orc.DeltaNet(*shape, seed=4)
    x = torch.from_numpy(orc.gen_dn_x(4, shape[0], 9)).to(dev)
    with pkg.DeltaNetContext(*shape, n_layers=1, max_tokens=4) as ctx:
        ctx.upload_layer(0, D.arrays())
        a = ctx.forward(0, x).clone()
        sa = read_states(ctx, 0)
        ctx.reset_state(0)
        b = torch.cat([ctx.forward(0, x[t:t + 1]).clone() for t in range(4)])
        torch.cuda.synchronize()
        sb = read_states(ctx, 0)
        assert torch.equal(a, b)
        np.testing.assert_array_equal(sa[0], sb[0])
        np.testing.assert_array_equal(sa[1], sb[1])


def test_graph_replay_and_reset(torch_dev):
    """a captured graph of reset + 3 one-token calls, replayed: every replay
    gives the eager outputs (the state fill is a kernel, not a memset)"""
    torch, dev = torch_dev
    pkg = load_pkg()
    shape = (256, 2, 4, 64, 64, 4)
    say("case: DeltaNet graph replay with state reset inside the graph")
    D = orc.DeltaNet(*shape, seed=6)
    x = torch.from_numpy(orc.gen_dn_x(3, shape[0], 2)).to(dev)
    with pkg.DeltaNetContext(*shape, n_layers=1, max_tokens=1) as ctx:
        ctx.upload_layer(0, D.arrays())
        outs = [torch.empty((1, shape[0]), device=dev) for _ in range(3)]

        def seq():
            ctx.reset_state(0)
            for t in range(3):
                ctx.forward(0, x[t:t + 1], out=outs[t])

        seq()
        torch.cuda.synchronize()
        ref = [o.clone() for o in outs]
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                seq()
        torch.cuda.synchronize()
        for rep in range(3):
            for o in outs:
                o.fill_(0.0)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            for o, r in zip(outs, ref):
                assert torch.equal(o, r), rep


def test_errors(torch_dev):
    torch, dev = torch_dev
    pkg = load_pkg()
    # the last: value_dim 3*32 = 96 is not a multiple of out_proj's q4 group of 64
    for bad in [(100, 1, 1, 64, 64, 4), (256, 2, 3, 64, 64, 4), (256, 1, 1, 48, 64, 4),
                (256, 1, 1, 64, 8, 4), (256, 1, 1, 64, 64, 0), (320, 1, 3, 32, 32, 7)]:
        with pytest.raises(pkg.QmoeError, match="DeltaNet shape unsupported"):
            pkg.DeltaNetContext(*bad)
    with pkg.DeltaNetContext(256, 2, 4, 64, 64, 4, n_layers=1, max_tokens=2) as ctx:
        x = torch.zeros((1, 256), device=dev)
        with pytest.raises(pkg.QmoeError, match="has no weights"):
            ctx.forward(0, x)
        with pytest.raises(pkg.QmoeError, match="out of range"):
            ctx.forward(1, x)
        ctx.upload_layer(0, orc.DeltaNet(256, 2, 4, 64, 64, 4).arrays())
        with pytest.raises(pkg.QmoeError, match="max_tokens"):
            ctx.forward(0, torch.zeros((3, 256), device=dev))
        arr = orc.DeltaNet(256, 2, 4, 64, 64, 4).arrays()
        arr["norm_w"] = None
        with pytest.raises(pkg.QmoeError, match="norm_w is NULL"):
            ctx.upload_layer(0, arr)
