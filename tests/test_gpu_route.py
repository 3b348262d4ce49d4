"""Router + top-k for batches of 256 tokens or more (route_mfma.hip): MFMA
logits with a bound per (token, expert), exact R64 logits for the experts
whose bound reaches the top k.  Selected experts, weights and shared-gate
values must equal, bit for bit, those of the exact router (every R64 logit,
then the canonical top-k: ctx.router with want_logits=True), and the
experts must equal the oracle's (orc_route), on random bf16 and f32 rows,
normalised rows, and inputs made to defeat an approximate selection: exact
and one-ulp near ties between router rows, constant logits, tokens that
hold NaN or inf or overflow the bound, zero and subnormal rows."""

import numpy as np
import pytest

from conftest import load_oracle, load_pkg

pytestmark = pytest.mark.gpu
orc = load_oracle()


def say(msg):
    print(msg, flush=True)


def to_dev(a, torch, dev):
    if a.dtype == np.uint16:  # bf16 bit patterns
        return torch.from_numpy(a.view(np.int16)).to(dev).view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.fixture(scope="module")
def torch_dev(gpu):
    import torch
    return torch, gpu


def bits(t):
    return t.cpu().numpy().view(np.int32)


def same_selection(ctx, xt, norm, torch, what):
    """the MFMA route against the exact route, bit for bit"""
    if norm:
        fast = ctx.router_norm(0, xt, want_logits=False)
        full = ctx.router_norm(0, xt, want_logits=True)
    else:
        fast = ctx.router(0, xt)
        full = ctx.router(0, xt, want_logits=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(fast["idx"].cpu().numpy(), full["idx"].cpu().numpy(), err_msg=what)
    np.testing.assert_array_equal(bits(fast["w"]), bits(full["w"]), err_msg=what)
    np.testing.assert_array_equal(bits(fast["shared_gate"]), bits(full["shared_gate"]), err_msg=what)
    if norm:
        np.testing.assert_array_equal(bits(fast["xn"]), bits(full["xn"]), err_msg=what)
    return fast, full


@pytest.mark.parametrize("n,bf16", [(256, True), (300, False)])
def test_route_decode_shape(torch_dev, n, bf16):
    """H=2048, E=512, k=10 with the Zipf router bias: bf16 rows go to MFMA
    as they are, f32 rows rounded to bf16"""
    torch, dev = torch_dev
    pkg = load_pkg()
    w = pkg.WORKLOADS["batched"]
    say(f"case: route n={n} bf16={bf16} H={w.hidden} E={w.n_experts} k={w.top_k} (Zipf bias)")
    rb = orc.zipf_bias(w.n_experts, w.zipf_s, w.zipf_scale, w.seed * 1000003)
    x = orc.gen_x(n, w.hidden, 31, bf16=bf16)
    Lr = orc.Layer(w.hidden, w.n_experts, w.top_k, w.moe_inter, seed=w.seed, router_bias=rb,
                   only_experts=[])
    ref = Lr.route(x, bf16)
    with pkg.MoeContext.for_workload(w, max_tokens=n, n_layers=1) as ctx:
        ctx.synth_layer(0, w.seed, router_bias=rb)
        fast, _ = same_selection(ctx, to_dev(x, torch, dev), False, torch, "decode shape")
        np.testing.assert_array_equal(fast["idx"].cpu().numpy(), ref["idx"])
        np.testing.assert_allclose(fast["w"].cpu().numpy(), ref["w"], rtol=1e-6)
        np.testing.assert_allclose(fast["shared_gate"].cpu().numpy(), ref["shared_gate"], rtol=1e-6)


@pytest.mark.parametrize("bf16", [True, False])
def test_route_norm_shape(torch_dev, bf16):
    """pre-router RMSNorm: the normalised rows (written by the MFMA route)
    and the selection equal the exact router's and the oracle's"""
    torch, dev = torch_dev
    pkg = load_pkg()
    w = pkg.WORKLOADS["depth48"]
    n = 257
    say(f"case: RMSNorm + route n={n} bf16={bf16}")
    rb = orc.zipf_bias(w.n_experts, w.zipf_s, w.zipf_scale, w.seed * 1000003)
    h = orc.gen_x(n, w.hidden, 33, bf16=bf16)
    Lr = orc.Layer(w.hidden, w.n_experts, w.top_k, w.moe_inter, seed=w.seed, layer=0,
                   with_norm=True, router_bias=rb, only_experts=[])
    ref = Lr.route(h, bf16)
    with pkg.MoeContext.for_workload(w, max_tokens=n, n_layers=1) as ctx:
        ctx.synth_layer(0, w.seed, with_norm=True, router_bias=rb)
        fast, _ = same_selection(ctx, to_dev(h, torch, dev), True, torch, "norm shape")
        np.testing.assert_array_equal(fast["xn"].cpu().numpy(), ref["xn"])
        np.testing.assert_array_equal(fast["idx"].cpu().numpy(), ref["idx"])


def _small_layer(H, E, k, I, seed, edit=None, bias=None):
    L = orc.Layer(H, E, k, I, seed=seed, router_bias=bias)
    if edit is not None:
        rw = L.t["router_w"].reshape(E, H).copy()
        edit(rw)
        L.t["router_w"] = rw.reshape(-1)
        L._build()
    return L


def _near_ties(rw):
    """pairs of rows: identical, or one bf16 ulp apart in one element"""
    E = rw.shape[0]
    for e in range(0, E - 1, 2):
        rw[e + 1] = rw[e]
        if e % 4 == 2:
            rw[e + 1, e % rw.shape[1]] += 1  # next bf16 up (same sign)


ADVERSARIAL = [
    # (label, H, E, k, edit, bias)
    ("exact and 1-ulp near ties", 512, 64, 8, _near_ties, None),
    ("all rows zero, no bias", 512, 64, 8, lambda rw: rw.fill(0), None),
    ("all rows zero, tied bias", 512, 128, 6, lambda rw: rw.fill(0),
     np.repeat(np.float32([0.5, -1.0, 0.25, 2.0]), 32)),
    ("E=1024 k=64", 512, 1024, 64, None, None),
    ("H=1024 E=256 k=16 ties", 1024, 256, 16, _near_ties, None),
]


@pytest.mark.parametrize("case", ADVERSARIAL, ids=[c[0] for c in ADVERSARIAL])
@pytest.mark.parametrize("bf16", [True, False])
def test_route_adversarial(torch_dev, case, bf16):
    torch, dev = torch_dev
    pkg = load_pkg()
    label, H, E, k, edit, bias = case
    n, I = 260, 64
    say(f"case: route, {label}, H={H} E={E} k={k} n={n} bf16={bf16}")
    L = _small_layer(H, E, k, I, seed=5, edit=edit, bias=bias)
    x = orc.gen_x(n, H, 7, bf16=False)
    # rows that the bound must hand to the exact path, and degenerate rows
    x[0, 3] = np.nan
    x[1, 5] = np.inf
    x[2, :] *= np.float32(3e19)   # |x|^2 overflows
    x[3, :] = 0.0
    x[4, :] = -0.0
    x[5, :] *= np.float32(1e-40)  # subnormal (f32) / flushed (bf16) rows
    x[6, :] = x[7, :]             # identical tokens
    xin = orc.f32_to_bf16(x) if bf16 else x
    with pkg.MoeContext(H, E, k, I, max_tokens=n) as ctx:
        ctx.upload_layer(0, L.arrays())
        xt = to_dev(xin, torch, dev)
        fast, _ = same_selection(ctx, xt, False, torch, label)
        ref = L.route(xin, bf16)
        fin = np.isfinite(ref["logits"]).all(axis=1)
        np.testing.assert_array_equal(fast["idx"].cpu().numpy()[fin], ref["idx"][fin])
        ctx.layer_forward(0, xt)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(ctx.last_routing(n)["idx"].cpu().numpy(), fast["idx"].cpu().numpy())
