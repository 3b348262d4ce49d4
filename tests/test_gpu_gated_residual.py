"""The stand-alone gated residual (qmoe_gr_*, through the C ABI): the
attention-block hyper connection of each decoder layer (with inject) and
the final mixer (without), against the oracle's gated_residual and inject
update (orc_hc_mix / orc_hc_inject, pinned by tests/test_oracle_hyper.py).

Bar: mixed and inject within 2e-2 max-abs and 1e-3 relative L2 of the
oracle on the same hyper state, on the GEMV path (n < 16) and the MFMA path
(n >= 16); the inject update bit-exact (one fused multiply-add per element,
as the oracle).

Then the reference's layer loop (c/src/model.c:1666-1745) composed from the
library's parts -- attention-block connection, DeltaNet or attention mixer,
inject update, MLP hyper connection + MoE layer, and after the last layer
the final mixer -- over a prefill chunk and decode steps.  Every stage is
held to the bar above on the GPU's own inputs (MoE routing bit-exact), and
the final mixer's output to the same bar against the oracle run end to end
from the same initial hyper state.  Weights are uploaded from the oracle's
host arrays (no device generator involved).
"""
import numpy as np
import pytest

from conftest import load_oracle, load_pkg

orc = load_oracle()

pytestmark = pytest.mark.gpu

MAX_ABS, REL_L2 = 2e-2, 1e-3


def say(msg):
    print(msg, flush=True)


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def assert_close(got, ref, what):
    err = float(np.abs(got - ref).max())
    rel = rel_l2(got, ref)
    say(f"{what}: max-abs {err:.3e} rel-L2 {rel:.3e} (|ref| max {np.abs(ref).max():.2f})")
    assert err < MAX_ABS and rel < REL_L2, (what, err, rel)


@pytest.fixture(scope="module")
def torch_dev(gpu):
    import torch
    return torch, gpu


@pytest.mark.parametrize("hc,d,R", [(4, 256, 128), (4, 2048, 320), (2, 192, 64)])
@pytest.mark.parametrize("n", [1, 7, 16, 200])
def test_mix_with_and_without_inject(torch_dev, hc, d, R, n):
    torch, dev = torch_dev
    pkg = load_pkg()
    say(f"case: gated residual hc={hc} d={d} R={R} n={n}")
    ah = orc.Hyper(hc, d, R, seed=11, layer=3, norm_std=0.1)
    mixer = orc.Hyper(hc, d, R, seed=12, layer=0, norm_std=0.1, with_inject=False)
    hyper = orc.gen_hyper(n, hc, d, seed=n + 5) * 2.0
    with pkg.GatedResidualContext(d, hc, R, n_slots=2, max_tokens=200) as gr:
        gr.upload_slot(0, ah.arrays())
        gr.upload_slot(1, mixer.arrays())
        ht = torch.from_numpy(hyper).to(dev)
        m0, i0 = gr.mix(0, ht)
        m1, i1 = gr.mix(1, ht)
        m0b, i0b = gr.mix(0, ht, want_inject=False)  # inject dots skipped
        torch.cuda.synchronize()
        assert i1 is None and i0b is None
        r0, r1 = ah.mix(hyper), mixer.mix(hyper)
        tag = f"hc{hc} d{d} R{R} n={n}"
        assert_close(m0.cpu().numpy(), r0["mixed"], f"{tag} attention-block mixed")
        assert_close(i0.cpu().numpy(), r0["inject"], f"{tag} attention-block inject")
        assert_close(m1.cpu().numpy(), r1["mixed"], f"{tag} final mixer")
        np.testing.assert_array_equal(m0b.cpu().numpy(), m0.cpu().numpy())
        # the inject update: one fma per element, as the oracle
        out = torch.from_numpy(orc.gen_attn_x(n, d, seed=n)).to(dev)
        h2 = gr.inject(i0, out, ht.clone())
        torch.cuda.synchronize()
        np.testing.assert_array_equal(
            h2.cpu().numpy(), ah.inject_update(hyper, i0.cpu().numpy(), out.cpu().numpy()))


def test_errors(torch_dev):
    torch, dev = torch_dev
    pkg = load_pkg()
    for bad in [(100, 4, 128), (256, 9, 128), (256, 4, 100), (4096, 4, 128)]:
        with pytest.raises(pkg.QmoeError, match="gated residual shape unsupported"):
            pkg.GatedResidualContext(*bad)
    with pytest.raises(pkg.QmoeError, match="n_slots"):
        pkg.GatedResidualContext(256, 4, 128, n_slots=0)
    mixer = orc.Hyper(4, 256, 128, seed=1, with_inject=False)
    with pkg.GatedResidualContext(256, 4, 128, n_slots=2, max_tokens=4) as gr:
        x = torch.zeros((2, 4 * 256), device=dev)
        with pytest.raises(pkg.QmoeError, match="has no weights"):
            gr.mix(0, x)
        with pytest.raises(pkg.QmoeError, match="out of range"):
            gr.mix(2, x)
        bad = dict(mixer.arrays())
        del bad["up_s"]
        with pytest.raises(pkg.QmoeError, match="up_s is NULL"):
            gr.upload_slot(0, bad)
        gr.upload_slot(0, mixer.arrays())
        with pytest.raises(pkg.QmoeError, match="no inject weights"):
            gr.mix(0, x, want_inject=True)
        with pytest.raises(pkg.QmoeError, match="max_tokens"):
            gr.mix(0, torch.zeros((5, 4 * 256), device=dev))
        m, _ = gr.mix(0, x)
        torch.cuda.synchronize()
        assert m.shape == (2, 256)


# ------------------------------------------------------------ layer loop

class Chain:
    """the weights and states of a small decoder (layer types as given),
    in the oracle and on the GPU"""

    def __init__(self, torch, dev, shp, types, seed, max_tokens):
        pkg = load_pkg()
        self.torch, self.dev, self.shp, self.types = torch, dev, shp, types
        d, hc, R = shp["d"], shp["hc"], shp["R"]
        E, k, I = shp["E"], shp["k"], shp["I"]
        L = len(types)
        self.ah = [orc.Hyper(hc, d, R, seed=seed + 10, layer=l, norm_std=0.1) for l in range(L)]
        self.mh = [orc.Hyper(hc, d, R, seed=seed + 20, layer=l, norm_std=0.1) for l in range(L)]
        self.mixer = orc.Hyper(hc, d, R, seed=seed + 30, norm_std=0.1, with_inject=False)
        self.moe = [orc.Layer(d, E, k, I, seed=seed + 40, layer=l) for l in range(L)]
        self.mixers = []
        for l, t in enumerate(types):
            if t == "dn":
                self.mixers.append(orc.DeltaNet(d, *shp["dn"], seed=seed + 50, layer=l))
            else:
                self.mixers.append(orc.Attention(d, *shp["attn"], seed=seed + 60 + l))
        # device side
        self.gr = pkg.GatedResidualContext(d, hc, R, n_slots=L + 1, max_tokens=max_tokens)
        for l in range(L):
            self.gr.upload_slot(l, self.ah[l].arrays())
        self.gr.upload_slot(L, self.mixer.arrays())
        self.ctx = pkg.MoeContext(d, E, k, I, n_layers=L, max_tokens=max_tokens)
        self.ctx.hc_enable(hc, R)
        for l in range(L):
            self.ctx.upload_layer(l, self.moe[l].arrays())
            self.ctx.hc_upload_layer(l, self.mh[l].arrays())
        dn_l = [l for l, t in enumerate(types) if t == "dn"]
        at_l = [l for l, t in enumerate(types) if t == "attn"]
        self.dn = pkg.DeltaNetContext(d, *shp["dn"], n_layers=L, max_tokens=max_tokens)
        a = shp["attn"]
        self.at = pkg.AttentionContext(d, *a[:7], kv_cap=a[7], rotary_factor=a[8], n_layers=L,
                                       max_tokens=max_tokens)
        for l in dn_l:
            self.dn.upload_layer(l, self.mixers[l].arrays())
        for l in at_l:
            self.at.upload_layer(l, self.mixers[l].arrays())
        # oracle states: one set that follows the GPU's inputs, one end to end
        self.st_gpu = [self._new_state(l) for l in range(L)]
        self.st_e2e = [self._new_state(l) for l in range(L)]

    def _new_state(self, l):
        return self.mixers[l].new_state()

    def close(self):
        self.gr.close()
        self.ctx.close()
        self.dn.close()
        self.at.close()

    def _mixer_ref(self, l, x, st, offset):
        m = self.mixers[l]
        if self.types[l] == "dn":
            return m.forward(x, st[0], st[1])
        return m.forward(x, st, offset)

    def step_gpu(self, h, offset, tag):
        """one call of the layer loop on the GPU, each stage checked against
        the oracle on the GPU's own inputs; returns the final mixer output"""
        torch = self.torch
        self.routes = []
        for l, t in enumerate(self.types):
            lt = f"{tag} layer {l} ({t})"
            hn = h.cpu().numpy()
            m, inj = self.gr.mix(l, h)
            out = (self.dn.forward(l, m) if t == "dn" else self.at.forward(l, m, offset))
            torch.cuda.synchronize()
            ref = self.ah[l].mix(hn)
            mg, ig = m.cpu().numpy(), inj.cpu().numpy()
            assert_close(mg, ref["mixed"], f"{lt} attention-block mixed")
            assert_close(ig, ref["inject"], f"{lt} attention-block inject")
            og = out.cpu().numpy()
            assert_close(og, self._mixer_ref(l, mg, self.st_gpu[l], offset), f"{lt} mixer out")
            self.gr.inject(inj, out, h)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(h.cpu().numpy(), self.ah[l].inject_update(hn, ig, og))
            # MLP hyper connection + MoE layer (mix, route, experts, inject)
            hn = h.cpu().numpy()
            mm = self.ctx.hc_mix(l, h)
            mo = self.ctx.hc_layer_forward(l, h)
            torch.cuda.synchronize()
            lr = self.ctx.last_routing(h.shape[0])
            mmg = mm["mixed"].cpu().numpy()
            mref = self.mh[l].mix(hn)
            assert_close(mmg, mref["mixed"], f"{lt} MLP mixed")
            route = self.moe[l].route(mmg, False)
            np.testing.assert_array_equal(lr["idx"].cpu().numpy(), route["idx"])
            self.routes.append(route["idx"])
            lref = self.moe[l].forward(mmg, False)["out"]
            assert_close(mo.cpu().numpy(), lref, f"{lt} moe out")
            assert_close(h.cpu().numpy(),
                         self.mh[l].inject_update(hn, mm["inject"].cpu().numpy(), lref),
                         f"{lt} hyper")
        fin, none = self.gr.mix(len(self.types), h)
        torch.cuda.synchronize()
        assert none is None
        fg = fin.cpu().numpy()
        assert_close(fg, self.mixer.mix(h.cpu().numpy())["mixed"], f"{tag} final mixer")
        return fg

    def step_oracle(self, hn, offset):
        """the same call run by the oracle alone; returns (final, routes)"""
        routes = []
        for l in range(len(self.types)):
            a = self.ah[l].mix(hn)
            out = self._mixer_ref(l, a["mixed"], self.st_e2e[l], offset)
            hn = self.ah[l].inject_update(hn, a["inject"], out)
            mref = self.mh[l].mix(hn)
            r = self.moe[l].forward(mref["mixed"], False)
            routes.append(self.moe[l].route(mref["mixed"], False)["idx"])
            hn = self.mh[l].inject_update(hn, mref["inject"], r["out"])
        return self.mixer.mix(hn)["mixed"], hn, routes


TINY = dict(d=256, hc=4, R=128, E=8, k=2, I=128,
            dn=(2, 4, 64, 64, 4),                       # hk, hv, dk, dv, conv kernel
            attn=(4, 2, 64, 2, 64, 8, 2, 64, 0.25))     # h, kvh, hd, ih, ihd, budget, comp, cap, rf
MODEL = dict(d=2048, hc=4, R=320, E=512, k=10, I=512,
             dn=(16, 32, 128, 128, 4),
             attn=(16, 2, 128, 4, 128, 512, 4, 1024, 0.25))


@pytest.mark.parametrize("shape,types,calls,seed", [
    ("tiny", ("dn", "attn", "dn"), (6, 1, 1, 20), 1),
    ("model", ("dn", "attn"), (5, 1, 1), 2),
])
def test_layer_loop(torch_dev, shape, types, calls, seed):
    torch, dev = torch_dev
    shp = TINY if shape == "tiny" else MODEL
    say(f"case: layer loop {shape} {types} calls {calls}")
    ch = Chain(torch, dev, shp, types, seed, max(calls))
    try:
        n_all = sum(calls)
        h0 = orc.gen_hyper(n_all, shp["hc"], shp["d"], seed=seed + 70)
        off = 0
        for i, n in enumerate(calls):
            tag = f"{shape} call {i} (n={n}, offset {off})"
            h = torch.from_numpy(h0[off:off + n].copy()).to(dev)
            fin = ch.step_gpu(h, off, tag)
            ref, _, routes = ch.step_oracle(h0[off:off + n], off)
            # end to end: the oracle's own chain from the same hyper state,
            # which routes every token as the GPU's chain did
            for l, r in enumerate(routes):
                assert np.array_equal(r, ch.routes[l]), \
                    f"{tag} layer {l}: the oracle chain routes differently (near tie); pick another seed"
            assert_close(fin, ref, f"{tag} final mixer end to end")
            off += n
    finally:
        ch.close()


@pytest.mark.parametrize("shape", ["tiny", "model"])
@pytest.mark.parametrize("n", [1, 3])
def test_mixer_forward_inject(torch_dev, shape, n):
    """qmoe_dn_forward_inject / qmoe_attn_forward_inject (the gated
    residual's update fused into the mixer's last launch) against the
    separate mixer call + qmoe_gr_inject from the same state: out and the
    hyper state bit-identical, the update bit-exact against the oracle's
    inject_update of the GPU's out; and with out NULL the same hyper
    state"""
    torch, dev = torch_dev
    shp = TINY if shape == "tiny" else MODEL
    types = ("dn", "attn")
    say(f"case: mixer forward_inject {shape} n={n}")
    ch = Chain(torch, dev, shp, types, 7, 4)
    try:
        h0 = torch.from_numpy(orc.gen_hyper(n, shp["hc"], shp["d"], seed=71)).to(dev)
        for l, t in enumerate(types):
            tag = f"{shape} n={n} {t}"
            m, inj = ch.gr.mix(l, h0)

            def fwd(**kw):
                if t == "dn":
                    ch.dn.reset_state(l)
                    return ch.dn.forward_inject(l, m, **kw) if "hyper" in kw else ch.dn.forward(l, m, **kw)
                ch.at.reset(l)
                return (ch.at.forward_inject(l, m, 0, **kw) if "hyper" in kw else ch.at.forward(l, m, 0, **kw))

            out_a = fwd()
            h_a = ch.gr.inject(inj, out_a, h0.clone())
            out_b = torch.empty_like(out_a)
            h_b = h0.clone()
            fwd(hyper=h_b, inject=inj, out=out_b)
            h_c = h0.clone()
            fwd(hyper=h_c, inject=inj)
            torch.cuda.synchronize()
            assert torch.equal(out_a, out_b), tag
            assert torch.equal(h_a, h_b), tag
            assert torch.equal(h_a, h_c), tag
            np.testing.assert_array_equal(
                h_b.cpu().numpy(), ch.ah[l].inject_update(h0.cpu().numpy(), inj.cpu().numpy(),
                                                          out_b.cpu().numpy()))
            say(f"{tag}: out and hyper bit-identical to the separate update, update exact")
        # refusals: hc out of range, missing hyper / inject
        bad_inj = torch.zeros((n, 9), device=dev)
        with pytest.raises(pkg_error()):
            ch.dn.forward_inject(0, m, h0, bad_inj)
        with pytest.raises(pkg_error()):
            ch.at.forward_inject(1, m, 0, h0, bad_inj)
    finally:
        ch.close()


def pkg_error():
    return load_pkg().QmoeError


def test_decoder_stack(torch_dev):
    """the benchmark's decoder stack (qmoe.DecoderStack: gated DeltaNet and
    full attention at 3 : 1 by the model's layer types, both hyper
    connections of every layer, the final mixer) at 4 of its 48 layers and
    the model's shapes, end to end against the oracle's own chain from the
    same hyper states: a 4-token prefill call, then one-token calls.  The
    final mixer output and the hyper state after the last layer within
    2e-2 max-abs and 1e-3 relative L2."""
    torch, dev = torch_dev
    pkg = load_pkg()
    types = tuple(pkg.decoder_layer_types(4))
    assert types == ("dn", "dn", "dn", "attn")
    seed, calls = 5, (4, 1, 1)
    say(f"case: decoder stack {types} calls {calls}")
    ch = Chain(torch, dev, MODEL, types, seed, max(calls))
    try:
        h0 = orc.gen_hyper(sum(calls), MODEL["hc"], MODEL["d"], seed=seed + 70)
        off = 0
        for i, n in enumerate(calls):
            tag = f"stack call {i} (n={n}, offset {off})"
            stack = pkg.DecoderStack(ch.gr, ch.ctx, ch.dn, ch.at, types, n)
            h = torch.from_numpy(h0[off:off + n].copy()).to(dev)
            fin = stack.step(h, off)
            torch.cuda.synchronize()
            ref, href, _ = ch.step_oracle(h0[off:off + n], off)
            assert_close(fin.cpu().numpy(), ref, f"{tag} final mixer")
            assert_close(h.cpu().numpy(), href, f"{tag} hyper state")
            say(f"{tag}: final mixer and hyper state within bounds")
            off += n
    finally:
        ch.close()
