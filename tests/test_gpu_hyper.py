"""The MLP hyper connection around the MoE layer on the GPU, through the C
ABI, against the oracle (c/src/model.c:728-796 and 1710-1731).

Bar: mixed, inject and normed within 2e-2 max-abs and 1e-3 relative L2 of
the oracle's gated_residual on the same hyper state.  The MoE layer then
runs on the GPU's own mixed rows, so its routing is held to the layer's
contract (expert ids and dispatch bit-exact against the oracle's router on
those rows) and its output and the updated hyper state to 2e-2 / 1e-3 of
the oracle's layer and inject update on them.  End to end (the oracle's own
mix, layer and update) the hyper state is held to the same bar where the
routing of the two mixes agrees, which it does on every case here.
"""
import ctypes

import numpy as np
import pytest

from ckpt_util import hc_name, hc_tensors, write_moe_layer
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


def device_bytes(ptr, nbytes):
    buf = np.empty(nbytes, np.uint8)
    rc = ctypes.CDLL("libamdhip64.so").hipMemcpy(ctypes.c_void_p(buf.ctypes.data),
                                                 ctypes.c_void_p(ptr), ctypes.c_size_t(nbytes), 2)
    assert rc == 0
    return buf


@pytest.fixture(scope="module")
def torch_dev(gpu):
    import torch
    return torch, gpu


TINY = dict(H=256, E=8, k=2, I=128, hc=4, R=128)
DECODE = dict(H=2048, E=512, k=10, I=512, hc=4, R=320)


def _case(torch, dev, shp, n, seed=0, n_check=8, upload=False):
    """GPU mix + layer + update vs the oracle on a selection of tokens"""
    pkg = load_pkg()
    H, E, k, I, hc, R = (shp[x] for x in ("H", "E", "k", "I", "hc", "R"))
    hp = orc.Hyper(hc, H, R, seed=seed, norm_std=0.1 if upload else 0.0)
    if upload:  # bf16-representable norm weights for the round trip
        hp = orc.Hyper.from_arrays(hc, H, R, dict(hp.arrays(), hc_norm=orc.bf16_to_f32(
            orc.f32_to_bf16(hp.arrays()["hc_norm"]))))
    hyper = orc.gen_hyper(n, hc, H, seed=seed + 100)
    sel = np.unique(np.linspace(0, n - 1, min(n, n_check)).astype(np.int32))
    with pkg.MoeContext(H, E, k, I, n_layers=1, max_tokens=n) as ctx:
        ctx.synth_layer(0, seed)
        ctx.hc_enable(hc, R)
        if upload:
            ctx.hc_upload_layer(0, hp.arrays())
        else:
            ctx.hc_synth_layer(0, seed)
        ht = torch.from_numpy(hyper).to(dev)
        m = ctx.hc_mix(0, ht)
        h2 = ht.clone()
        out = ctx.hc_layer_forward(0, h2)
        torch.cuda.synchronize()
        lr = ctx.last_routing(n)
        mixed_g = m["mixed"].cpu().numpy()
        inject_g = m["inject"].cpu().numpy()
        ref = hp.mix(hyper[sel])
        tag = f"H{H} E{E} k{k} hc{hc} R{R} n={n}"
        assert_close(m["normed"].cpu().numpy()[sel], ref["normed"], f"{tag} normed")
        assert_close(inject_g[sel], ref["inject"], f"{tag} inject")
        assert_close(mixed_g[sel], ref["mixed"], f"{tag} mixed")
        # the layer on the GPU's mixed rows
        L0 = orc.Layer(H, E, k, I, seed=seed, only_experts=[])
        route = L0.route(mixed_g, False)
        np.testing.assert_array_equal(lr["idx"].cpu().numpy(), route["idx"])
        dref = orc.dispatch(route["idx"], E)
        np.testing.assert_array_equal(lr["perm"].cpu().numpy(), dref["perm"])
        L = orc.Layer(H, E, k, I, seed=seed, only_experts=route["idx"][sel].reshape(-1))
        lref = L.forward(mixed_g, False, token_sel=sel)["out"]
        assert_close(out.cpu().numpy()[sel], lref, f"{tag} moe out")
        href = hp.inject_update(hyper[sel], inject_g[sel], lref)
        assert_close(h2.cpu().numpy()[sel], href, f"{tag} hyper")
        # end to end against the oracle's own mix
        route_o = L0.route(ref["mixed"], False)
        if np.array_equal(route_o["idx"], route["idx"][sel]):
            Lo = orc.Layer(H, E, k, I, seed=seed, only_experts=route_o["idx"].reshape(-1))
            e2e = hp.inject_update(hyper[sel], ref["inject"],
                                   Lo.forward(ref["mixed"], False)["out"])
            assert_close(h2.cpu().numpy()[sel], e2e, f"{tag} hyper end to end")
        else:
            pytest.fail(f"{tag}: oracle mix routes differently (near tie); pick another seed")
        return ctx


@pytest.mark.parametrize("n", [1, 4, 37])
def test_tiny_hyper_layer(torch_dev, n):
    torch, dev = torch_dev
    say(f"case: tiny hyper layer n={n}")
    _case(torch, dev, TINY, n, seed=n)


def test_tiny_hyper_layer_uploaded_weights(torch_dev):
    torch, dev = torch_dev
    say("case: tiny hyper layer, host-uploaded weights with a non-unit norm")
    _case(torch, dev, TINY, 5, seed=3, upload=True)


@pytest.mark.parametrize("n", [1, 4, 64, 300])
def test_decode_shape_hyper_layer(torch_dev, n):
    torch, dev = torch_dev
    say(f"case: decode-shape hyper layer (hc 4, rank 320) n={n}")
    _case(torch, dev, DECODE, n, seed=7, n_check=6)


@pytest.mark.parametrize("shp,n", [
    (dict(H=768, E=16, k=2, I=128, hc=3, R=192), 1),
    (dict(H=768, E=16, k=2, I=128, hc=3, R=192), 20),
    (dict(H=512, E=8, k=1, I=64, hc=1, R=64), 5),
    (dict(H=1536, E=32, k=4, I=256, hc=8, R=512), 70),
    (dict(H=2048, E=64, k=4, I=128, hc=2, R=2048), 17),
])
def test_hyper_shape_sweep(torch_dev, shp, n):
    """copy counts 1 to 8, ranks 64 to 2048, hidden 512 to 2048 (1536 =
    3 * 512 included): mix, layer and update against the oracle on both the
    GEMV (few tokens) and the MFMA (16 and more) paths"""
    torch, dev = torch_dev
    say(f"case: hyper sweep {shp} n={n}")
    _case(torch, dev, shp, n, seed=9, n_check=n)


def test_prefill_hyper_layer(torch_dev):
    torch, dev = torch_dev
    say("case: decode-shape hyper layer n=4096 (16 tokens checked)")
    _case(torch, dev, DECODE, 4096, seed=9, n_check=16)


def test_golden_hyper_tiny(torch_dev):
    """tests/golden/hyper_tiny.npz: the tiny layer inside its hyper connection"""
    import os
    torch, dev = torch_dev
    pkg = load_pkg()
    say("case: golden hyper_tiny (4 tokens, hc 4, rank 128, non-unit hc_norm)")
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "hyper_tiny.npz"))
    L = orc.Layer(256, 8, 2, 128, seed=0)
    a = orc.Hyper(4, 256, 128, seed=0, norm_std=0.2).arrays()
    a["hc_norm"] = np.array(g["hc_norm"])
    with pkg.MoeContext(256, 8, 2, 128, max_tokens=4) as ctx:
        ctx.upload_layer(0, L.arrays())
        ctx.hc_enable(4, 128)
        ctx.hc_upload_layer(0, a)
        h = torch.from_numpy(np.array(g["hyper_in"])).to(dev)
        out = ctx.hc_layer_forward(0, h)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(ctx.last_routing(4)["idx"].cpu().numpy(), g["idx"])
        assert_close(out.cpu().numpy(), g["moe_out"], "golden moe out")
        assert_close(h.cpu().numpy(), g["hyper_out"], "golden hyper")


def test_hc_synth_matches_host_generator(torch_dev):
    torch, dev = torch_dev
    pkg = load_pkg()
    say("case: qmoe_hc_synth_layer == oracle Hyper streams")
    H, hc, R = 256, 4, 128
    hp = orc.Hyper(hc, H, R, seed=11, layer=2)
    with pkg.MoeContext(H, 8, 2, 128, n_layers=3, max_tokens=2) as ctx:
        ctx.hc_enable(hc, R)
        ctx.hc_synth_layer(2, 11)
        dw = ctx.hc_device_weights(2)
        for key, a in hp.arrays().items():
            a = np.ascontiguousarray(a)
            assert device_bytes(dw[key], a.nbytes).tobytes() == a.tobytes(), key


def test_inject_alone(torch_dev):
    """qmoe_hc_inject: one fma per element, bit-identical to the oracle"""
    torch, dev = torch_dev
    pkg = load_pkg()
    say("case: qmoe_hc_inject alone")
    H, hc, n = 256, 4, 6
    rng = np.random.default_rng(1)
    hyper = rng.standard_normal((n, hc * H)).astype(np.float32)
    inject = rng.uniform(0, 2, (n, hc)).astype(np.float32)
    out = rng.standard_normal((n, H)).astype(np.float32)
    with pkg.MoeContext(H, 8, 2, 128, max_tokens=n) as ctx:
        ctx.hc_enable(hc, 128)
        ht = torch.from_numpy(hyper).to(dev)
        ctx.hc_inject(torch.from_numpy(inject).to(dev), torch.from_numpy(out).to(dev), ht)
        torch.cuda.synchronize()
        want = orc.Hyper(hc, H, 128).inject_update(hyper, inject, out)
        assert np.array_equal(ht.cpu().numpy(), want)


def test_hyper_errors(torch_dev):
    torch, dev = torch_dev
    pkg = load_pkg()
    say("case: hyper-connection argument errors")
    with pkg.MoeContext(256, 8, 2, 128, max_tokens=4) as ctx:
        x = torch.zeros((1, 1024), dtype=torch.float32, device=dev)
        with pytest.raises(pkg.QmoeError, match="not enabled"):
            ctx.hc = 4
            ctx.hc_mix(0, x)
        for hc, R, needle in ((9, 128, "unsupported"), (4, 96, "unsupported"),
                              (4, 4096, "unsupported"), (40, 128, "unsupported")):
            with pytest.raises(pkg.QmoeError, match=needle):
                ctx.hc_enable(hc, R)
        ctx.hc_enable(4, 128)
        ctx.hc_enable(4, 128)  # same values: no-op
        with pytest.raises(pkg.QmoeError, match="already enabled"):
            ctx.hc_enable(2, 128)
        with pytest.raises(pkg.QmoeError, match="no hyper-connection weights"):
            ctx.hc_mix(0, x)
        ctx.hc_synth_layer(0, 1)
        with pytest.raises(pkg.QmoeError, match="has no weights"):
            ctx.hc_layer_forward(0, x)  # the MoE layer itself is empty
        with pytest.raises(pkg.QmoeError, match="out of range"):
            ctx.hc_mix(0, torch.zeros((5, 1024), dtype=torch.float32, device=dev))
        arrays = orc.Hyper(4, 256, 128).arrays()
        arrays["up_b"] = None
        with pytest.raises(pkg.QmoeError, match="missing hyper-connection tensor up_b"):
            ctx.hc_upload_layer(0, arrays)


# ------------------------------------------------------------ checkpoint

def _hc_ckpt(tmp_path, hp, H, E, I, layer, drop=(), replace=None):
    L = orc.Layer(H, E, 2, I, seed=0)
    extra = hc_tensors(hp.arrays(), hp.hc, H, hp.R, layer, drop=drop)
    extra.update(replace or {})
    write_moe_layer(str(tmp_path), L.arrays(), H, E, I, layer=layer, shards=2, extra=extra)
    return L


def test_hc_checkpoint_upload(torch_dev, tmp_path):
    torch, dev = torch_dev
    pkg = load_pkg()
    say("case: hyper connection uploaded from checkpoint layer 3")
    H, E, I, hc, R = 256, 8, 128, 4, 128
    base = orc.Hyper(hc, H, R, seed=2, norm_std=0.1)
    a = base.arrays()
    a["hc_norm"] = orc.bf16_to_f32(orc.f32_to_bf16(a["hc_norm"]))
    hp = orc.Hyper.from_arrays(hc, H, R, a)
    _hc_ckpt(tmp_path, hp, H, E, I, layer=3)
    with pkg.Checkpoint(str(tmp_path)) as ck, pkg.MoeContext(H, E, 2, I, n_layers=2,
                                                             max_tokens=4) as ctx:
        ctx.hc_enable(hc, R)
        ctx.hc_upload_layer_st(1, ck, 3)
        ctx.hc_upload_layer(0, hp.arrays())
        d1, d0 = ctx.hc_device_weights(1), ctx.hc_device_weights(0)
        for key, arr in hp.arrays().items():
            arr = np.ascontiguousarray(arr)
            assert device_bytes(d1[key], arr.nbytes).tobytes() == arr.tobytes(), key
        ht = torch.from_numpy(orc.gen_hyper(4, hc, H, seed=5)).to(dev)
        m1, m0 = ctx.hc_mix(1, ht), ctx.hc_mix(0, ht)
        torch.cuda.synchronize()
        assert np.array_equal(m1["mixed"].cpu().numpy(), m0["mixed"].cpu().numpy())


@pytest.mark.parametrize("case,needle", [
    ("dense_mix", "dense mix weights are not supported"),
    ("quant_inject", "block_inject_weight must be dense BF16"),
    ("norm_f32", "must be BF16 (got F32)"),
    ("wrong_rank", "has shape [64,128]"),
    ("missing", "missing tensor model.layers.0.mlp_hyper_connection.block_inject_weight.weight"),
])
def test_hc_checkpoint_errors(torch_dev, tmp_path, case, needle):
    torch, dev = torch_dev
    pkg = load_pkg()
    say(f"case: hyper-connection checkpoint error {case}")
    H, E, I, hc, R = 256, 8, 128, 4, 128
    hp = orc.Hyper(hc, H, R, seed=1)
    drop, replace = (), {}
    if case == "dense_mix":
        drop = ("up_s",)
    elif case == "quant_inject":
        replace[hc_name(0, "inject_w").replace(".weight", ".scales")] = \
            torch.zeros((hc, hc * H // 64), dtype=torch.bfloat16)
    elif case == "norm_f32":
        replace[hc_name(0, "hc_norm")] = torch.ones(hc * H, dtype=torch.float32)
    elif case == "wrong_rank":
        replace[hc_name(0, "down_q")] = torch.zeros((64, hc * H // 8),
                                                    dtype=torch.int32).view(torch.uint32)
    elif case == "missing":
        drop = ("inject_w",)
    _hc_ckpt(tmp_path, hp, H, E, I, layer=0, drop=drop, replace=replace)
    with pkg.Checkpoint(str(tmp_path)) as ck, pkg.MoeContext(H, E, 2, I, max_tokens=4) as ctx:
        ctx.hc_enable(hc, R)
        with pytest.raises(pkg.QmoeError) as ei:
            ctx.hc_upload_layer_st(0, ck, 0)
        assert needle in str(ei.value), str(ei.value)
