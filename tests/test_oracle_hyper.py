"""Pins of the oracle's hyper connection (orc_hc_mix, orc_hc_inject) -- CPU.

The C restatement of gated_residual (c/src/model.c:728-796) is checked
against an independent float64 numpy statement of the MLX module
(src/colibri_runtime/model.py:463-481: GatedResidual.__call__), and against
closed forms that a plausible mistake breaks: the grouped RMSNorm is per
copy (scaling one copy changes nothing), a zero mix matrix gives
sigmoid(0) = 1/2 gates and a zero inject matrix gives inject = 2*sigmoid(0)
= 1 exactly, the copies are averaged (not summed, not one copy), and the
inject update is one fused multiply-add per element (model.c:1724-1731)."""
import numpy as np
import pytest

from conftest import load_oracle

orc = load_oracle()


def dequant64(q, s, b, rows, cols, g=64):
    """MLX affine q4 (low nibble first) to float64, [rows, cols]"""
    q = np.asarray(q, np.uint32).reshape(rows, cols // 8)
    codes = np.stack([(q >> np.uint32(4 * i)) & np.uint32(15) for i in range(8)], axis=-1)
    codes = codes.reshape(rows, cols).astype(np.float64)
    sc = orc.bf16_to_f32(s).astype(np.float64).reshape(rows, cols // g)
    bi = orc.bf16_to_f32(b).astype(np.float64).reshape(rows, cols // g)
    return codes * np.repeat(sc, g, axis=1) + np.repeat(bi, g, axis=1)


def gated_residual_f64(hp, hyper):
    """model.py:472-481 in float64"""
    hc, d, R = hp.hc, hp.d, hp.R
    t = hp.arrays()
    x = np.asarray(hyper, np.float64).reshape(-1, hc, d)
    rms = np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6)
    normed = (x / rms * t["hc_norm"].astype(np.float64).reshape(hc, d)).reshape(-1, hc * d)
    wd = dequant64(t["down_q"], t["down_s"], t["down_b"], R, hc * d)
    wu = dequant64(t["up_q"], t["up_s"], t["up_b"], hc * d, R)
    v = normed @ wd.T / hc
    w = v / (1.0 + np.exp(-v))
    gate = 1.0 / (1.0 + np.exp(-(w @ wu.T)))
    mixed = (gate.reshape(-1, hc, d) * normed.reshape(-1, hc, d)).mean(-2)
    wi = orc.bf16_to_f32(t["inject_w"]).astype(np.float64).reshape(hc, hc * d)
    inject = 2.0 / (1.0 + np.exp(-(normed @ wi.T) / hc))
    return mixed, inject, normed


@pytest.mark.parametrize("hc,d,R,n", [(4, 256, 128, 3), (2, 128, 64, 5), (4, 64, 320, 1)])
def test_mix_vs_float64_statement(hc, d, R, n):
    hp = orc.Hyper(hc, d, R, seed=3, norm_std=0.2)
    hyper = orc.gen_hyper(n, hc, d, seed=9) * 3.0
    got = hp.mix(hyper)
    mixed, inject, normed = gated_residual_f64(hp, hyper)
    np.testing.assert_allclose(got["normed"], normed, rtol=2e-5, atol=2e-5)
    np.testing.assert_allclose(got["inject"], inject, rtol=1e-5, atol=1e-6)
    scale = np.abs(mixed).max()
    assert np.abs(got["mixed"] - mixed).max() < 1e-5 * scale


def test_final_mixer_has_no_inject():
    """the final mixer (model.c:1743-1745) passes no inject matrix: mixed is
    the float64 statement's, bit for bit the mix of the same weights with an
    inject matrix, and no inject comes back"""
    hc, d, R, n = 4, 128, 64, 4
    full = orc.Hyper(hc, d, R, seed=5, layer=1, norm_std=0.1)
    mixer = orc.Hyper(hc, d, R, seed=5, layer=1, norm_std=0.1, with_inject=False)
    assert "inject_w" not in mixer.arrays()
    hyper = orc.gen_hyper(n, hc, d, seed=4) * 2.0
    got = mixer.mix(hyper)
    assert got["inject"] is None
    np.testing.assert_array_equal(got["mixed"], full.mix(hyper)["mixed"])
    mixed, _, _ = gated_residual_f64(full, hyper)
    assert np.abs(got["mixed"] - mixed).max() < 1e-5 * np.abs(mixed).max()


def test_norm_is_per_copy():
    """scaling one copy of the hyper state leaves mixed and inject unchanged
    (a norm over the whole hc*d row would not)"""
    hp = orc.Hyper(4, 128, 64, seed=1)
    hyper = orc.gen_hyper(2, 4, 128, seed=2)
    a = hp.mix(hyper)
    h2 = hyper.copy()
    h2[:, 128:256] *= 8.0  # (only eps breaks the invariance, far below 1e-5)
    b = hp.mix(h2)
    for key in ("normed", "mixed", "inject"):
        np.testing.assert_allclose(a[key], b[key], rtol=1e-5, atol=1e-6)


def test_zero_mix_and_inject_closed_form():
    hc, d, R = 4, 128, 64
    hp = orc.Hyper(hc, d, R, seed=5)
    t = hp.arrays()
    for k in ("down_q", "down_s", "down_b", "up_q", "up_s", "up_b", "inject_w"):
        t[k] = np.zeros_like(t[k])
    hz = orc.Hyper.from_arrays(hc, d, R, t)
    # all copies equal to v: normed copies are v / rms(v) and the gates are 1/2
    v = orc.gen_hyper(3, 1, d, seed=4)
    hyper = np.tile(v, (1, hc))
    m = hz.mix(hyper)
    assert np.array_equal(m["inject"], np.ones((3, hc), np.float32))
    want = 0.5 * v / np.sqrt((v.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-6)
    np.testing.assert_allclose(m["mixed"], want, rtol=1e-6, atol=1e-7)


def test_copies_are_averaged():
    """with zero mix weights, copies 0..hc-1 set to distinct multiples of one
    unit-rms vector u give the mean of the normalised copies: every copy
    normalises to u, so mixed = u/2 whatever the multiples"""
    hc, d, R = 4, 64, 64
    t = orc.Hyper(hc, d, R, seed=6).arrays()
    for k in ("down_q", "down_s", "down_b", "up_q", "up_s", "up_b"):
        t[k] = np.zeros_like(t[k])
    w = np.linspace(0.5, 2.0, hc * d).astype(np.float32)
    t["hc_norm"] = w
    hz = orc.Hyper.from_arrays(hc, d, R, t)
    u = np.sign(orc.gen_hyper(1, 1, d, seed=8)).astype(np.float32)  # rms exactly 1
    hyper = np.concatenate([u * 2.0 ** h for h in range(hc)], axis=1)
    m = hz.mix(hyper)
    r = np.float32(1.0) / np.sqrt(np.float32(1.0 + 1e-6))
    want = 0.5 * (u * r * w.reshape(hc, d)).astype(np.float64).mean(0)
    np.testing.assert_allclose(m["mixed"][0], want, rtol=1e-6)


def test_inject_update_is_one_fma():
    hc, d, n = 4, 96, 3
    rng = np.random.default_rng(0)
    hyper = rng.standard_normal((n, hc * d)).astype(np.float32)
    inject = rng.uniform(0, 2, (n, hc)).astype(np.float32)
    out = rng.standard_normal((n, d)).astype(np.float32)
    hp = orc.Hyper(hc, d, 64, seed=0)
    got = hp.inject_update(hyper, inject, out)
    # one rounding of the exact value: within half an ulp of it (a product
    # rounded before the add is off by more for some elements)
    from fractions import Fraction
    got = got.reshape(n, hc, d)
    hv = hyper.reshape(n, hc, d)
    for t in range(n):
        for hh in range(hc):
            for j in range(d):
                exact = Fraction(float(hv[t, hh, j])) + \
                    Fraction(float(inject[t, hh])) * Fraction(float(out[t, j]))
                r = got[t, hh, j]
                assert abs(Fraction(float(r)) - exact) <= Fraction(float(np.spacing(np.abs(r)))) / 2


def test_hyper_generator_is_seeded_and_shaped():
    a = orc.Hyper(4, 128, 64, seed=1, layer=2)
    b = orc.Hyper(4, 128, 64, seed=1, layer=2)
    c = orc.Hyper(4, 128, 64, seed=1, layer=3)
    for k in orc.Hyper.KEYS:
        assert np.array_equal(a.t[k], b.t[k])
    assert not np.array_equal(a.t["down_q"], c.t["down_q"])
    assert a.t["down_q"].size == 64 * 512 // 8 and a.t["up_s"].size == 512 * 64 // 64
    assert a.t["inject_w"].size == 4 * 512 and np.all(a.t["hc_norm"] == 1.0)


def _golden_case():
    """the case of tests/golden/hyper_tiny.npz (make_golden.py:hyper_tiny_case)"""
    L = orc.Layer(256, 8, 2, 128, seed=0)
    a = orc.Hyper(4, 256, 128, seed=0, norm_std=0.2).arrays()
    a["hc_norm"] = orc.bf16_to_f32(orc.f32_to_bf16(a["hc_norm"]))
    return L, orc.Hyper.from_arrays(4, 256, 128, a), orc.gen_hyper(4, 4, 256, seed=0)


def test_golden_hyper_tiny_reproduces():
    import hashlib
    import os
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "hyper_tiny.npz"))
    L, hp, hyper = _golden_case()
    for name, digest in zip(g["weight_names"], g["weight_sha256"]):
        assert hashlib.sha256(np.ascontiguousarray(hp.t[str(name)]).tobytes()).hexdigest() == digest
    assert np.array_equal(hyper, g["hyper_in"])
    r = hp.layer_forward(L, hyper)
    for k in ("mixed", "inject", "moe_out"):
        assert np.array_equal(r[k], g[k]), k
    assert np.array_equal(r["hyper"], g["hyper_out"])
