"""Pins of the DeltaNet oracle (oracle/dn_oracle.c, the restatement of
c/src/model.c:1146-1278):

* a float64 evaluation of the mixer written from its definitions (the conv as
  a sliding window over [state; mixed], the recurrence in outer-product form
  S <- g S + beta (v - g S k) k^T, the norms as vector operations), on the
  dequantised weights;
* the recurrence against transformers' own gated delta rule
  (torch_recurrent_gated_delta_rule, an independent implementation), when
  transformers is importable;
* closed forms: beta = 0 and g = 1 leave the state unchanged and give
  o = S q; a conv with only its newest tap keeps the newest input;
* one call over n tokens equals n one-token calls, bit for bit.
"""
import numpy as np
import pytest

from conftest import load_oracle

orc = load_oracle()


def dequant(q, s, b, rows, cols, g=64):
    """w[r, c] = code * scale + bias (float64), codes low nibble first"""
    q = np.asarray(q, np.uint32).reshape(rows, cols // 8)
    codes = np.stack([(q >> (4 * i)) & 15 for i in range(8)], axis=-1).reshape(rows, cols)
    sc = orc.bf16_to_f32(s).astype(np.float64).reshape(rows, cols // g)
    bi = orc.bf16_to_f32(b).astype(np.float64).reshape(rows, cols // g)
    return codes * np.repeat(sc, g, axis=1) + np.repeat(bi, g, axis=1)


def f64_mixer(D, x, conv_state, rec_state):
    """the mixer in float64 from its definitions; returns out, core, states"""
    t = D.t
    d, hk, hv, dk, dv, kc = D.d, D.hk, D.hv, D.dk, D.dv, D.kc
    kd, vd, cd = D.key_dim, D.value_dim, D.conv_dim
    x = x.astype(np.float64)
    n = x.shape[0]
    mixed = x @ dequant(t["qkv_q"], t["qkv_s"], t["qkv_b"], cd, d).T
    z = x @ dequant(t["z_q"], t["z_s"], t["z_b"], vd, d).T
    a = x @ orc.bf16_to_f32(t["a_w"]).astype(np.float64).reshape(hv, d).T
    b = x @ orc.bf16_to_f32(t["b_w"]).astype(np.float64).reshape(hv, d).T
    seq = np.concatenate([conv_state.astype(np.float64), mixed], axis=0)
    w = orc.bf16_to_f32(t["conv_w"]).astype(np.float64).reshape(cd, kc)
    conv = sum(seq[i:i + n] * w[:, i] for i in range(kc))
    new_conv = seq[n:n + kc - 1].copy()
    act = conv / (1.0 + np.exp(-conv))
    q = act[:, :kd].reshape(n, hk, dk)
    k = act[:, kd:2 * kd].reshape(n, hk, dk)
    v = act[:, 2 * kd:].reshape(n, hv, dv)
    q = q / np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6) / np.sqrt(dk)
    k = k / np.sqrt((k * k).sum(-1, keepdims=True) + 1e-6)
    rep = hv // hk
    S = rec_state.astype(np.float64).copy()
    core = np.zeros((n, hv, dv))
    for ti in range(n):
        for h in range(hv):
            g = np.exp(-np.exp(t["a_log"][h]) * np.log1p(np.exp(a[ti, h] + t["dt_bias"][h])))
            beta = 1.0 / (1.0 + np.exp(-b[ti, h]))
            kk, qq = k[ti, h // rep], q[ti, h // rep]
            Sd = g * S[h]
            S[h] = Sd + beta * np.outer(v[ti, h] - Sd @ kk, kk)
            core[ti, h] = S[h] @ qq
    o = core / np.sqrt((core * core).mean(-1, keepdims=True) + 1e-6) * t["norm_w"].astype(np.float64)
    o = o * (1.0 / (1.0 + np.exp(-z.reshape(n, hv, dv))))
    out = o.reshape(n, vd) @ dequant(t["out_q"], t["out_s"], t["out_b"], d, vd).T
    return out, core.reshape(n, vd), new_conv, S


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


SHAPES = [(256, 2, 4, 64, 64, 4), (128, 1, 2, 32, 128, 3), (192, 2, 2, 32, 32, 2)]


@pytest.mark.parametrize("shape", SHAPES)
def test_oracle_matches_float64_definition(shape):
    d, hk, hv, dk, dv, kc = shape
    D = orc.DeltaNet(d, hk, hv, dk, dv, kc, seed=3)
    cs, rs = D.new_state()
    rng = np.random.default_rng(1)
    cs[:] = rng.normal(0, 2.0, cs.shape)
    rs[:] = rng.normal(0, 0.3, rs.shape)
    x = orc.gen_dn_x(5, d, 7)
    ref = f64_mixer(D, x, cs, rs)
    out, core = D.forward(x, cs, rs, want_core=True)
    assert rel(core, ref[1]) < 1e-5, rel(core, ref[1])
    assert rel(out, ref[0]) < 1e-5, rel(out, ref[0])
    assert rel(cs, ref[2]) < 1e-6  # the newest rows of [state; mixed]
    assert rel(rs, ref[3]) < 1e-5


def test_recurrence_matches_transformers():
    tr = pytest.importorskip("transformers.models.qwen3_next.modeling_qwen3_next")
    torch = pytest.importorskip("torch")
    d, hk, hv, dk, dv, kc = 256, 2, 4, 64, 64, 4
    D = orc.DeltaNet(d, hk, hv, dk, dv, kc, seed=11)
    cs, rs = D.new_state()
    rs[:] = np.random.default_rng(2).normal(0, 0.3, rs.shape)
    rs0 = rs.copy()
    x = orc.gen_dn_x(6, d, 13)
    # q, k, v, g, beta of these tokens from the float64 definition
    t = D.t
    n = x.shape[0]
    mixed = x.astype(np.float64) @ dequant(t["qkv_q"], t["qkv_s"], t["qkv_b"], D.conv_dim, d).T
    a = x.astype(np.float64) @ orc.bf16_to_f32(t["a_w"]).astype(np.float64).reshape(hv, d).T
    b = x.astype(np.float64) @ orc.bf16_to_f32(t["b_w"]).astype(np.float64).reshape(hv, d).T
    w = orc.bf16_to_f32(t["conv_w"]).astype(np.float64).reshape(D.conv_dim, kc)
    seq = np.concatenate([cs.astype(np.float64), mixed])
    conv = sum(seq[i:i + n] * w[:, i] for i in range(kc))
    act = conv / (1.0 + np.exp(-conv))
    rep = hv // hk
    q = np.repeat(act[:, :D.key_dim].reshape(n, hk, dk), rep, axis=1)
    k = np.repeat(act[:, D.key_dim:2 * D.key_dim].reshape(n, hk, dk), rep, axis=1)
    v = act[:, 2 * D.key_dim:].reshape(n, hv, dv)
    g = -np.exp(t["a_log"].astype(np.float64)) * np.log1p(np.exp(a + t["dt_bias"]))
    beta = 1.0 / (1.0 + np.exp(-b))
    T = lambda arr: torch.from_numpy(np.ascontiguousarray(arr, dtype=np.float64))[None]
    init = torch.from_numpy(rs0.astype(np.float64).transpose(0, 2, 1).copy())[None]
    o, fin = tr.torch_recurrent_gated_delta_rule(T(q), T(k), T(v), T(g), T(beta), init, True,
                                                use_qk_l2norm_in_kernel=True)
    o = o[0].numpy().reshape(n, hv * dv)  # [T, H, dv]
    fin = fin[0].numpy().transpose(0, 2, 1)
    _, core = D.forward(x, cs, rs, want_core=True)
    assert rel(core, o) < 1e-4, rel(core, o)
    assert rel(rs, fin) < 1e-4, rel(rs, fin)


def test_closed_forms():
    d, hk, hv, dk, dv, kc = 128, 1, 2, 32, 32, 4
    D = orc.DeltaNet(d, hk, hv, dk, dv, kc, seed=5)
    arr = D.arrays()
    # beta = sigmoid(-inf) = 0 and g = exp(-exp(-100) softplus(.)) = 1
    arr["b_w"] = np.full_like(arr["b_w"], orc.f32_to_bf16(np.float32(-100.0)))
    arr["a_log"] = np.full_like(arr["a_log"], -100.0)
    # conv with only its newest tap, weight 1
    cw = np.zeros((D.conv_dim, kc), np.float32)
    cw[:, kc - 1] = 1.0
    arr["conv_w"] = orc.f32_to_bf16(cw).reshape(-1)
    E = orc.DeltaNet.from_arrays(d, hk, hv, dk, dv, kc, arr)
    cs, rs = E.new_state()
    rng = np.random.default_rng(3)
    cs[:] = rng.normal(0, 1.0, cs.shape)
    rs[:] = rng.normal(0, 0.5, rs.shape)
    rs0 = rs.copy()
    x = np.ones((1, d), np.float32)
    _, core = E.forward(x, cs, rs, want_core=True)
    np.testing.assert_array_equal(rs, rs0)  # S unchanged
    # o = S q with q = l2norm(silu(mixed_q)) / sqrt(dk): the newest tap only
    mixed = x.astype(np.float64) @ dequant(arr["qkv_q"], arr["qkv_s"], arr["qkv_b"], E.conv_dim, d).T
    qa = mixed[0, :dk] / (1 + np.exp(-mixed[0, :dk]))
    qa = qa / np.sqrt((qa * qa).sum() + 1e-6) / np.sqrt(dk)
    exp = np.concatenate([rs0[h].astype(np.float64) @ qa for h in range(hv)])
    assert rel(core[0], exp) < 1e-5


def test_tokens_at_once_equal_one_by_one():
    D = orc.DeltaNet(256, 2, 4, 64, 64, 4, seed=9)
    x = orc.gen_dn_x(4, 256, 3)
    cs1, rs1 = D.new_state()
    all_at_once = D.forward(x, cs1, rs1)
    cs2, rs2 = D.new_state()
    steps = np.concatenate([D.forward(x[t:t + 1], cs2, rs2) for t in range(4)])
    np.testing.assert_array_equal(all_at_once, steps)
    np.testing.assert_array_equal(cs1, cs2)
    np.testing.assert_array_equal(rs1, rs2)
