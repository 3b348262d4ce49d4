"""Pins of the CPU oracle (oracle/moe_oracle.c) -- CPU only.

Every oracle function is checked against something other than itself:
the reference's own known-answer vectors and tolerance tests
(c/tests/test_kernel.c), the reference's own compiled bf16 helpers
(oracle/_ref, built from c/src/util.h), closed forms, brute force, an
independent float64 numpy restatement, and transformers' Qwen3Next MoE block
(a third-party statement of the same router/expert/shared-gate semantics).
"""
import numpy as np
import pytest

from conftest import load_oracle

orc = load_oracle()


# ------------------------------------------------------------ helpers

def lcg_frand(state, count):
    """frand of c/tests/test_kernel.c:9-12 (64-bit LCG, 16 bits -> [-0.5,0.5))"""
    out = np.empty(count, np.float32)
    s = state
    for i in range(count):
        s = (s * 6364136223846793005 + 1442695040888963407) & 0xFFFFFFFFFFFFFFFF
        out[i] = np.float32(((s >> 33) & 0xFFFF) / 65536.0 - 0.5)
    return out, s


def close_enough(a, b, tol):
    """c/tests/test_kernel.c:14-16"""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return np.abs(a - b) <= tol * (1.0 + np.abs(a) + np.abs(b))


def mlx_quantize_group(wg):
    """the MLX-style affine quantiser of c/tests/test_kernel.c:155-184"""
    gmn, gmx = np.float32(wg.min()), np.float32(wg.max())
    scale = np.float32(max((gmx - gmn) / np.float32(15.0), np.float32(1e-7)))
    side = abs(gmn) > abs(gmx)
    scale = scale if side else -scale
    edge = gmn if side else gmx
    q0 = np.float32(np.round(edge / scale))
    if q0 != 0:
        scale = np.float32(edge / q0)
    bias = np.float32(0.0) if q0 == 0 else np.float32(edge)
    v = np.clip(np.minimum(np.round((wg - bias) / scale), 15), 0, None).astype(np.uint32)
    return v, scale, bias


def pack_nibbles(codes):
    codes = np.asarray(codes, np.uint32).reshape(-1, 8)
    w = np.zeros(codes.shape[0], np.uint32)
    for i in range(8):
        w |= codes[:, i] << np.uint32(4 * i)
    return w


def fma32(a, b, c):
    """correctly rounded fma for float32 operands via float64 (exact here:
    the operands are small codes / bf16 / f32 whose product and sum fit)"""
    return (np.float64(a) * np.float64(b) + np.float64(c)).astype(np.float32)


# ------------------------------------------------------------ bf16

def test_bf16_widen_all_patterns():
    # widening is a 16-bit shift (util.h:56-61): every pattern, bit-exact
    lib = orc.lib()
    for h in list(range(0, 65536, 97)) + [0, 0x8000, 0x7F80, 0xFF80, 0x3F80, 0xFFFF]:
        got = np.float32(lib.orc_bf16_to_f32(h)).view(np.uint32)
        assert int(got) == (h << 16) or (np.isnan(np.float32(lib.orc_bf16_to_f32(h))))


def test_bf16_rne_is_nearest_with_ties_to_even():
    # the narrowing is round-to-nearest-even (util.h:63-71): check against the
    # definition -- nearest representable value, exact ties to an even mantissa
    rng = np.random.default_rng(1)
    xs = rng.standard_normal(20000).astype(np.float32) * np.float32(37.0)
    lib = orc.lib()
    for x in xs[:4000]:
        b = lib.orc_f32_to_bf16(float(x))
        v = orc.bf16_to_f32(np.array([b]))[0]
        lo = orc.bf16_to_f32(np.array([b - 1]))[0]
        hi = orc.bf16_to_f32(np.array([b + 1]))[0]
        d = abs(np.float64(x) - np.float64(v))
        assert d <= abs(np.float64(x) - np.float64(lo)) and d <= abs(np.float64(x) - np.float64(hi))
    # exact ties: bits ...8000 round to the even neighbour
    for hi16 in (0x3F80, 0x3F81, 0x4000, 0xC123, 0x0001):
        bits = np.array([(hi16 << 16) | 0x8000], np.uint32)
        x = bits.view(np.float32)[0]
        b = lib.orc_f32_to_bf16(float(x))
        assert b == (hi16 if hi16 % 2 == 0 else hi16 + 1)
    # the vectorised numpy twin used by the tests agrees
    np.testing.assert_array_equal(orc.f32_to_bf16(xs),
                                  np.array([lib.orc_f32_to_bf16(float(v)) for v in xs], np.uint16))


def test_bf16_matches_reference_util_h():
    """against the reference's own util.h, compiled from the reference
    checkout into oracle/_ref (skipped where the reference is absent)"""
    ref = orc.ref_util()
    if ref is None:
        pytest.skip("oracle/_ref/libref_util.so not built (no reference checkout)")
    lib = orc.lib()
    rng = np.random.default_rng(7)
    xs = np.concatenate([rng.standard_normal(5000).astype(np.float32) * 100,
                         rng.integers(0, 2**32, 5000, dtype=np.uint64).astype(np.uint32).view(np.float32)])
    for x in xs:
        if np.isnan(x):
            continue
        assert lib.orc_f32_to_bf16(float(x)) == ref.ref_f32_to_bf16(float(x))
    for h in range(0, 65536, 13):
        a, b = lib.orc_bf16_to_f32(h), ref.ref_bf16_to_f32(h)
        assert (a == b) or (np.isnan(a) and np.isnan(b))


# ------------------------------------------------------------ dequant KATs

def test_dequant_mlx_known_answers():
    """c/tests/test_kernel.c:122-141 (vectors from mlx 0.32.2)"""
    q = np.array([0x43322110, 0, 0, 0], np.uint32)
    s = np.array([2.0], np.float32)
    b = np.array([-16.0], np.float32)
    out = orc.dequant_q4_f32sb(q, s, b, 1, 32, 32)[0]
    np.testing.assert_array_equal(out[:8], [-16, -14, -14, -12, -12, -10, -10, -8])
    q2 = np.array([0x76543210, 0, 0, 0], np.uint32)
    out2 = orc.dequant_q4_f32sb(q2, s, b, 1, 32, 32)[0]
    assert out2[0] == -16 and out2[1] == -14 and out2[2] == -12
    assert out2[6] == -4 and out2[7] == -2


def test_dequant_mlx_roundtrip_exact():
    """c/tests/test_kernel.c:143-187: quantise with the MLX rule, dequantise,
    and require exactly q*scale+bias (one rounding, as the contracted
    expression of kernel.c:167-168)"""
    w, _ = lcg_frand(23, 128)
    w = w * np.float32(8)
    codes, scales, biases, ref = [], [], [], []
    for g in range(2):
        v, sc, bi = mlx_quantize_group(w[g * 64:(g + 1) * 64])
        codes.append(v)
        scales.append(sc)
        biases.append(bi)
        ref.append(fma32(v.astype(np.float32), sc, bi))
    q = pack_nibbles(np.concatenate(codes))
    out = orc.dequant_q4_f32sb(q, np.array(scales), np.array(biases), 2, 64, 64)
    np.testing.assert_array_equal(out.reshape(-1), np.concatenate(ref))


def test_nibble_order_low_first():
    # kernel.h:46-50: 8 nibbles per u32, low nibble first
    codes = np.arange(64) % 16
    q = pack_nibbles(codes)
    out = orc.dequant_q4_f32sb(q, np.ones(1, np.float32), np.zeros(1, np.float32), 1, 64, 64)[0]
    np.testing.assert_array_equal(out, codes.astype(np.float32))


# ------------------------------------------------------------ gemms

def test_gemm_fp32_vs_naive():
    """c/tests/test_kernel.c:189-203"""
    A, s = lcg_frand(29, 5 * 33)
    W, _ = lcg_frand(s, 7 * 33)
    A, W = A.reshape(5, 33), W.reshape(7, 33)
    C = orc.gemm_fp32(A, W)
    assert close_enough(C, A.astype(np.float64) @ W.astype(np.float64).T, 1e-5).all()


def test_gemm_bf16_vs_naive():
    """c/tests/test_kernel.c:205-220"""
    A, s = lcg_frand(31, 5 * 129)
    Wf, _ = lcg_frand(s, 7 * 129)
    Wb = orc.f32_to_bf16(Wf).reshape(7, 129)
    C = orc.gemm_bf16(A.reshape(5, 129), Wb)
    ref = A.reshape(5, 129).astype(np.float64) @ orc.bf16_to_f32(Wb).astype(np.float64).T
    assert close_enough(C, ref, 2e-3).all()


def test_gemm_q4_vs_dequant_sgemm():
    """c/tests/test_kernel.c:222-269: gemm_q4 == dequant + sgemm at 1e-4"""
    M, N, K = 4, 9, 256
    A, s = lcg_frand(37, M * K)
    A = (A * 2).reshape(M, K)
    scales = np.empty(N * 4, np.float32)
    biases = np.empty(N * 4, np.float32)
    for n in range(N):
        vals, s = lcg_frand(s, 256)
        vals = vals * 4
        mn, mx = np.float32(1e30), np.float32(-1e30)
        for g in range(4):
            mn = min(mn, vals[g * 64:(g + 1) * 64].min())
            mx = max(mx, vals[g * 64:(g + 1) * 64].max())
            scale = np.float32(max((mx - mn) / np.float32(15.0), np.float32(1e-7)))
            side = abs(mn) > abs(mx)
            scale = scale if side else -scale
            edge = mn if side else mx
            q0 = np.float32(np.round(edge / scale))
            if q0 != 0:
                scale = np.float32(edge / q0)
            scales[n * 4 + g] = scale
            biases[n * 4 + g] = 0.0 if q0 == 0 else edge
    codes = np.empty(N * K, np.uint32)
    for n in range(N):
        for g in range(4):
            sc, bi = scales[n * 4 + g], biases[n * 4 + g]
            v, s = lcg_frand(s, 64)
            v = v * 4
            codes[n * K + g * 64:n * K + (g + 1) * 64] = np.clip(
                np.minimum(np.round((v - bi) / sc), 15), 0, None).astype(np.uint32)
    W = pack_nibbles(codes)
    C = orc.gemm_q4_f32sb(A, W, scales, biases, N, K, 64)
    Wd = orc.dequant_q4_f32sb(W, scales, biases, N, K, 64)
    ref = orc.gemm_fp32(A, Wd)
    assert close_enough(C, ref, 1e-4).all()
    # and against float64 ground truth
    exact = A.astype(np.float64) @ Wd.astype(np.float64).T
    assert close_enough(C, exact, 1e-4).all()


def test_gemm_q4_identity_catches_dropped_bias():
    # a q4 GEMM without the b*sum(x) term must fail this check
    rng = np.random.default_rng(3)
    N, K = 6, 128
    A = rng.standard_normal((3, K)).astype(np.float32)
    W = rng.integers(0, 2**32, N * K // 8, dtype=np.uint64).astype(np.uint32)
    sc = rng.standard_normal(N * 2).astype(np.float32) * 0.02
    bi = rng.standard_normal(N * 2).astype(np.float32) * 0.5
    C = orc.gemm_q4_f32sb(A, W, sc, bi, N, K, 64)
    exact = A.astype(np.float64) @ orc.dequant_q4_f32sb(W, sc, bi, N, K, 64).astype(np.float64).T
    np.testing.assert_allclose(C, exact, rtol=1e-5, atol=1e-4)
    C0 = orc.gemm_q4_f32sb(A, W, sc, np.zeros_like(bi), N, K, 64)
    assert np.abs(C0 - exact).max() > 1e-2


# ------------------------------------------------------------ top-k

@pytest.mark.parametrize("k", [1, 3, 10, 64, 512])
def test_topk_invariants(k):
    """c/tests/test_kernel.c:95-120 for both the quickselect restatement and
    the canonical order"""
    x, _ = lcg_frand(17, 512)
    x = x * 10
    for fn in (orc.topk_quickselect, orc.topk_canonical):
        idx = fn(x, k)
        assert len(idx) == k and len(set(idx.tolist())) == k
        assert ((idx >= 0) & (idx < 512)).all()
        used = np.zeros(512, bool)
        used[idx] = True
        chosen_min = x[idx].min()
        unchosen_max = x[~used].max() if k < 512 else -1e30
        assert chosen_min >= unchosen_max - 1e-6


def test_topk_canonical_brute_force_with_ties():
    rng = np.random.default_rng(11)
    for trial in range(200):
        E = int(rng.integers(2, 600))
        k = int(rng.integers(1, min(E, 64) + 1))
        # few distinct values -> many exact ties, plus signed zeros
        x = rng.integers(-4, 5, E).astype(np.float32) * np.float32(0.25)
        x[rng.random(E) < 0.1] = np.float32(-0.0)
        got = orc.topk_canonical(x, k)
        order = np.lexsort((np.arange(E), -(x.astype(np.float64) + 0.0)))
        np.testing.assert_array_equal(got, order[:k])


def test_quickselect_same_set_without_boundary_tie():
    rng = np.random.default_rng(5)
    for trial in range(300):
        x = rng.standard_normal(512).astype(np.float32)
        k = 10
        srt = np.sort(x)[::-1]
        if srt[k - 1] == srt[k]:
            continue
        assert set(orc.topk_quickselect(x, k).tolist()) == set(orc.topk_canonical(x, k).tolist())


# ------------------------------------------------------------ R64 / rmsnorm

def test_r64_dot_exact_on_integers_and_close_on_reals():
    rng = np.random.default_rng(2)
    for K in (64, 256, 2048, 2560):
        # small integers: every partial sum is exact, so any correct order
        # must give the exact sum -- a dropped or doubled chunk fails
        xi = rng.integers(-8, 9, K).astype(np.float32)
        wi = rng.integers(-8, 9, K).astype(np.float32)
        got = orc.dot_r64(xi, orc.f32_to_bf16(wi))
        assert got == float(np.dot(xi.astype(np.int64), wi.astype(np.int64)))
        x = rng.standard_normal(K).astype(np.float32)
        wb = orc.f32_to_bf16(rng.standard_normal(K).astype(np.float32) * 0.02)
        exact = np.dot(x.astype(np.float64), orc.bf16_to_f32(wb).astype(np.float64))
        bound = K * np.finfo(np.float32).eps * np.dot(np.abs(x), np.abs(orc.bf16_to_f32(wb)))
        assert abs(orc.dot_r64(x, wb) - exact) <= bound
        assert abs(orc.sumsq_r64(x) - np.dot(x.astype(np.float64), x)) <= K * 1.2e-7 * np.dot(x, x)


def test_rmsnorm_closed_form():
    """c/tests/test_kernel.c:18-30 (sequential and R64 sums)"""
    x, s = lcg_frand(7, 257 * 2)
    x, w = x[0::2].copy(), x[1::2] + np.float32(1.0)
    xd = x.astype(np.float64)
    r = 1.0 / np.sqrt(np.dot(xd, xd) / 257.0 + 1e-6)
    ref = xd * r * w
    for r64 in (False, True):
        y = orc.rmsnorm(x, w, 1e-6, r64=r64)
        assert close_enough(y, ref, 1e-6).all()


def test_silu_sigmoid_closed_form():
    lib = orc.lib()
    for v in np.linspace(-20, 20, 81, dtype=np.float32):
        vd = float(v)
        assert abs(lib.orc_silu(vd) - vd / (1 + np.exp(-vd))) <= 1e-6 * (1 + abs(vd))
        assert abs(lib.orc_sigmoid(vd) - 1 / (1 + np.exp(-vd))) <= 1e-7


# ------------------------------------------------------------ dispatch

@pytest.mark.parametrize("n,k,E", [(1, 10, 512), (4, 2, 8), (64, 10, 512), (300, 8, 64),
                                   (4096, 10, 512), (17, 64, 1024)])
def test_dispatch_is_stable_counting_sort(n, k, E):
    rng = np.random.default_rng(n * 7 + k)
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(n)]).astype(np.int32)
    d = orc.dispatch(idx, E)
    flat = idx.reshape(-1)
    np.testing.assert_array_equal(d["perm"], np.argsort(flat, kind="stable"))
    np.testing.assert_array_equal(d["offsets"], np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=E))]))
    np.testing.assert_array_equal(d["unique"], np.unique(flat))
    np.testing.assert_array_equal(d["pos"][d["perm"]], np.arange(n * k))
    # tokens ascending inside every expert (the MLX order, model.py:433-441)
    for e in d["unique"][:20]:
        toks = d["perm"][d["offsets"][e]:d["offsets"][e + 1]] // k
        assert (np.diff(toks) > 0).all()


# ------------------------------------------------------------ whole layer

def numpy_layer_f64(L, x, idx, w, sg):
    """independent float64 restatement of model.c:1338-1403 given the
    routing: dequantise every used expert, SwiGLU, weighted combine, shared"""
    H, I, g = L.H, L.I, L.g
    t = L.t
    out = np.zeros((x.shape[0], H))
    xd = x.astype(np.float64)

    def deq(q, s, b, rows, cols, base_q, base_s):
        qq = q[base_q: base_q + rows * cols // 8]
        codes = ((qq[:, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(rows, cols)
        sc = orc.bf16_to_f32(s[base_s: base_s + rows * cols // g]).reshape(rows, cols // g)
        bi = orc.bf16_to_f32(b[base_s: base_s + rows * cols // g]).reshape(rows, cols // g)
        return codes * np.repeat(sc, g, 1).astype(np.float64) + np.repeat(bi, g, 1)

    def ffn(e, xr):
        if e is None:
            Wg = deq(t["sh_gate_q"], t["sh_gate_s"], t["sh_gate_b"], I, H, 0, 0)
            Wu = deq(t["sh_up_q"], t["sh_up_s"], t["sh_up_b"], I, H, 0, 0)
            Wd = deq(t["sh_down_q"], t["sh_down_s"], t["sh_down_b"], H, I, 0, 0)
        else:
            qo, so = e * I * H // 8, e * I * H // g
            Wg = deq(t["gate_q"], t["gate_s"], t["gate_b"], I, H, qo, so)
            Wu = deq(t["up_q"], t["up_s"], t["up_b"], I, H, qo, so)
            Wd = deq(t["down_q"], t["down_s"], t["down_b"], H, I, qo, so)
        gg, uu = Wg @ xr, Wu @ xr
        return Wd @ (gg / (1 + np.exp(-gg)) * uu)

    for tt in range(x.shape[0]):
        for s in range(L.k):
            out[tt] += w[tt, s] * ffn(int(idx[tt, s]), xd[tt])
        out[tt] += sg[tt] * ffn(None, xd[tt])
    return out


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)


def test_tiny_layer_vs_float64_restatement():
    L = orc.Layer(256, 8, 2, 128, seed=0)
    x = orc.gen_x(4, 256, 0, bf16=False)
    r = L.forward(x, False)
    ref = numpy_layer_f64(L, x, r["idx"], r["w"].astype(np.float64), r["shared_gate"].astype(np.float64))
    assert np.abs(r["out"] - ref).max() < 1e-4 * max(1.0, np.abs(ref).max())
    # the router part: softmax over all E, top-k, renormalise (model.c:1305-1318)
    xd = x.astype(np.float64)
    logits = xd @ orc.bf16_to_f32(L.t["router_w"]).reshape(8, 256).astype(np.float64).T
    for tt in range(4):
        sel = np.argsort(-logits[tt], kind="stable")[:2]
        np.testing.assert_array_equal(np.sort(r["idx"][tt]), np.sort(sel))
        p = np.exp(logits[tt] - logits[tt].max())
        p /= p.sum()
        np.testing.assert_allclose(r["w"][tt], p[r["idx"][tt]] / p[r["idx"][tt]].sum(), rtol=1e-5)
        gl = xd[tt] @ orc.bf16_to_f32(L.t["sh_gate_w"]).astype(np.float64)
        assert abs(r["shared_gate"][tt] - 1 / (1 + np.exp(-gl))) < 1e-6


def test_tiny_layer_vs_transformers_qwen3next_block():
    """third-party statement of the same semantics: transformers'
    Qwen3NextSparseMoeBlock (softmax over all experts, top-k, renormalise,
    SwiGLU experts, sigmoid-gated shared expert) on the dequantised weights"""
    torch = pytest.importorskip("torch")
    try:
        from transformers.models.qwen3_next.configuration_qwen3_next import Qwen3NextConfig
        from transformers.models.qwen3_next.modeling_qwen3_next import Qwen3NextSparseMoeBlock
    except Exception as e:  # pragma: no cover
        pytest.skip(f"transformers qwen3_next unavailable: {e}")
    H, E, k, I = 256, 8, 2, 128
    L = orc.Layer(H, E, k, I, seed=0)
    x = orc.gen_x(4, H, 0, bf16=False)
    r = L.forward(x, False)
    cfg = Qwen3NextConfig(hidden_size=H, num_experts=E, num_experts_per_tok=k,
                          moe_intermediate_size=I, shared_expert_intermediate_size=I,
                          norm_topk_prob=True, hidden_act="silu")
    blk = Qwen3NextSparseMoeBlock(cfg).double()
    t = L.t

    def deq(q, s, b, rows, cols, e=0):
        qn, sn = rows * cols // 8, rows * cols // 64
        return orc.dequant_q4_f32sb(q[e * qn:(e + 1) * qn], orc.bf16_to_f32(s[e * sn:(e + 1) * sn]),
                                    orc.bf16_to_f32(b[e * sn:(e + 1) * sn]), rows, cols, 64)

    with torch.no_grad():
        blk.gate.weight.copy_(torch.from_numpy(orc.bf16_to_f32(t["router_w"]).reshape(E, H).astype(np.float64)))
        for e in range(E):
            g = deq(t["gate_q"], t["gate_s"], t["gate_b"], I, H, e)
            u = deq(t["up_q"], t["up_s"], t["up_b"], I, H, e)
            blk.experts.gate_up_proj[e].copy_(torch.from_numpy(np.concatenate([g, u]).astype(np.float64)))
            blk.experts.down_proj[e].copy_(torch.from_numpy(
                deq(t["down_q"], t["down_s"], t["down_b"], H, I, e).astype(np.float64)))
        blk.shared_expert.gate_proj.weight.copy_(torch.from_numpy(deq(t["sh_gate_q"], t["sh_gate_s"], t["sh_gate_b"], I, H).astype(np.float64)))
        blk.shared_expert.up_proj.weight.copy_(torch.from_numpy(deq(t["sh_up_q"], t["sh_up_s"], t["sh_up_b"], I, H).astype(np.float64)))
        blk.shared_expert.down_proj.weight.copy_(torch.from_numpy(deq(t["sh_down_q"], t["sh_down_s"], t["sh_down_b"], H, I).astype(np.float64)))
        blk.shared_expert_gate.weight.copy_(torch.from_numpy(orc.bf16_to_f32(t["sh_gate_w"]).reshape(1, H).astype(np.float64)))
        ref = blk(torch.from_numpy(x.astype(np.float64)).reshape(1, 4, H)).reshape(4, H).numpy()
    assert np.abs(r["out"] - ref).max() < 2e-4 * max(1.0, np.abs(ref).max())
    assert rel_l2(r["out"], ref) < 1e-5


def test_prefill_equals_token_by_token():
    """c/tests/test_model.c:300-333 idea: the layer is per-token, so a batch
    equals its tokens run one at a time (bit-identical in the oracle)"""
    L = orc.Layer(256, 8, 2, 128, seed=3)
    x = orc.gen_x(6, 256, 3, bf16=True)
    full = L.forward(x, True)["out"]
    for tt in range(6):
        np.testing.assert_array_equal(L.forward(x[tt:tt + 1], True)["out"][0], full[tt])
    sel = L.forward(x, True, token_sel=[5, 1])["out"]
    np.testing.assert_array_equal(sel, full[[5, 1]])


def test_residual_and_norm_options():
    L = orc.Layer(256, 8, 2, 128, seed=4, with_norm=True, router_bias=np.linspace(-1, 1, 8))
    x = orc.gen_x(3, 256, 4, bf16=False)
    base = L.forward(x, False)["out"]
    res = L.forward(x, False, residual=True)["out"]
    np.testing.assert_array_equal(res, x + base)
    rt = L.route(x, False)
    for tt in range(3):
        np.testing.assert_array_equal(rt["xn"][tt], orc.rmsnorm(x[tt], np.ones(256, np.float32), 1e-6))
        lg = np.array([orc.dot_r64(rt["xn"][tt], L.t["router_w"][e * 256:(e + 1) * 256])
                       for e in range(8)], np.float32) + L.t["router_bias"]
        np.testing.assert_array_equal(rt["logits"][tt], lg)


# ------------------------------------------------------------ generators

def test_generator_distributions():
    n = 200000
    b = orc.bf16_to_f32(orc.gen_bf16(n, 0, 0, "GATE_S", 0.02))
    assert abs(b.mean()) < 3e-4 and abs(b.std() - 0.02) < 3e-4
    f = orc.gen_f32(n, 1, 2, "X", 1.0)
    assert abs(f.mean()) < 0.01 and abs(f.std() - 1.0) < 0.01
    c = orc.gen_codes(n // 8, 0, 0, "GATE_Q")
    nib = ((c[:, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(-1)
    counts = np.bincount(nib, minlength=16)
    assert counts.min() > 0.9 * n / 16 and counts.max() < 1.1 * n / 16
    # different tags/layers/seeds give different streams; the same key repeats
    assert not np.array_equal(orc.gen_codes(64, 0, 0, "GATE_Q"), orc.gen_codes(64, 0, 0, "UP_Q"))
    assert not np.array_equal(orc.gen_codes(64, 0, 0, "GATE_Q"), orc.gen_codes(64, 0, 1, "GATE_Q"))
    np.testing.assert_array_equal(orc.gen_codes(64, 5, 0, "GATE_Q")[10:],
                                  orc.gen_codes(54, 5, 0, "GATE_Q", start=10))


def test_zipf_bias():
    b = orc.zipf_bias(512, 1.1, 1.0, 0)
    p = np.exp(b.astype(np.float64))
    assert abs(p.sum() - 1.0) < 1e-5
    ranks = np.sort(p)[::-1]
    r = np.arange(1, 513, dtype=np.float64)
    np.testing.assert_allclose(ranks, r ** -1.1 / (r ** -1.1).sum(), rtol=1e-5)


def test_warm_fp32_mode_matches_faithful():
    """the CPU baseline's weight mode (i) -- warm fp32-dequantised experts,
    sgemm-blocked fp32 products -- computes the same layer as the faithful
    oracle (fp32 dequant + one fma chain per dot) up to fp32 summation
    order, and refuses a routed expert it does not hold"""
    import pytest
    for (H, E, k, I, n, bf, zipf) in ((256, 8, 2, 128, 4, False, 0.0), (512, 64, 6, 128, 40, True, 1.1)):
        rb = orc.zipf_bias(E, zipf, 1.0, 3) if zipf else None
        x = orc.gen_x(n, H, 3, bf16=bf)
        r = orc.Layer(H, E, k, I, seed=1, router_bias=rb, only_experts=[]).route(x, bf)
        L = orc.Layer(H, E, k, I, seed=1, router_bias=rb, only_experts=r["idx"].reshape(-1))
        ref = L.forward(x, bf)["out"]
        W = orc.Warm(L, r["idx"].reshape(-1))
        got = W.forward(x, bf)
        assert W.nbytes == len(set(r["idx"].reshape(-1).tolist())) * 3 * I * H * 4
        rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        assert np.abs(got - ref).max() < 1e-3 * np.abs(ref).max() and rel < 1e-5, rel
        # residual form
        got_r = W.forward(x, bf, residual=True)
        xf = orc.bf16_to_f32(x) if bf else x
        np.testing.assert_allclose(got_r, xf + got, rtol=1e-6, atol=1e-4)
        W.close()
        partial = orc.Warm(L, r["idx"].reshape(-1)[:1])
        with pytest.raises(RuntimeError, match="not in the warm set"):
            partial.forward(x, bf)
        partial.close()
