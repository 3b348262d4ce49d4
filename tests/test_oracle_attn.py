"""Pins of the attention oracle (oracle/attn_oracle.c, the restatement of
c/src/model.c:798-1144):

* a float64 evaluation written from the definitions (masked softmax over
  the cache, RoPE as a rotation of the first rot dims' halves, the indexer's
  pooled-block selection with a sort), dense and past the indexer budget;
* closed form: the first token of an empty cache attends only to itself, so
  out = o_proj(v * sigmoid(gate));
* RoPE's relative-position property: one-token calls at positions p.. and
  at p+37.. give the same outputs (to rounding);
* n tokens in one call equal n one-token calls, bit for bit.
"""
import numpy as np
import pytest

from conftest import load_oracle

orc = load_oracle()


def dequant(q, s, b, rows, cols, g=64):
    q = np.asarray(q, np.uint32).reshape(rows, cols // 8)
    codes = np.stack([(q >> (4 * i)) & 15 for i in range(8)], axis=-1).reshape(rows, cols)
    sc = orc.bf16_to_f32(s).astype(np.float64).reshape(rows, cols // g)
    bi = orc.bf16_to_f32(b).astype(np.float64).reshape(rows, cols // g)
    return codes * np.repeat(sc, g, axis=1) + np.repeat(bi, g, axis=1)


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def rms(x, w):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6) * w


def rope(x, pos, rot, theta):
    """rotate pairs (i, i + rot/2), i < rot/2, by pos * theta^(-2i/rot)"""
    half = rot // 2
    inv = theta ** (-(2.0 * np.arange(half)) / rot)
    ang = np.asarray(pos, np.float64)[..., None] * inv
    c, s = np.cos(ang), np.sin(ang)
    y = x.copy()
    x0, x1 = x[..., :half], x[..., half:rot]
    y[..., :half] = x0 * c - x1 * s
    y[..., half:rot] = x0 * s + x1 * c
    return y


class F64:
    """the mixer in float64 from its definitions, with its own caches"""

    def __init__(self, A):
        self.A, t = A, A.t
        d, h, kvh, hd = A.d, A.h, A.kvh, A.hd
        self.Wq = dequant(t["q_q"], t["q_s"], t["q_b"], 2 * h * hd, d)
        self.Wk = dequant(t["k_q"], t["k_s"], t["k_b"], kvh * hd, d)
        self.Wv = dequant(t["v_q"], t["v_s"], t["v_b"], kvh * hd, d)
        self.Wo = dequant(t["o_q"], t["o_s"], t["o_b"], d, h * hd)
        self.Wi = orc.bf16_to_f32(t["idx_w"]).astype(np.float64).reshape(-1, d)
        self.K = np.zeros((0, kvh, hd))
        self.V = np.zeros((0, kvh, hd))
        self.I = np.zeros((0, A.ihd))

    def forward(self, x, offset, base=0):
        """x at positions offset..; with base > 0 only keys at positions >=
        base (and key blocks starting there) are attended: the sliding
        window stated over the full history"""
        A, t = self.A, self.A.t
        h, kvh, hd, ih, ihd = A.h, A.kvh, A.hd, A.ih, A.ihd
        rot = int(hd * A.rf)
        x = x.astype(np.float64)
        n = x.shape[0]
        pos = offset + np.arange(n)
        qk = x @ self.Wi.T
        self.I = np.concatenate([self.I, qk[:, ih * ihd:]])
        qg = (x @ self.Wq.T).reshape(n, h, 2, hd)
        q = rope(rms(qg[:, :, 0], t["q_norm"]), pos[:, None], rot, A.theta)
        gate = qg[:, :, 1]
        k = rope(rms((x @ self.Wk.T).reshape(n, kvh, hd), t["k_norm"]), pos[:, None], rot, A.theta)
        self.K = np.concatenate([self.K, k])
        self.V = np.concatenate([self.V, (x @ self.Wv.T).reshape(n, kvh, hd)])
        L = self.K.shape[0]
        kk = np.arange(L)
        out = np.zeros((n, h, hd))
        for ti in range(n):
            allowed = (kk <= offset + ti) & (kk >= base)
            if L - base > A.budget:
                c = A.compress
                nb = L // c
                pooled = self.I[:nb * c].reshape(nb, c, ihd).mean(1)
                pooled = rope(rms(pooled, t["idx_k_norm"]), np.arange(nb) * c, rot, A.theta)
                qi = rope(rms(qk[ti, :ih * ihd].reshape(ih, ihd), t["idx_q_norm"]), pos[ti], rot, A.theta)
                sc = np.maximum(qi[:, None, :] * pooled[None], 0).sum((0, 2)) / np.sqrt(ihd)
                sc[np.arange(nb) * c + c - 1 > offset + ti] = -np.inf
                cand = [b for b in range(nb) if b * c >= base]
                order = sorted(cand, key=lambda b: (-sc[b], b))[:A.budget // c]
                keep = np.isin(kk // c, order) & (kk // c < nb)
                own = (offset + ti + 1) // c * c
                keep |= (kk >= own) & (kk <= offset + ti)
                allowed &= keep
            for hh in range(h):
                s = self.K[:, hh % kvh] @ q[ti, hh] / np.sqrt(hd)
                s = np.where(allowed, s, -np.inf)
                p = np.exp(s - s.max())
                p /= p.sum()
                out[ti, hh] = (p @ self.V[:, hh % kvh]) / (1 + np.exp(-gate[ti, hh]))
        return out.reshape(n, h * hd) @ self.Wo.T


CASES = [
    # d, h, kvh, hd, idx heads, idx hd, budget, compress, cap, rotary factor
    (256, 4, 2, 64, 2, 64, 4096, 4, 64, 0.25),   # dense (budget past the cache)
    (256, 4, 2, 64, 2, 64, 8, 2, 64, 0.25),      # the indexer masks from 9 keys on
    (192, 2, 1, 32, 2, 32, 6, 3, 48, 1.0),       # full rotary, one kv head
]


@pytest.mark.parametrize("case", CASES)
def test_oracle_matches_float64_definition(case):
    d, h, kvh, hd, ih, ihd, budget, comp, cap, rf = case
    A = orc.Attention(d, h, kvh, hd, ih, ihd, budget, comp, kv_cap=cap, rotary_factor=rf, seed=2)
    st = A.new_state()
    ref = F64(A)
    x = orc.gen_attn_x(24, d, 3)
    t0 = 0
    for n in (1, 3, 1, 8, 1, 5, 1, 4):
        got = A.forward(x[t0:t0 + n], st, t0)
        exp = ref.forward(x[t0:t0 + n], t0)
        assert rel(got, exp) < 1e-5, (t0, n, rel(got, exp))
        t0 += n


def test_first_token_closed_form():
    A = orc.Attention(256, 4, 2, 64, 2, 64, 4096, 4, kv_cap=16, seed=4)
    x = orc.gen_attn_x(1, 256, 8)
    got = A.forward(x, A.new_state(), 0)
    f = F64(A)
    qg = (x.astype(np.float64) @ f.Wq.T).reshape(4, 2, 64)
    v = (x.astype(np.float64) @ f.Wv.T).reshape(2, 64)
    o = np.stack([v[hh % 2] / (1 + np.exp(-qg[hh, 1])) for hh in range(4)]).reshape(-1)
    assert rel(got[0], o @ f.Wo.T) < 1e-5


def test_rope_relative_positions():
    A = orc.Attention(256, 4, 2, 64, 2, 64, 4096, 4, kv_cap=32, rotary_factor=0.5, seed=5)
    x = orc.gen_attn_x(6, 256, 9)
    s1, s2 = A.new_state(), A.new_state()
    a = np.concatenate([A.forward(x[t:t + 1], s1, t) for t in range(6)])
    b = np.concatenate([A.forward(x[t:t + 1], s2, t + 37) for t in range(6)])
    assert rel(a, b) < 1e-5, rel(a, b)
    # and a rotation that is wrong by a sign would not keep it
    assert rel(a[1:], np.concatenate([A.forward(x[t:t + 1], A.new_state(), 0) for t in range(1, 6)])) > 1e-3


@pytest.mark.parametrize("budget", [4096, 6])
def test_tokens_at_once_equal_one_by_one(budget):
    A = orc.Attention(256, 4, 2, 64, 2, 64, budget, 2, kv_cap=32, seed=6)
    x = orc.gen_attn_x(9, 256, 1)
    s1, s2 = A.new_state(), A.new_state()
    a = np.concatenate([A.forward(x[:4], s1, 0), A.forward(x[4:], s1, 4)])
    b = np.concatenate([A.forward(x[t:t + 1], s2, t) for t in range(9)])
    np.testing.assert_array_equal(a, b)


def test_capacity_refused():
    A = orc.Attention(256, 4, 2, 64, 2, 64, 4096, 4, kv_cap=4, seed=7)
    st = A.new_state()
    A.forward(orc.gen_attn_x(4, 256, 1), st, 0)
    with pytest.raises(ValueError, match="capacity"):
        A.forward(orc.gen_attn_x(1, 256, 2), st, 4)


SLIDE_CASES = [
    # d, h, kvh, hd, idx heads, idx hd, budget, compress, cap, rotary factor
    (256, 4, 2, 64, 2, 64, 8, 2, 16, 0.25),      # the indexer masks inside the window
    (256, 4, 1, 64, 2, 64, 8, 4, 20, 0.5),       # blocks of 4, one kv head
    (192, 2, 1, 32, 2, 32, 4096, 3, 12, 1.0),    # dense window, blocks of 3
]


@pytest.mark.parametrize("case", SLIDE_CASES)
def test_sliding_window_matches_float64(case):
    """past kv_cap the sliding oracle drops the oldest rows of k, v and the
    indexer keys together, compress rows at a time; it must equal the
    float64 mixer over the whole history with every key (and key block)
    before the window's first position masked, where that position is
    round_up(tokens - cap, compress) -- stated here without the oracle's
    bookkeeping.  Calls cross the capacity several times, in chunks and
    one token at a time."""
    d, h, kvh, hd, ih, ihd, budget, comp, cap, rf = case
    A = orc.Attention(d, h, kvh, hd, ih, ihd, budget, comp, kv_cap=cap, rotary_factor=rf, seed=3,
                      slide=True)
    st = A.new_state()
    ref = F64(A)
    x = orc.gen_attn_x(64, d, 4)
    t0 = 0
    for n in (5, 7, 1, 1, 6, 1, 9, 1, 1, 8, 1, 3, 1):
        got = A.forward(x[t0:t0 + n], st, t0)
        total = t0 + n
        base = max(0, -(-(total - cap) // comp) * comp)
        exp = ref.forward(x[t0:t0 + n], t0, base)
        assert st.base == base and st.len == total - base, (t0, n, st.base, st.len, base)
        assert rel(got, exp) < 1e-5, (t0, n, rel(got, exp))
        t0 += n
    assert st.base > 0


def test_sliding_window_refusals():
    A = orc.Attention(256, 4, 2, 64, 2, 64, 4096, 4, kv_cap=8, seed=7, slide=True)
    st = A.new_state()
    A.forward(orc.gen_attn_x(3, 256, 1), st, 0)
    with pytest.raises(ValueError, match="base"):   # positions must continue the window
        A.forward(orc.gen_attn_x(1, 256, 2), st, 5)
    with pytest.raises(ValueError, match="capacity"):  # the drop would exceed the 3 cached rows
        A.forward(orc.gen_attn_x(8, 256, 2), st, 3)
