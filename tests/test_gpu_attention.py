"""The HIP full-attention mixer with the QSA indexer (qmoe_attn_*, through
the C ABI) against the oracle (oracle/attn_oracle.c, pinned by
tests/test_oracle_attn.py).

Bar: per call, outputs within 2e-2 max-abs and 1e-3 relative L2 of the
oracle run on the same weights and inputs from the same caches; the k and v
caches within 1e-4 relative L2.  The indexer path is index work and is
compared bit for bit: the raw indexer-key cache, the pooled block keys, the
block scores of every token (as order keys) and the kept-block set over
each token's visible blocks.  Dense (budget past the cache) and sparse (the
QSA block mask active) cases, several shapes, prefill chunks of up to 2048
tokens and one-token steps, up to 6,000+ cached keys with the mask on.
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


def d2h(ptr, shape, dtype=np.float32):
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
    buf = np.empty(shape, dtype)
    assert _hip.hipMemcpy(ctypes.c_void_p(buf.ctypes.data), ctypes.c_void_p(ptr),
                          ctypes.c_size_t(buf.nbytes), 2) == 0
    return buf


@pytest.fixture(scope="module")
def torch_dev(gpu):
    import torch
    return torch, gpu


def ordkeys(v):
    """float32 -> the kernels' order keys (-0 as +0)"""
    b = (np.asarray(v, np.float32) + np.float32(0.0)).view(np.uint32)
    return np.where(b & 0x80000000, ~b, b | 0x80000000).astype(np.uint32)


def check_index(ctx, dbg, case, n, t0, ln):
    """the indexer's values of the last call against the oracle's, bit for
    bit: pooled keys, every token's block scores and kept blocks (exact
    ties at the budget boundary to the lower block on both sides).  Returns
    the number of tokens whose boundary is such a tie among the blocks the
    token can see."""
    d, h, kvh, hd, ih, ihd, budget, comp, cap, rf = case
    nb, btop = ln // comp, budget // comp
    pp, kp, kw, sp, ld = ctx.index_state(1)
    pooled = d2h(pp, (nb, ihd))
    assert np.array_equal(pooled.view(np.uint32), dbg["pooled"].view(np.uint32)), \
        ("pooled keys", int((pooled != dbg["pooled"]).sum()))
    skey = d2h(sp, (n, ld), np.uint32)[:, :nb]
    okey = ordkeys(dbg["scores"])
    bad = np.argwhere(skey != okey)
    assert bad.size == 0, ("block scores differ", bad[:5].tolist(), int(len(bad)))
    bits = d2h(kp, (n, kw), np.uint32)
    keep = ((bits[:, np.arange(nb) // 32] >> (np.arange(nb) % 32).astype(np.uint32)) & 1).astype(bool)
    bad = np.argwhere(keep != dbg["keep"].astype(bool))
    assert bad.size == 0, ("kept blocks differ", bad[:8].tolist(), int(len(bad)))
    ties = 0
    for t in range(n):
        vis = (np.arange(nb) * comp + comp - 1) <= t0 + t
        sc = dbg["scores"][t][vis]
        if btop < sc.size:
            srt = np.sort(sc)[::-1]
            ties += int(srt[btop - 1] == srt[btop])
    return ties


def run_calls(torch, dev, case, calls, seed=1, slide=False):
    d, h, kvh, hd, ih, ihd, budget, comp, cap, rf = case
    pkg = load_pkg()
    A = orc.Attention(d, h, kvh, hd, ih, ihd, budget, comp, kv_cap=cap, rotary_factor=rf, seed=seed,
                      slide=slide)
    st = A.new_state()
    x = orc.gen_attn_x(sum(calls), d, seed + 50)
    masked = 0
    with pkg.AttentionContext(d, h, kvh, hd, ih, ihd, budget, comp, kv_cap=cap, rotary_factor=rf,
                              n_layers=2, max_tokens=max(calls), slide=slide,
                              max_position=sum(calls) if slide else 0) as ctx:
        ctx.upload_layer(1, A.arrays())
        t0 = 0
        for i, n in enumerate(calls):
            ref, dbg = A.forward(x[t0:t0 + n], st, t0, dbg=True)
            got = ctx.forward(1, torch.from_numpy(x[t0:t0 + n]).to(dev), t0)
            torch.cuda.synchronize()
            g = got.cpu().numpy()
            err, r = float(np.abs(g - ref).max()), rel(g, ref)
            kp, vp, ip, ln = ctx.cache(1)
            assert ln == st.len and (slide or ln == t0 + n), (ln, st.len, t0 + n)
            kc = d2h(kp, (ln, kvh * hd))
            vc = d2h(vp, (ln, kvh * hd))
            ic = d2h(ip, (ln, ihd))
            rk, rv = rel(kc, st.k[:ln]), rel(vc, st.v[:ln])
            ties = check_index(ctx, dbg, case, n, t0, ln) if dbg else 0
            masked += n if dbg else 0
            say(f"{case} call {i} (n={n}, cached {ln} from position {st.base}, mask {'on' if dbg else 'off'}): "
                f"max-abs {err:.2e} rel-L2 {r:.2e} (|ref| max {np.abs(ref).max():.2f}); "
                f"caches rel {rk:.1e}/{rv:.1e}; indexer keys, pooled keys, scores and kept blocks "
                f"{'bit-exact' if dbg else 'n/a'}{f' ({ties} exact boundary ties)' if ties else ''}")
            assert np.array_equal(ic.view(np.uint32), st.idx[:ln].view(np.uint32)), "indexer keys differ"
            assert err < MAX_ABS and r < REL_L2, (i, err, r)
            assert rk < 1e-4 and rv < 1e-4, (i, rk, rv)
            t0 += n
    return masked


CASES = [
    # d, h, kvh, hd, idx heads, idx hd, budget, compress, cap, rotary factor
    (256, 4, 2, 64, 2, 64, 4096, 4, 64, 0.25),
    (256, 4, 2, 64, 2, 64, 8, 2, 64, 0.25),
    (192, 2, 1, 64, 2, 32, 6, 3, 48, 0.5),
]


@pytest.mark.parametrize("case", CASES)
def test_small_shapes(torch_dev, case):
    torch, dev = torch_dev
    say(f"case: attention {case}")
    run_calls(torch, dev, case, [1, 3, 1, 8, 1, 5, 1, 4])


def test_model_shape_long_context(torch_dev):
    """hidden 2048, 16 heads of 128 over 2 kv heads, indexer 4 x 128,
    rotary 1/4, cache 2048: a 700-token prefill in chunks, then decode
    steps; the budget of 512 turns the block mask on past 512 keys"""
    torch, dev = torch_dev
    case = (2048, 16, 2, 128, 4, 128, 512, 4, 2048, 0.25)
    say(f"case: attention {case}")
    run_calls(torch, dev, case, [256, 256, 188, 1, 1, 1], seed=2)


WIDE_CASES = [
    # head_dim 256 (the register arrays' bound), one kv head for 4 heads
    (512, 4, 1, 256, 2, 64, 4096, 4, 256, 0.25),
    # 16 query heads on one kv head: several head groups per workgroup row
    (256, 16, 1, 64, 2, 64, 16, 4, 128, 0.25),
]


@pytest.mark.parametrize("case", WIDE_CASES)
def test_wide_head_shapes(torch_dev, case):
    torch, dev = torch_dev
    say(f"case: attention {case}")
    run_calls(torch, dev, case, [1, 3, 1, 40, 1, 5, 1])


IRREGULAR_CASES = [
    # hidden 320, 5 query heads on 1 kv head, indexer 3 heads of 68, budget
    # 12 keys in blocks of 3, full rotary
    (320, 5, 1, 64, 3, 68, 12, 3, 96, 1.0),
    # hidden 448, 6 heads on 3 kv heads of 192, compress 1 (every key its own block)
    (448, 6, 3, 192, 1, 64, 20, 1, 80, 0.25),
    # hidden 640, 4 heads of 128 on 2 kv heads, indexer 2 heads of 36, blocks of 5
    (640, 4, 2, 128, 2, 36, 25, 5, 120, 0.25),
]


@pytest.mark.parametrize("case", IRREGULAR_CASES)
def test_irregular_shapes(torch_dev, case):
    """valid shapes off the usual ones (odd head counts and hidden sizes,
    head dim 192, indexer dims 36 and 68, compress 1, 3 and 5, full rotary):
    one-token calls and chunks, the block mask switching on past the budget"""
    torch, dev = torch_dev
    say(f"case: attention irregular {case}")
    run_calls(torch, dev, case, [1, 4, 1, 17, 1, 30, 1, 2])


def test_long_cache_decode(torch_dev):
    """6,000+ cached keys with the block mask on (budget 2048): 2048-token
    prefill chunks, then one-token calls that split the cache into ~97
    chunks of 64 keys, more than one lane of the combine holds"""
    torch, dev = torch_dev
    case = (256, 4, 1, 64, 2, 64, 2048, 4, 8192, 0.25)
    say(f"case: attention {case}")
    assert run_calls(torch, dev, case, [2048, 2048, 2048, 50, 1, 1], seed=4) == 2048 + 2048 + 50 + 2


def test_bench_indexer_setting(torch_dev):
    """the benchmark's indexer (4 heads of 128, rotary 32 of 128, budget
    2048, compress 4) with the mask on: 2048-token chunks to 4,096+ cached
    keys, then one-token steps; hidden 256 and 2 query heads keep the
    oracle's attention part short"""
    torch, dev = torch_dev
    case = (256, 2, 1, 128, 4, 128, 2048, 4, 8192, 0.25)
    say(f"case: attention {case}")
    assert run_calls(torch, dev, case, [2048, 2048, 40, 1, 1], seed=5) == 2048 + 40 + 2


SLIDE_CASES = [
    # d, h, kvh, hd, idx heads, idx hd, budget, compress, cap, rotary factor
    (256, 4, 2, 64, 2, 64, 8, 2, 16, 0.25),      # the block mask inside a 16-row window
    (256, 4, 1, 64, 2, 64, 8, 4, 20, 0.5),       # blocks of 4, one kv head
    (192, 2, 1, 64, 2, 32, 4096, 3, 12, 0.5),    # dense window, blocks of 3
]


@pytest.mark.parametrize("case", SLIDE_CASES)
def test_sliding_window(torch_dev, case):
    """slide = 1: calls past kv_cap drop the oldest rows of k, v and the
    indexer keys together, compress rows at a time; the window moves
    through buffers of twice the capacity and is copied back when it
    reaches their end (several times here).  Against the oracle with the
    same option (pinned by tests/test_oracle_attn.py against a float64
    statement over the full history): outputs, the window's k and v, and
    the indexer bit for bit"""
    torch, dev = torch_dev
    say(f"case: sliding attention {case}")
    calls = [5, 7, 1, 1, 6, 1, 9, 1, 1, 8, 1, 3, 1] * 3
    run_calls(torch, dev, case, calls, seed=6, slide=True)


def test_sliding_window_model_shape(torch_dev):
    """the model's attention shape in a 1024-row window with the benchmark's
    indexer budget and compress (mask on from 513 keys): 256-token chunks
    past the capacity, then one-token steps"""
    torch, dev = torch_dev
    case = (2048, 16, 2, 128, 4, 128, 512, 4, 1024, 0.25)
    say(f"case: sliding attention {case}")
    run_calls(torch, dev, case, [256] * 6 + [1, 1, 1], seed=7, slide=True)


def test_sliding_errors(torch_dev):
    torch, dev = torch_dev
    pkg = load_pkg()
    with pytest.raises(pkg.QmoeError, match="slide"):
        pkg.AttentionContext(256, 4, 2, 64, 2, 64, 8, 3, kv_cap=16, slide=True)  # 16 % 3
    A = orc.Attention(256, 4, 2, 64, 2, 64, 8, 4, kv_cap=8, slide=True)
    with pkg.AttentionContext(256, 4, 2, 64, 2, 64, 8, 4, kv_cap=8, max_tokens=8, slide=True,
                              max_position=64) as ctx:
        ctx.upload_layer(0, A.arrays())
        ctx.forward(0, torch.zeros((3, 256), device=dev), 0)
        with pytest.raises(pkg.QmoeError, match="continues at position 3"):
            ctx.forward(0, torch.zeros((1, 256), device=dev), 5)
        with pytest.raises(pkg.QmoeError, match="would drop 4 rows of the 3 cached"):
            ctx.forward(0, torch.zeros((8, 256), device=dev), 3)
        ctx.forward(0, torch.zeros((5, 256), device=dev), 3)   # fills the window
        ctx.forward(0, torch.zeros((1, 256), device=dev), 8)   # slides by 4
        torch.cuda.synchronize()
        assert ctx.cache(0)[3] == 5


def test_dense_model_shape(torch_dev):
    torch, dev = torch_dev
    case = (2048, 16, 2, 128, 4, 128, 2048, 4, 2048, 0.25)
    say(f"case: attention {case}")
    run_calls(torch, dev, case, [64, 1, 1, 1], seed=3)


def test_errors(torch_dev):
    torch, dev = torch_dev
    pkg = load_pkg()
    for bad in [(100, 4, 2, 64, 2, 64, 8, 2, 64), (256, 4, 3, 64, 2, 64, 8, 2, 64),
                (256, 4, 2, 96, 2, 64, 8, 2, 64), (256, 4, 2, 64, 2, 8, 8, 2, 64),
                (256, 4, 2, 64, 65, 64, 8, 2, 64), (256, 4, 2, 64, 40, 256, 8, 2, 64)]:
        with pytest.raises(pkg.QmoeError, match="attention shape unsupported"):
            pkg.AttentionContext(*bad)
    with pkg.AttentionContext(256, 4, 2, 64, 2, 64, 8, 2, kv_cap=4, max_tokens=4) as ctx:
        x = torch.zeros((1, 256), device=dev)
        with pytest.raises(pkg.QmoeError, match="has no weights"):
            ctx.forward(0, x, 0)
        A = orc.Attention(256, 4, 2, 64, 2, 64, 8, 2, kv_cap=4)
        ctx.upload_layer(0, A.arrays())
        ctx.forward(0, torch.zeros((4, 256), device=dev), 0)
        with pytest.raises(pkg.QmoeError, match="pass kv_cap"):
            ctx.forward(0, x, 4)
        ctx.reset(0)
        ctx.forward(0, x, 0)
        torch.cuda.synchronize()
        assert ctx.cache(0)[3] == 1
        with pytest.raises(pkg.QmoeError, match="pass max_position"):
            ctx.forward(0, x, 4)
    with pkg.AttentionContext(256, 4, 2, 64, 2, 64, 8, 2, kv_cap=4, max_tokens=4, max_position=16) as ctx:
        ctx.upload_layer(0, A.arrays())
        ctx.forward(0, x, 15)
        with pytest.raises(pkg.QmoeError, match="pass max_position"):
            ctx.forward(0, x, 16)
    with pytest.raises(pkg.QmoeError, match="max_position"):
        pkg.AttentionContext(256, 4, 2, 64, 2, 64, 8, 2, kv_cap=4, max_position=-1)
