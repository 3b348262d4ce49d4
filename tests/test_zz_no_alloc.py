"""qmoe_layer_forward_noalloc -- the MoE layer with its scratch in a static
device block instead of allocated memory -- through the C ABI, against
qmoe_layer_forward on the same resident layer.

Both run the same kernels on the same inputs, so the bar is bit-identical
outputs.  Every case makes two calls in a row, the second with fewer
tokens (the static block keeps the first call's contents, laid out for the
larger n), and checks after them that qmoe_layer_forward still returns what
it returned before.  Sizes past the static block and bad arguments come
back as errors.
"""
import ctypes

import pytest

from conftest import load_pkg

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def torch_dev(gpu):
    import torch
    return torch, gpu


def run_ref(pkg, ctx, x, dtype, flags):
    import torch
    n = x.shape[0]
    out = torch.empty((n, ctx.H), dtype=torch.float32, device=x.device)
    err = pkg.QmoeErr()
    rc = pkg.lib().qmoe_layer_forward(ctx._h, 0, x.data_ptr(), dtype, n, out.data_ptr(), flags, None,
                                      ctypes.byref(err))
    assert rc == 0, err.msg
    return out


def run_noalloc(pkg, cfg, w, x, dtype, flags):
    import torch
    n = x.shape[0]
    out = torch.full((n, cfg.hidden), float("nan"), dtype=torch.float32, device=x.device)
    err = pkg.QmoeErr()
    rc = pkg.lib().qmoe_layer_forward_noalloc(ctypes.byref(cfg), ctypes.byref(w), x.data_ptr(), dtype,
                                              n, out.data_ptr(), flags, None, ctypes.byref(err))
    assert rc == 0, err.msg
    return out


def device_weights(pkg, ctx):
    w = pkg.QmoeLayerWeights()
    err = pkg.QmoeErr()
    assert pkg.lib().qmoe_layer_device_weights(ctx._h, 0, ctypes.byref(w), ctypes.byref(err)) == 0, err.msg
    return w


SHAPES = {"tiny": (256, 8, 2, 128), "model": (2048, 512, 10, 512),
          "odd": (768, 60, 6, 320)}


@pytest.mark.parametrize("shape,with_norm,calls", [
    # calls: (n, bf16 input, QMOE_RESIDUAL), larger first
    ("tiny", False, [(40, False, 0), (3, True, 1)]),
    ("tiny", True, [(64, True, 0), (1, False, 0)]),
    ("model", False, [(300, False, 0), (1, False, 0)]),
    ("model", False, [(64, True, 1), (16, False, 0)]),
    ("odd", True, [(90, False, 1), (1, True, 0)]),
])
def test_noalloc_matches_layer_forward(torch_dev, shape, with_norm, calls):
    torch, dev = torch_dev
    pkg = load_pkg()
    H, E, k, I = SHAPES[shape]
    max_n = max(n for n, _, _ in calls)
    say(f"case: no-alloc layer {shape} norm={with_norm} calls {calls}")
    with pkg.MoeContext(H, E, k, I, n_layers=1, max_tokens=max_n) as ctx:
        ctx.synth_layer(0, 7, with_norm=with_norm)
        w = device_weights(pkg, ctx)
        cfg = pkg.QmoeConfig(H, E, k, I, 64, 1, max_n, 1e-6)
        gen = torch.Generator(device="cpu").manual_seed(11)
        refs = []
        for n, bf, flags in calls:
            x = torch.randn((n, H), generator=gen).to(dev)
            if bf:
                x = x.to(torch.bfloat16)
            dt = pkg.BF16 if bf else pkg.F32
            say(f"  call n={n} bf16={bf} flags={flags}")
            ref = run_ref(pkg, ctx, x, dt, flags)
            got = run_noalloc(pkg, cfg, w, x, dt, flags)
            torch.cuda.synchronize()
            assert torch.isfinite(ref).all()
            diff = (got != ref).sum().item()
            say(f"  n={n}: {diff} of {ref.numel()} elements differ")
            assert diff == 0
            refs.append((x, dt, flags, ref))
        # the context's entry point is unaffected by the static block
        for x, dt, flags, ref in refs:
            again = run_ref(pkg, ctx, x, dt, flags)
            torch.cuda.synchronize()
            assert torch.equal(again, ref)


def test_noalloc_errors(torch_dev):
    torch, dev = torch_dev
    pkg = load_pkg()
    lib = pkg.lib()
    H, E, k, I = SHAPES["model"]
    say("case: no-alloc errors")
    with pkg.MoeContext(H, E, k, I, n_layers=1, max_tokens=8) as ctx:
        ctx.synth_layer(0, 3)
        w = device_weights(pkg, ctx)
        x = torch.zeros((8, H), device=dev)
        out = torch.zeros((8, H), device=dev)
        err = pkg.QmoeErr()

        def call(cfg, weights, n, flags=0, dtype=pkg.F32):
            return lib.qmoe_layer_forward_noalloc(
                ctypes.byref(cfg) if cfg is not None else None,
                ctypes.byref(weights) if weights is not None else None, x.data_ptr(), dtype, n,
                out.data_ptr(), flags, None, ctypes.byref(err))

        big = pkg.QmoeConfig(H, E, k, I, 64, 1, 100000, 1e-6)
        assert call(big, w, 460) == -1 and b"static scratch holds" in err.msg
        cfg = pkg.QmoeConfig(H, E, k, I, 64, 1, 8, 1e-6)
        assert call(cfg, w, 9) == -1 and b"max_tokens" in err.msg
        assert call(cfg, w, 1, flags=4) == -1 and b"unknown flags" in err.msg
        assert call(cfg, w, 1, dtype=7) == -1
        assert call(None, w, 1) == -1 and b"cfg is NULL" in err.msg
        assert call(cfg, None, 1) == -1 and b"dev_weights is NULL" in err.msg
        bad = pkg.QmoeLayerWeights.from_buffer_copy(w)
        bad.gate_q = None
        assert call(cfg, bad, 1) == -1 and b"is NULL" in err.msg
        assert call(cfg, w, 0) == 0
        # a good call after the refusals
        assert call(cfg, w, 8) == 0, err.msg
        ref = run_ref(pkg, ctx, x, pkg.F32, 0)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
