"""C-ABI checks that need no GPU: libqmoe.so loads, exports every function
that include/qmoe.h declares (and the binding covers them), and argument
errors come back as -1 + message without touching the device."""
import ctypes
import os
import re

import pytest

from conftest import ROOT, load_pkg

HEADER = os.path.join(ROOT, "include", "qmoe.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w \*]*?\b(qmoe_\w+)\s*\(", src, flags=re.M)
    return sorted(set(names))


def test_header_lists_entry_points():
    names = declared_functions()
    for must in ("qmoe_create", "qmoe_router", "qmoe_dispatch", "qmoe_expert_ffn",
                 "qmoe_combine", "qmoe_layer_forward", "qmoe_moe_forward_host"):
        assert must in names


def test_library_exports_every_declared_symbol():
    pkg = load_pkg()
    lib = ctypes.CDLL(pkg.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding declares a signature for each of them
    assert set(declared_functions()) <= set(pkg.SIGNATURES)


def test_version():
    pkg = load_pkg()
    assert "gfx950" in pkg.version()


def test_null_and_bad_arguments_return_errors():
    pkg = load_pkg()
    lib = pkg.lib()
    err = pkg.QmoeErr()
    # every entry point rejects a NULL context with a message, no abort
    assert lib.qmoe_layer_forward(None, 0, None, 0, 1, None, 0, None, ctypes.byref(err)) == -1
    assert b"ctx is NULL" in err.msg
    assert lib.qmoe_dispatch(None, None, 1, None, None, None, None, ctypes.byref(err)) == -1
    assert lib.qmoe_combine(None, None, None, None, None, 1, None, 0, None, None,
                            ctypes.byref(err)) == -1
    assert lib.qmoe_last_routing(None, 1, None, None, None, None, None, None, None,
                                 ctypes.byref(err)) == -1
    # the hyper-connection entry points too
    for rc in (lib.qmoe_hc_enable(None, 4, 320, ctypes.byref(err)),
               lib.qmoe_hc_mix(None, 0, None, 1, None, None, None, None, ctypes.byref(err)),
               lib.qmoe_hc_inject(None, None, None, 1, None, None, ctypes.byref(err)),
               lib.qmoe_hc_layer_forward(None, 0, None, 1, None, None, ctypes.byref(err)),
               lib.qmoe_hc_synth_layer(None, 0, 1, ctypes.byref(err))):
        assert rc == -1 and b"ctx is NULL" in err.msg
    # config validation happens before any device call
    h = ctypes.c_void_p()
    for bad, msg in (((256, 8, 2, 128, 128, 1, 4, 1e-6), b"group_size"),
                     ((250, 8, 2, 128, 64, 1, 4, 1e-6), b"hidden"),
                     ((256, 8, 9, 128, 64, 1, 4, 1e-6), b"top_k"),
                     ((256, 2000, 2, 128, 64, 1, 4, 1e-6), b"n_experts"),
                     ((256, 8, 2, 100, 64, 1, 4, 1e-6), b"moe_inter"),
                     ((256, 8, 2, 128, 64, 0, 4, 1e-6), b"n_layers"),
                     ((256, 8, 2, 128, 64, 1, 0, 1e-6), b"max_tokens")):
        cfg = pkg.QmoeConfig(*bad)
        assert lib.qmoe_create(ctypes.byref(h), ctypes.byref(cfg), ctypes.byref(err)) == -1
        assert msg in err.msg, (bad, err.msg)
    assert lib.qmoe_synth_fill(None, 10, 0, 0, 0, 0, 0, 1.0, None, ctypes.byref(err)) == -1


def test_create_without_device_fails_cleanly():
    try:
        import torch
        if torch.cuda.is_available():
            pytest.skip("a HIP device is present")
    except Exception:
        pass
    pkg = load_pkg()
    with pytest.raises(pkg.QmoeError, match="HIP error"):
        pkg.MoeContext(256, 8, 2, 128)


def test_workloads_match_the_benchmarked_shapes():
    pkg = load_pkg()
    w = pkg.WORKLOADS
    assert (w["tiny"].hidden, w["tiny"].n_experts, w["tiny"].top_k, w["tiny"].moe_inter,
            w["tiny"].n_tokens) == (256, 8, 2, 128, 4)
    for name in ("decode", "batched", "prefill", "depth48"):
        assert (w[name].hidden, w[name].n_experts, w[name].top_k, w[name].moe_inter) == \
            (2048, 512, 10, 512)
    assert w["decode"].n_tokens == 1 and w["batched"].n_tokens == 64
    assert w["prefill"].n_tokens == 4096 and w["depth48"].n_layers == 48
