"""Helpers for the GPU tests: device-to-host copies of a context's weights
and the check that the device-generated tensors a parity case uses are the
host generator's bit for bit."""
import ctypes

import numpy as np

ROUTED = ("gate_q", "gate_s", "gate_b", "up_q", "up_s", "up_b", "down_q", "down_s", "down_b")
RESIDENT = ("router_w", "router_bias", "sh_gate_q", "sh_gate_s", "sh_gate_b", "sh_up_q", "sh_up_s",
            "sh_up_b", "sh_down_q", "sh_down_s", "sh_down_b", "sh_gate_w", "norm_w")

_hip = None


def d2h(ptr, like, offset_elems=0, count=None):
    """copy `count` elements of like's dtype from device address ptr (+offset)"""
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
    count = like.size if count is None else count
    buf = np.empty(count, like.dtype)
    rc = _hip.hipMemcpy(ctypes.c_void_p(buf.ctypes.data),
                        ctypes.c_void_p(ptr + offset_elems * like.dtype.itemsize),
                        ctypes.c_size_t(buf.nbytes), 2)
    assert rc == 0, rc
    return buf


def assert_synth_matches(ctx, layer, L, experts):
    """every resident tensor of a synthesised layer, and the routed tensors
    of `experts`, equal the oracle Layer's arrays with zero mismatches"""
    dw = ctx.device_weights(layer)
    for name in RESIDENT:
        ref = L.t[name]
        if ref is None:
            assert dw[name] is None, name
            continue
        got = d2h(dw[name], ref)
        assert np.array_equal(got, ref), (layer, name, int((got != ref).sum()))
    E = L.E
    for name in ROUTED:
        ref = L.t[name]
        per = ref.size // E
        for e in sorted(set(int(v) for v in np.asarray(experts).reshape(-1))):
            got = d2h(dw[name], ref, e * per, per)
            assert np.array_equal(got, ref[e * per:(e + 1) * per]), (layer, name, e)
