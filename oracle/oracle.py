"""ctypes binding of liboracle.so -- the CPU restatement of the reference
C port's MoE layer (see moe_oracle.h for what it restates and where).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
the cpu_baseline leg of bench.py, as the checker.  The product library never
loads it.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")
REF_UTIL_PATH = os.path.join(_HERE, "_ref", "libref_util.so")

# synthetic stream tags, identical to include/qmoe.h QMOE_TAG_*
TAG = dict(
    ROUTER_W=1, GATE_Q=2, GATE_S=3, GATE_B=4, UP_Q=5, UP_S=6, UP_B=7, DOWN_Q=8, DOWN_S=9,
    DOWN_B=10, SH_GATE_Q=11, SH_GATE_S=12, SH_GATE_B=13, SH_UP_Q=14, SH_UP_S=15, SH_UP_B=16,
    SH_DOWN_Q=17, SH_DOWN_S=18, SH_DOWN_B=19, SHGATE_W=20, X=22,
    HC_DOWN_Q=24, HC_DOWN_S=25, HC_DOWN_B=26, HC_UP_Q=27, HC_UP_S=28, HC_UP_B=29,
    HC_INJECT_W=30, HYPER=31,
    DN_QKV_Q=40, DN_QKV_S=41, DN_QKV_B=42, DN_Z_Q=43, DN_Z_S=44, DN_Z_B=45, DN_A_W=46,
    DN_B_W=47, DN_OUT_Q=48, DN_OUT_S=49, DN_OUT_B=50, DN_CONV_W=51, DN_NORM_W=52, DN_A_LOG=53,
    DN_DT_BIAS=54, DN_X=55,
    AT_Q_Q=60, AT_Q_S=61, AT_Q_B=62, AT_K_Q=63, AT_K_S=64, AT_K_B=65, AT_V_Q=66, AT_V_S=67,
    AT_V_B=68, AT_O_Q=69, AT_O_S=70, AT_O_B=71, AT_IDX_W=72, AT_Q_NORM=73, AT_K_NORM=74,
    AT_IDX_Q_NORM=75, AT_IDX_K_NORM=76, AT_X=77,
)

ROUTED_FAITHFUL, ROUTED_Q4 = 0, 1

_F = ctypes.c_float
_I = ctypes.c_int
_P = ctypes.c_void_p
_U64 = ctypes.c_uint64
_SZ = ctypes.c_size_t


class OrcLayer(ctypes.Structure):
    _fields_ = [
        ("hidden", _I), ("n_experts", _I), ("top_k", _I), ("moe_inter", _I), ("group_size", _I),
        ("rms_eps", _F),
        ("router_w", _P), ("router_bias", _P),
        ("gate_q", _P), ("gate_s", _P), ("gate_b", _P),
        ("up_q", _P), ("up_s", _P), ("up_b", _P),
        ("down_q", _P), ("down_s", _P), ("down_b", _P),
        ("sh_gate_q", _P), ("sh_gate_s", _P), ("sh_gate_b", _P),
        ("sh_up_q", _P), ("sh_up_s", _P), ("sh_up_b", _P),
        ("sh_down_q", _P), ("sh_down_s", _P), ("sh_down_b", _P),
        ("sh_gate_w", _P), ("norm_w", _P),
    ]


class OrcHc(ctypes.Structure):
    _fields_ = [
        ("hc", _I), ("d", _I), ("lowrank", _I), ("group_size", _I), ("hc_norm", _P),
        ("down_q", _P), ("down_s", _P), ("down_b", _P),
        ("up_q", _P), ("up_s", _P), ("up_b", _P), ("inject_w", _P),
    ]


class OrcDn(ctypes.Structure):
    _fields_ = [
        ("hidden", _I), ("n_k_heads", _I), ("n_v_heads", _I), ("k_head_dim", _I),
        ("v_head_dim", _I), ("conv_kernel", _I), ("group_size", _I),
        ("qkv_q", _P), ("qkv_s", _P), ("qkv_b", _P), ("z_q", _P), ("z_s", _P), ("z_b", _P),
        ("a_w", _P), ("b_w", _P), ("out_q", _P), ("out_s", _P), ("out_b", _P), ("conv_w", _P),
        ("norm_w", _P), ("a_log", _P), ("dt_bias", _P),
    ]


class OrcAttn(ctypes.Structure):
    _fields_ = [
        ("hidden", _I), ("n_heads", _I), ("n_kv_heads", _I), ("head_dim", _I), ("idx_heads", _I),
        ("idx_head_dim", _I), ("idx_budget", _I), ("idx_compress", _I), ("kv_cap", _I),
        ("group_size", _I), ("rotary_factor", _F), ("rope_theta", _F),
        ("q_q", _P), ("q_s", _P), ("q_b", _P), ("k_q", _P), ("k_s", _P), ("k_b", _P),
        ("v_q", _P), ("v_s", _P), ("v_b", _P), ("o_q", _P), ("o_s", _P), ("o_b", _P),
        ("idx_w", _P), ("q_norm", _P), ("k_norm", _P), ("idx_q_norm", _P), ("idx_k_norm", _P),
        ("slide", _I),
    ]


class OrcAttnState(ctypes.Structure):
    _fields_ = [("k_cache", _P), ("v_cache", _P), ("idx_keys", _P), ("kv_len", _I), ("idx_len", _I),
                ("base", _I)]


class OrcAttnDbg(ctypes.Structure):
    _fields_ = [("pooled", _P), ("qs", _P), ("scores", _P), ("keep", _P)]


class OrcOpts(ctypes.Structure):
    _fields_ = [("x_is_bf16", _I), ("residual", _I), ("routed_mode", _I), ("n_threads", _I)]


_SIG = {
    "orc_bf16_to_f32": (_F, [ctypes.c_uint16]),
    "orc_f32_to_bf16": (ctypes.c_uint16, [_F]),
    "orc_rmsnorm_seq": (None, [_P, _P, _SZ, _F, _P]),
    "orc_rmsnorm_r64": (None, [_P, _P, _SZ, _F, _P]),
    "orc_silu": (_F, [_F]),
    "orc_sigmoid": (_F, [_F]),
    "orc_dot_r64_bf16w": (_F, [_P, _P, _I]),
    "orc_sumsq_r64": (_F, [_P, _I]),
    "orc_topk_quickselect": (None, [_P, _I, _I, _P]),
    "orc_topk_canonical": (None, [_P, _I, _I, _P]),
    "orc_dequant_q4": (None, [_P, _P, _P, _SZ, _SZ, _SZ, _P]),
    "orc_dequant_q4_f32sb": (None, [_P, _P, _P, _SZ, _SZ, _SZ, _P]),
    "orc_gemm_fp32": (None, [_I, _I, _I, _P, _P, _P]),
    "orc_gemm_bf16": (None, [_I, _I, _I, _P, _P, _P]),
    "orc_gemm_q4_f32sb": (None, [_I, _I, _I, _P, _P, _P, _P, _I, _P]),
    "orc_gemm_q4": (None, [_I, _I, _I, _P, _P, _P, _P, _I, _P]),
    "orc_warm_create": (_P, [_P, _P, _I, _I]),
    "orc_warm_destroy": (None, [_P]),
    "orc_warm_bytes": (_SZ, [_P]),
    "orc_moe_forward_warm": (_I, [_P, _P, _P, _I, _P, _P, _P]),
    "orc_time_forward_warm": (ctypes.c_double, [_P, _P, _P, _I, _P, _P, _I, _I]),
    "orc_dispatch": (_I, [_P, _I, _I, _I, _P, _P, _P, _P]),
    "orc_moe_forward": (_I, [ctypes.POINTER(OrcLayer), _P, _I, _P, ctypes.POINTER(OrcOpts), _P, _I,
                             _P, _P, _P, _P, _P, _P, _P]),
    "orc_route": (_I, [ctypes.POINTER(OrcLayer), _P, _I, _I, _P, _P, _P, _P, _P, _P, _I, _P]),
    "orc_hc_mix": (_I, [ctypes.POINTER(OrcHc), _P, _I, _P, _P, _P]),
    "orc_hc_inject": (None, [_I, _I, _I, _P, _P, _P]),
    "orc_mix64": (_U64, [_U64]),
    "orc_tensor_key": (_U64, [_U64, ctypes.c_uint32, ctypes.c_uint32]),
    "orc_gen_normal_bf16": (None, [_P, _SZ, _U64, _U64, _F]),
    "orc_gen_normal_f32": (None, [_P, _SZ, _U64, _U64, _F]),
    "orc_gen_codes": (None, [_P, _SZ, _U64, _U64]),
    "orc_zipf_bias": (None, [_P, _I, ctypes.c_double, ctypes.c_double, _U64]),
    "orc_attn_forward": (_I, [ctypes.POINTER(OrcAttn), ctypes.POINTER(OrcAttnState), _P, _I, _I, _P]),
    "orc_attn_forward_dbg": (_I, [ctypes.POINTER(OrcAttn), ctypes.POINTER(OrcAttnState), _P, _I, _I, _P,
                                  ctypes.POINTER(OrcAttnDbg)]),
    "orc_dn_decay": (_F, [_F, _F, _F]),
    "orc_dn_forward": (_I, [ctypes.POINTER(OrcDn), _P, _I, _P, _P, _P, _P]),
    "orc_time_forward": (ctypes.c_double, [ctypes.POINTER(OrcLayer), _P, _I, _P,
                                           ctypes.POINTER(OrcOpts), _I, _I]),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        _lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIG.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


def ref_util():
    """the reference's own util.h bf16 conversions, or None when not built"""
    if not os.path.exists(REF_UTIL_PATH):
        return None
    r = ctypes.CDLL(REF_UTIL_PATH)
    r.ref_bf16_to_f32.restype = _F
    r.ref_bf16_to_f32.argtypes = [ctypes.c_uint16]
    r.ref_f32_to_bf16.restype = ctypes.c_uint16
    r.ref_f32_to_bf16.argtypes = [_F]
    return r


def _p(a):
    return None if a is None else a.ctypes.data


# ------------------------------------------------------------- generators

def tensor_key(seed, layer, tag):
    return lib().orc_tensor_key(seed, layer, tag)


def gen_bf16(count, seed, layer, tag, std, start=0):
    out = np.empty(count, dtype=np.uint16)
    lib().orc_gen_normal_bf16(_p(out), count, tensor_key(seed, layer, TAG[tag]), start, std)
    return out


def gen_f32(count, seed, layer, tag, std, start=0):
    out = np.empty(count, dtype=np.float32)
    lib().orc_gen_normal_f32(_p(out), count, tensor_key(seed, layer, TAG[tag]), start, std)
    return out


def gen_codes(count, seed, layer, tag, start=0):
    out = np.empty(count, dtype=np.uint32)
    lib().orc_gen_codes(_p(out), count, tensor_key(seed, layer, TAG[tag]), start)
    return out


def zipf_bias(E, s, scale, seed):
    out = np.empty(E, dtype=np.float32)
    lib().orc_zipf_bias(_p(out), E, s, scale, seed)
    return out


def bf16_to_f32(a):
    """exact widening of bf16 bit patterns (uint16) to float32"""
    return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a):
    """round-to-nearest-even narrowing, as c/src/util.h:63-71 (vectorised)"""
    b = np.asarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    return (r & 0xFFFF).astype(np.uint16)


class Layer:
    """One synthetic layer in host memory, checkpoint layout, generated from
    the same seeded streams as qmoe_synth_layer (codes U{0..15}, scales
    N(0,0.02), biases N(0,0.01), router and shared gate N(0,0.02))."""

    def __init__(self, H, E, k, I, seed=0, layer=0, with_norm=False, router_bias=None,
                 group_size=64, eps=1e-6, only_experts=None):
        self.H, self.E, self.k, self.I, self.g, self.eps = H, E, k, I, group_size, eps
        G, GI = H // group_size, I // group_size
        s, L = seed, layer
        self.t = {}
        self.t["router_w"] = gen_bf16(E * H, s, L, "ROUTER_W", 0.02)
        self.t["router_bias"] = (None if router_bias is None
                                 else np.ascontiguousarray(router_bias, dtype=np.float32))
        if only_experts is None:
            self.t["gate_q"] = gen_codes(E * I * H // 8, s, L, "GATE_Q")
            self.t["gate_s"] = gen_bf16(E * I * G, s, L, "GATE_S", 0.02)
            self.t["gate_b"] = gen_bf16(E * I * G, s, L, "GATE_B", 0.01)
            self.t["up_q"] = gen_codes(E * I * H // 8, s, L, "UP_Q")
            self.t["up_s"] = gen_bf16(E * I * G, s, L, "UP_S", 0.02)
            self.t["up_b"] = gen_bf16(E * I * G, s, L, "UP_B", 0.01)
            self.t["down_q"] = gen_codes(E * H * I // 8, s, L, "DOWN_Q")
            self.t["down_s"] = gen_bf16(E * H * GI, s, L, "DOWN_S", 0.02)
            self.t["down_b"] = gen_bf16(E * H * GI, s, L, "DOWN_B", 0.01)
        else:
            # sparse fill: only the listed experts get their real values (the
            # streams are counter-based), everything else stays zero
            self.t["gate_q"] = np.zeros(E * I * H // 8, np.uint32)
            self.t["up_q"] = np.zeros(E * I * H // 8, np.uint32)
            self.t["down_q"] = np.zeros(E * H * I // 8, np.uint32)
            for nm in ("gate_s", "gate_b", "up_s", "up_b"):
                self.t[nm] = np.zeros(E * I * G, np.uint16)
            for nm in ("down_s", "down_b"):
                self.t[nm] = np.zeros(E * H * GI, np.uint16)
            qn, sn, dqn, dsn = I * H // 8, I * G, H * I // 8, H * GI
            for e in sorted(set(int(v) for v in only_experts)):
                for nm, tg in (("gate_q", "GATE_Q"), ("up_q", "UP_Q")):
                    self.t[nm][e * qn:(e + 1) * qn] = gen_codes(qn, s, L, tg, start=e * qn)
                self.t["down_q"][e * dqn:(e + 1) * dqn] = gen_codes(dqn, s, L, "DOWN_Q", start=e * dqn)
                for nm, tg, sd in (("gate_s", "GATE_S", 0.02), ("gate_b", "GATE_B", 0.01),
                                   ("up_s", "UP_S", 0.02), ("up_b", "UP_B", 0.01)):
                    self.t[nm][e * sn:(e + 1) * sn] = gen_bf16(sn, s, L, tg, sd, start=e * sn)
                for nm, tg, sd in (("down_s", "DOWN_S", 0.02), ("down_b", "DOWN_B", 0.01)):
                    self.t[nm][e * dsn:(e + 1) * dsn] = gen_bf16(dsn, s, L, tg, sd, start=e * dsn)
        self.t["sh_gate_q"] = gen_codes(I * H // 8, s, L, "SH_GATE_Q")
        self.t["sh_gate_s"] = gen_bf16(I * G, s, L, "SH_GATE_S", 0.02)
        self.t["sh_gate_b"] = gen_bf16(I * G, s, L, "SH_GATE_B", 0.01)
        self.t["sh_up_q"] = gen_codes(I * H // 8, s, L, "SH_UP_Q")
        self.t["sh_up_s"] = gen_bf16(I * G, s, L, "SH_UP_S", 0.02)
        self.t["sh_up_b"] = gen_bf16(I * G, s, L, "SH_UP_B", 0.01)
        self.t["sh_down_q"] = gen_codes(H * I // 8, s, L, "SH_DOWN_Q")
        self.t["sh_down_s"] = gen_bf16(H * GI, s, L, "SH_DOWN_S", 0.02)
        self.t["sh_down_b"] = gen_bf16(H * GI, s, L, "SH_DOWN_B", 0.01)
        self.t["sh_gate_w"] = gen_bf16(H, s, L, "SHGATE_W", 0.02)
        self.t["norm_w"] = np.ones(H, np.float32) if with_norm else None
        self._build()

    @classmethod
    def from_arrays(cls, H, E, k, I, arrays, group_size=64, eps=1e-6):
        self = cls.__new__(cls)
        self.H, self.E, self.k, self.I, self.g, self.eps = H, E, k, I, group_size, eps
        self.t = {}
        for f in ("router_w", "router_bias", "gate_q", "gate_s", "gate_b", "up_q", "up_s", "up_b",
                  "down_q", "down_s", "down_b", "sh_gate_q", "sh_gate_s", "sh_gate_b", "sh_up_q",
                  "sh_up_s", "sh_up_b", "sh_down_q", "sh_down_s", "sh_down_b", "sh_gate_w",
                  "norm_w"):
            a = arrays.get(f)
            self.t[f] = None if a is None else np.ascontiguousarray(a)
        self._build()
        return self

    def _build(self):
        st = OrcLayer()
        st.hidden, st.n_experts, st.top_k, st.moe_inter = self.H, self.E, self.k, self.I
        st.group_size, st.rms_eps = self.g, self.eps
        for f, a in self.t.items():
            setattr(st, f, _p(a))
        self.st = st

    def arrays(self):
        """dict for MoeContext.upload_layer"""
        return dict(self.t)

    # -- oracle calls
    def route(self, x, x_is_bf16, n_threads=0):
        n = x.shape[0]
        logits = np.empty((n, self.E), np.float32)
        gl = np.empty(n, np.float32)
        idx = np.empty((n, self.k), np.int32)
        w = np.empty((n, self.k), np.float32)
        sg = np.empty(n, np.float32)
        xn = np.empty((n, self.H), np.float32)
        err = ctypes.create_string_buffer(512)
        rc = lib().orc_route(ctypes.byref(self.st), _p(np.ascontiguousarray(x)), int(x_is_bf16), n,
                             _p(logits), _p(gl), _p(idx), _p(w), _p(sg), _p(xn), n_threads, err)
        if rc:
            raise RuntimeError(err.value.decode())
        return dict(logits=logits, gate_logit=gl, idx=idx, w=w, shared_gate=sg, xn=xn)

    def forward(self, x, x_is_bf16, residual=False, routed_mode=ROUTED_FAITHFUL, token_sel=None,
                n_threads=0):
        x = np.ascontiguousarray(x)
        n = x.shape[0]
        sel = None if token_sel is None else np.ascontiguousarray(token_sel, dtype=np.int32)
        nout = n if sel is None else len(sel)
        out = np.empty((nout, self.H), np.float32)
        opts = OrcOpts(int(x_is_bf16), int(residual), routed_mode, n_threads)
        idx = np.empty((n, self.k), np.int32)
        w = np.empty((n, self.k), np.float32)
        sg = np.empty(n, np.float32)
        err = ctypes.create_string_buffer(512)
        rc = lib().orc_moe_forward(ctypes.byref(self.st), _p(x), n, _p(out), ctypes.byref(opts),
                                   _p(sel), 0 if sel is None else len(sel), None, None, _p(idx),
                                   _p(w), _p(sg), None, err)
        if rc:
            raise RuntimeError(err.value.decode())
        return dict(out=out, idx=idx, w=w, shared_gate=sg)

    def time_forward(self, x, x_is_bf16, n_threads, warmup=1, iters=3, routed_mode=ROUTED_Q4,
                     residual=False):
        x = np.ascontiguousarray(x)
        out = np.empty((x.shape[0], self.H), np.float32)
        opts = OrcOpts(int(x_is_bf16), int(residual), routed_mode, n_threads)
        return lib().orc_time_forward(ctypes.byref(self.st), _p(x), x.shape[0], _p(out),
                                      ctypes.byref(opts), warmup, iters)


class Warm:
    """Weight mode (i) of the CPU baseline: the listed routed experts of a
    Layer dequantised once to fp32 (the C port's warm expert cache); calls
    run fp32 GEMMs on them.  Timing only."""

    def __init__(self, layer: Layer, experts, n_threads=0):
        ids = np.ascontiguousarray(sorted(set(int(e) for e in experts)), dtype=np.int32)
        self.layer = layer
        self.h = lib().orc_warm_create(ctypes.byref(layer.st), _p(ids), len(ids), n_threads)
        if not self.h:
            raise MemoryError("orc_warm_create failed")

    @property
    def nbytes(self):
        return int(lib().orc_warm_bytes(self.h))

    def close(self):
        if self.h:
            lib().orc_warm_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def forward(self, x, x_is_bf16, residual=False, n_threads=0):
        x = np.ascontiguousarray(x)
        out = np.empty((x.shape[0], self.layer.H), np.float32)
        opts = OrcOpts(int(x_is_bf16), int(residual), ROUTED_FAITHFUL, n_threads)
        err = ctypes.create_string_buffer(512)
        rc = lib().orc_moe_forward_warm(ctypes.byref(self.layer.st), self.h, _p(x), x.shape[0],
                                        _p(out), ctypes.byref(opts), err)
        if rc:
            raise RuntimeError(err.value.decode())
        return out

    def time_forward(self, x, x_is_bf16, n_threads, warmup=1, iters=3, residual=False):
        x = np.ascontiguousarray(x)
        out = np.empty((x.shape[0], self.layer.H), np.float32)
        opts = OrcOpts(int(x_is_bf16), int(residual), ROUTED_FAITHFUL, n_threads)
        t = lib().orc_time_forward_warm(ctypes.byref(self.layer.st), self.h, _p(x), x.shape[0],
                                        _p(out), ctypes.byref(opts), warmup, iters)
        if t < 0:
            raise RuntimeError("warm forward failed (expert not warm?)")
        return t


class Hyper:
    """The MLP hyper connection of one layer (c/src/model.c:728-796,
    1703-1731) in host memory: hc_norm [hc*d] f32, input_mix_weight_down
    [R, hc*d] and input_mix_weight_up [hc*d, R] as q4 (codes U{0..15},
    scales N(0,0.02), biases N(0,0.01)), block_inject_weight [hc, hc*d] bf16
    N(0,0.02), from the same seeded streams as qmoe_hc_synth_layer;
    hc_norm is all ones there (norm_std = 0) or 1 + N(0, norm_std).
    with_inject=False leaves block_inject_weight out: the final mixer
    (model.c:1743-1745), whose mix returns no inject."""

    KEYS = ("hc_norm", "down_q", "down_s", "down_b", "up_q", "up_s", "up_b", "inject_w")

    def __init__(self, hc, d, lowrank, seed=0, layer=0, group_size=64, norm_std=0.0, with_inject=True):
        self.hc, self.d, self.R, self.g = hc, d, lowrank, group_size
        D, R, g, s, L = hc * d, lowrank, group_size, seed, layer
        self.t = {}
        if norm_std:
            self.t["hc_norm"] = (1.0 + np.random.default_rng(seed * 7919 + layer)
                                 .normal(0.0, norm_std, D)).astype(np.float32)
        else:
            self.t["hc_norm"] = np.ones(D, np.float32)
        self.t["down_q"] = gen_codes(R * D // 8, s, L, "HC_DOWN_Q")
        self.t["down_s"] = gen_bf16(R * D // g, s, L, "HC_DOWN_S", 0.02)
        self.t["down_b"] = gen_bf16(R * D // g, s, L, "HC_DOWN_B", 0.01)
        self.t["up_q"] = gen_codes(D * R // 8, s, L, "HC_UP_Q")
        self.t["up_s"] = gen_bf16(D * R // g, s, L, "HC_UP_S", 0.02)
        self.t["up_b"] = gen_bf16(D * R // g, s, L, "HC_UP_B", 0.01)
        if with_inject:
            self.t["inject_w"] = gen_bf16(hc * D, s, L, "HC_INJECT_W", 0.02)
        self._build()

    @classmethod
    def from_arrays(cls, hc, d, lowrank, arrays, group_size=64):
        self = cls.__new__(cls)
        self.hc, self.d, self.R, self.g = hc, d, lowrank, group_size
        self.t = {k: np.ascontiguousarray(arrays[k]) for k in cls.KEYS if arrays.get(k) is not None}
        self._build()
        return self

    def _build(self):
        st = OrcHc()
        st.hc, st.d, st.lowrank, st.group_size = self.hc, self.d, self.R, self.g
        for f, a in self.t.items():
            setattr(st, f, _p(a))
        self.st = st

    def arrays(self):
        return dict(self.t)

    def mix(self, hyper):
        """gated_residual: hyper [n, hc*d] f32 -> mixed [n, d], inject [n, hc], normed"""
        hyper = np.ascontiguousarray(hyper, dtype=np.float32)
        n = hyper.shape[0]
        mixed = np.empty((n, self.d), np.float32)
        inject = np.empty((n, self.hc), np.float32) if "inject_w" in self.t else None
        normed = np.empty((n, self.hc * self.d), np.float32)
        if lib().orc_hc_mix(ctypes.byref(self.st), _p(hyper), n, _p(mixed),
                            None if inject is None else _p(inject), _p(normed)):
            raise MemoryError("orc_hc_mix")
        return dict(mixed=mixed, inject=inject, normed=normed)

    def inject_update(self, hyper, inject, out):
        """hyper[t, hh, :] += inject[t, hh] * out[t, :] on a copy"""
        h = np.array(hyper, dtype=np.float32, order="C", copy=True)
        inject = np.ascontiguousarray(inject, dtype=np.float32)
        out = np.ascontiguousarray(out, dtype=np.float32)
        lib().orc_hc_inject(self.hc, self.d, h.shape[0], _p(inject), _p(out), _p(h))
        return h

    def layer_forward(self, layer, hyper):
        """model.c:1710-1731: mix, the MoE layer on mixed (f32), inject update;
        returns the new hyper state and the intermediates"""
        m = self.mix(hyper)
        r = layer.forward(m["mixed"], False)
        return dict(hyper=self.inject_update(hyper, m["inject"], r["out"]), moe_out=r["out"],
                    **m)


class DeltaNet:
    """One gated DeltaNet mixer (c/src/model.c:1146-1278) in host memory,
    checkpoint layout (names model.c:1866-1883): in_proj_qkv [conv_dim, d],
    in_proj_z [value_dim, d] and out_proj [d, value_dim] q4 (codes
    U{0..15}, scales N(0,0.02), biases N(0,0.01)); in_proj_a, in_proj_b
    [hv, d] bf16 N(0,0.02); conv1d [conv_dim, kc] bf16 N(0, conv_std);
    norm.weight [dv] = 1 + N(0,0.1), A_log and dt_bias [hv] N(0,1), all
    three rounded to bf16 and widened, as the reference loads them
    (mw_load_f32, model.c:275-293)."""

    KEYS = ("qkv_q", "qkv_s", "qkv_b", "z_q", "z_s", "z_b", "a_w", "b_w", "out_q", "out_s",
            "out_b", "conv_w", "norm_w", "a_log", "dt_bias")

    def __init__(self, d, hk, hv, dk, dv, kc=4, seed=0, layer=0, group_size=64, conv_std=0.5):
        self.d, self.hk, self.hv, self.dk, self.dv, self.kc, self.g = d, hk, hv, dk, dv, kc, group_size
        self.key_dim, self.value_dim = hk * dk, hv * dv
        self.conv_dim = 2 * self.key_dim + self.value_dim
        cd, vd, g, s, L = self.conv_dim, self.value_dim, group_size, seed, layer
        t = {}
        t["qkv_q"] = gen_codes(cd * d // 8, s, L, "DN_QKV_Q")
        t["qkv_s"] = gen_bf16(cd * d // g, s, L, "DN_QKV_S", 0.02)
        t["qkv_b"] = gen_bf16(cd * d // g, s, L, "DN_QKV_B", 0.01)
        t["z_q"] = gen_codes(vd * d // 8, s, L, "DN_Z_Q")
        t["z_s"] = gen_bf16(vd * d // g, s, L, "DN_Z_S", 0.02)
        t["z_b"] = gen_bf16(vd * d // g, s, L, "DN_Z_B", 0.01)
        t["a_w"] = gen_bf16(hv * d, s, L, "DN_A_W", 0.02)
        t["b_w"] = gen_bf16(hv * d, s, L, "DN_B_W", 0.02)
        t["out_q"] = gen_codes(d * vd // 8, s, L, "DN_OUT_Q")
        t["out_s"] = gen_bf16(d * vd // g, s, L, "DN_OUT_S", 0.02)
        t["out_b"] = gen_bf16(d * vd // g, s, L, "DN_OUT_B", 0.01)
        t["conv_w"] = gen_bf16(cd * kc, s, L, "DN_CONV_W", conv_std)
        t["norm_w"] = bf16_to_f32(f32_to_bf16(1.0 + gen_f32(dv, s, L, "DN_NORM_W", 0.1)))
        t["a_log"] = bf16_to_f32(gen_bf16(hv, s, L, "DN_A_LOG", 1.0))
        t["dt_bias"] = bf16_to_f32(gen_bf16(hv, s, L, "DN_DT_BIAS", 1.0))
        self.t = t
        self._build()

    @classmethod
    def from_arrays(cls, d, hk, hv, dk, dv, kc, arrays, group_size=64):
        self = cls.__new__(cls)
        self.d, self.hk, self.hv, self.dk, self.dv, self.kc, self.g = d, hk, hv, dk, dv, kc, group_size
        self.key_dim, self.value_dim = hk * dk, hv * dv
        self.conv_dim = 2 * self.key_dim + self.value_dim
        self.t = {k: np.ascontiguousarray(arrays[k]) for k in cls.KEYS if arrays.get(k) is not None}
        self._build()
        return self

    def _build(self):
        st = OrcDn()
        st.hidden, st.n_k_heads, st.n_v_heads = self.d, self.hk, self.hv
        st.k_head_dim, st.v_head_dim, st.conv_kernel, st.group_size = self.dk, self.dv, self.kc, self.g
        for f, a in self.t.items():
            setattr(st, f, _p(a))
        self.st = st

    def arrays(self):
        return dict(self.t)

    def new_state(self):
        return (np.zeros((self.kc - 1, self.conv_dim), np.float32),
                np.zeros((self.hv, self.dv, self.dk), np.float32))

    def forward(self, x, conv_state, rec_state, want_core=False):
        """x [n, d] f32; conv_state, rec_state updated IN PLACE (float32,
        C-contiguous); returns out [n, d] (and the recurrence output)"""
        x = np.ascontiguousarray(x, dtype=np.float32)
        assert conv_state.dtype == np.float32 and conv_state.flags.c_contiguous
        assert rec_state.dtype == np.float32 and rec_state.flags.c_contiguous
        n = x.shape[0]
        out = np.empty((n, self.d), np.float32)
        core = np.empty((n, self.value_dim), np.float32) if want_core else None
        if lib().orc_dn_forward(ctypes.byref(self.st), _p(x), n, _p(out), _p(conv_state),
                                _p(rec_state), _p(core)):
            raise MemoryError("orc_dn_forward")
        return (out, core) if want_core else out


class Attention:
    """One full-attention mixer with the QSA indexer (c/src/model.c:798-1144)
    in host memory, checkpoint layout (names model.c:1833-1850): q_proj
    [2*h*hd, d] (q and gate interleaved per head), k_proj, v_proj
    [kvh*hd, d], o_proj [d, h*hd] q4 (codes U{0..15}, scales N(0,0.02),
    biases N(0,0.01)); index_qk_proj [idx_heads*idx_hd + idx_hd, d] bf16
    N(0,0.02); the four norm weights 1 + N(0,0.1), rounded to bf16 and
    widened (mw_load_f32).  A State holds the caches."""

    KEYS = ("q_q", "q_s", "q_b", "k_q", "k_s", "k_b", "v_q", "v_s", "v_b", "o_q", "o_s", "o_b",
            "idx_w", "q_norm", "k_norm", "idx_q_norm", "idx_k_norm")

    def __init__(self, d, h, kvh, hd, idx_heads, idx_hd, budget, compress, kv_cap=2048,
                 rotary_factor=0.25, rope_theta=1e7, seed=0, layer=0, group_size=64, slide=False):
        self.slide = bool(slide)
        self.d, self.h, self.kvh, self.hd = d, h, kvh, hd
        self.ih, self.ihd, self.budget, self.compress = idx_heads, idx_hd, budget, compress
        self.cap, self.rf, self.theta, self.g = kv_cap, rotary_factor, rope_theta, group_size
        g, s, L = group_size, seed, layer
        t = {}
        for nm, rows, cols in (("q", 2 * h * hd, d), ("k", kvh * hd, d), ("v", kvh * hd, d),
                               ("o", d, h * hd)):
            T = nm.upper()
            t[nm + "_q"] = gen_codes(rows * cols // 8, s, L, f"AT_{T}_Q")
            t[nm + "_s"] = gen_bf16(rows * cols // g, s, L, f"AT_{T}_S", 0.02)
            t[nm + "_b"] = gen_bf16(rows * cols // g, s, L, f"AT_{T}_B", 0.01)
        t["idx_w"] = gen_bf16((idx_heads * idx_hd + idx_hd) * d, s, L, "AT_IDX_W", 0.02)
        for nm, n in (("q_norm", hd), ("k_norm", hd), ("idx_q_norm", idx_hd), ("idx_k_norm", idx_hd)):
            t[nm] = bf16_to_f32(f32_to_bf16(1.0 + gen_f32(n, s, L, "AT_" + nm.upper(), 0.1)))
        self.t = t
        self._build()

    @classmethod
    def from_arrays(cls, proto, arrays):
        self = cls.__new__(cls)
        self.__dict__.update({k: v for k, v in proto.__dict__.items() if k not in ("t", "st")})
        self.t = {k: np.ascontiguousarray(arrays[k]) for k in cls.KEYS if arrays.get(k) is not None}
        self._build()
        return self

    def _build(self):
        st = OrcAttn()
        st.hidden, st.n_heads, st.n_kv_heads, st.head_dim = self.d, self.h, self.kvh, self.hd
        st.idx_heads, st.idx_head_dim, st.idx_budget, st.idx_compress = self.ih, self.ihd, self.budget, self.compress
        st.kv_cap, st.group_size, st.rotary_factor, st.rope_theta = self.cap, self.g, self.rf, self.theta
        st.slide = 1 if getattr(self, "slide", False) else 0
        for f, a in self.t.items():
            setattr(st, f, _p(a))
        self.st = st

    def arrays(self):
        return dict(self.t)

    class State:
        def __init__(self, A):
            self.k = np.zeros((A.cap, A.kvh * A.hd), np.float32)
            self.v = np.zeros((A.cap, A.kvh * A.hd), np.float32)
            self.idx = np.zeros((A.cap, A.ihd), np.float32)
            self.len = 0
            self.base = 0  # sliding window: position of row 0

    def new_state(self):
        return Attention.State(self)

    def forward(self, x, state, offset, dbg=False):
        """x [n, d] f32 at positions offset..offset+n-1 -> out [n, d]; appends to state.
        With dbg, returns (out, d) where d holds the indexer's pooled keys
        [nb, ihd], queries [n, ih*ihd], block scores and kept flags [n, nb]
        when the call runs the block mask (else an empty dict)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        n = x.shape[0]
        out = np.empty((n, self.d), np.float32)
        S = OrcAttnState(_p(state.k), _p(state.v), _p(state.idx), state.len, state.len, state.base)
        kv = state.len + n
        if self.slide and kv > self.cap:  # the window after the drop (a multiple of compress)
            kv -= (kv - self.cap + self.compress - 1) // self.compress * self.compress
        extra = {}
        D = None
        if dbg and kv > self.budget:
            nb = kv // self.compress
            extra = {"pooled": np.zeros((nb, self.ihd), np.float32),
                     "qs": np.zeros((n, self.ih * self.ihd), np.float32),
                     "scores": np.zeros((n, nb), np.float32),
                     "keep": np.zeros((n, nb), np.uint8)}
            D = OrcAttnDbg(*(_p(extra[k]) for k in ("pooled", "qs", "scores", "keep")))
        rc = lib().orc_attn_forward_dbg(ctypes.byref(self.st), ctypes.byref(S), _p(x), n, offset, _p(out),
                                        ctypes.byref(D) if D is not None else None)
        if rc == -2:
            raise ValueError("the call passes the cache capacity")
        if rc == -3:
            raise ValueError("a sliding call must continue at position base + cached rows")
        if rc:
            raise MemoryError("orc_attn_forward")
        state.len = S.kv_len
        state.base = S.base
        return (out, extra) if dbg else out


def gen_attn_x(n, d, seed, layer=0, std=1.0):
    """attention inputs [n, d] f32 from their own stream"""
    return gen_f32(n * d, seed, layer, "AT_X", std).reshape(n, d)


def dn_decay(a_log, a, dt_bias):
    return lib().orc_dn_decay(a_log, a, dt_bias)


def gen_dn_x(n, d, seed, layer=0, std=1.0):
    """DeltaNet inputs [n, d] f32 from their own stream"""
    return gen_f32(n * d, seed, layer, "DN_X", std).reshape(n, d)


def gen_hyper(n, hc, d, seed, layer=0, std=1.0):
    """hyper states [n, hc*d] f32 from the HYPER stream"""
    return gen_f32(n * hc * d, seed, layer, "HYPER", std).reshape(n, hc * d)


def gen_x(n, H, seed, bf16, layer=0, std=1.0):
    """activations from the X stream: bf16 bits (uint16) or float32"""
    if bf16:
        return gen_bf16(n * H, seed, layer, "X", std).reshape(n, H)
    return gen_f32(n * H, seed, layer, "X", std).reshape(n, H)


def dispatch(idx, E):
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    n, k = idx.shape
    offsets = np.empty(E + 1, np.int32)
    perm = np.empty(max(1, n * k), np.int32)
    pos = np.empty(max(1, n * k), np.int32)
    active = np.empty(E, np.int32)
    na = lib().orc_dispatch(_p(idx), n, k, E, _p(offsets), _p(perm), _p(pos), _p(active))
    return dict(offsets=offsets, perm=perm[: n * k], pos=pos[: n * k], unique=active[:na])


def topk_canonical(x, k):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(k, np.int32)
    lib().orc_topk_canonical(_p(x), len(x), k, _p(out))
    return out


def topk_quickselect(x, k):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(min(k, len(x)), np.int32)
    lib().orc_topk_quickselect(_p(x), len(x), k, _p(out))
    return out


def dequant_q4_f32sb(q, scales, biases, rows, cols, group_size):
    out = np.empty((rows, cols), np.float32)
    lib().orc_dequant_q4_f32sb(_p(np.ascontiguousarray(q, dtype=np.uint32)),
                               _p(np.ascontiguousarray(scales, dtype=np.float32)),
                               _p(np.ascontiguousarray(biases, dtype=np.float32)), rows, cols,
                               group_size, _p(out))
    return out


def gemm_q4_f32sb(A, W, scales, biases, N, K, group_size):
    A = np.ascontiguousarray(A, dtype=np.float32)
    M = A.shape[0]
    C = np.empty((M, N), np.float32)
    lib().orc_gemm_q4_f32sb(M, N, K, _p(A), _p(np.ascontiguousarray(W, dtype=np.uint32)),
                            _p(np.ascontiguousarray(scales, dtype=np.float32)),
                            _p(np.ascontiguousarray(biases, dtype=np.float32)), group_size, _p(C))
    return C


def gemm_fp32(A, W):
    A = np.ascontiguousarray(A, dtype=np.float32)
    W = np.ascontiguousarray(W, dtype=np.float32)
    C = np.empty((A.shape[0], W.shape[0]), np.float32)
    lib().orc_gemm_fp32(A.shape[0], W.shape[0], A.shape[1], _p(A), _p(W), _p(C))
    return C


def gemm_bf16(A, Wbits):
    A = np.ascontiguousarray(A, dtype=np.float32)
    Wbits = np.ascontiguousarray(Wbits, dtype=np.uint16)
    C = np.empty((A.shape[0], Wbits.shape[0]), np.float32)
    lib().orc_gemm_bf16(A.shape[0], Wbits.shape[0], A.shape[1], _p(A), _p(Wbits), _p(C))
    return C


def dot_r64(x, wbits):
    return lib().orc_dot_r64_bf16w(_p(np.ascontiguousarray(x, dtype=np.float32)),
                                   _p(np.ascontiguousarray(wbits, dtype=np.uint16)), len(x))


def sumsq_r64(x):
    return lib().orc_sumsq_r64(_p(np.ascontiguousarray(x, dtype=np.float32)), len(x))


def rmsnorm(x, w, eps, r64=True):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    fn = lib().orc_rmsnorm_r64 if r64 else lib().orc_rmsnorm_seq
    fn(_p(x), None if w is None else _p(np.ascontiguousarray(w, dtype=np.float32)), len(x), eps,
       _p(y))
    return y


def workload_layer(w, layer=0, only_experts=None):
    """host Layer for a qmoe Workload (same seeds/biases the bench uses)"""
    rb = None
    if w.zipf_s > 0:
        rb = zipf_bias(w.n_experts, w.zipf_s, w.zipf_scale, w.seed * 1000003 + layer)
    return Layer(w.hidden, w.n_experts, w.top_k, w.moe_inter, seed=w.seed, layer=layer,
                 with_norm=w.rms_norm, router_bias=rb, group_size=w.group_size,
                 only_experts=only_experts)
