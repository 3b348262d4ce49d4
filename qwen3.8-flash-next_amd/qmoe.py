"""ctypes binding of libqmoe.so, the MI355X MoE-layer library.

The C ABI (include/qmoe.h) is the product boundary; this module is the thin
Python-side caller used by the tests and the benchmark.  Device buffers are
torch CUDA (HIP) tensors; their data pointers and torch's current HIP stream
are handed to the library unchanged.

The library is the only compute path: if libqmoe.so is missing this module
raises at import time instead of falling back to anything else.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import Optional

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libqmoe.so")

F32, BF16 = 0, 1
RESIDUAL = 1

# synthetic stream tags (include/qmoe.h QMOE_TAG_*)
TAGS = dict(
    ROUTER_W=1, GATE_Q=2, GATE_S=3, GATE_B=4, UP_Q=5, UP_S=6, UP_B=7, DOWN_Q=8, DOWN_S=9,
    DOWN_B=10, SH_GATE_Q=11, SH_GATE_S=12, SH_GATE_B=13, SH_UP_Q=14, SH_UP_S=15, SH_UP_B=16,
    SH_DOWN_Q=17, SH_DOWN_S=18, SH_DOWN_B=19, SHGATE_W=20, X=22,
    HC_DOWN_Q=24, HC_DOWN_S=25, HC_DOWN_B=26, HC_UP_Q=27, HC_UP_S=28, HC_UP_B=29,
    HC_INJECT_W=30, HYPER=31,
)

WEIGHT_FIELDS = [
    "router_w", "router_bias", "gate_q", "gate_s", "gate_b", "up_q", "up_s", "up_b",
    "down_q", "down_s", "down_b", "sh_gate_q", "sh_gate_s", "sh_gate_b", "sh_up_q",
    "sh_up_s", "sh_up_b", "sh_down_q", "sh_down_s", "sh_down_b", "sh_gate_w", "norm_w",
]


class QmoeConfig(ctypes.Structure):
    _fields_ = [
        ("hidden", ctypes.c_int), ("n_experts", ctypes.c_int), ("top_k", ctypes.c_int),
        ("moe_inter", ctypes.c_int), ("group_size", ctypes.c_int), ("n_layers", ctypes.c_int),
        ("max_tokens", ctypes.c_int), ("rms_eps", ctypes.c_float),
    ]


class QmoeErr(ctypes.Structure):
    _fields_ = [("msg", ctypes.c_char * 512)]


class QmoeLayerWeights(ctypes.Structure):
    _fields_ = [(f, ctypes.c_void_p) for f in WEIGHT_FIELDS]


HC_FIELDS = ["hc_norm", "down_q", "down_s", "down_b", "up_q", "up_s", "up_b", "inject_w"]


class QmoeHcWeights(ctypes.Structure):
    _fields_ = [(f, ctypes.c_void_p) for f in HC_FIELDS]


class QmoeStreamStats(ctypes.Structure):
    _fields_ = [(f, ctypes.c_uint64) for f in ("hits", "misses", "evictions", "rejected",
                                               "bytes_in", "prefetched", "prefetch_hits")]


CACHE_LRU, CACHE_LFU, CACHE_ADAPTIVE = 0, 1, 2


class QmoeError(RuntimeError):
    pass


class QmoeDnConfig(ctypes.Structure):
    _fields_ = [(f, ctypes.c_int) for f in ("hidden", "n_k_heads", "n_v_heads", "k_head_dim",
                                            "v_head_dim", "conv_kernel", "group_size", "n_layers",
                                            "max_tokens")]


class QmoeAttnConfig(ctypes.Structure):
    _fields_ = [(f, ctypes.c_int) for f in ("hidden", "n_heads", "n_kv_heads", "head_dim", "idx_heads",
                                            "idx_head_dim", "idx_budget", "idx_compress", "kv_cap",
                                            "group_size")] + \
               [("rotary_factor", ctypes.c_float), ("rope_theta", ctypes.c_float),
                ("n_layers", ctypes.c_int), ("max_tokens", ctypes.c_int), ("max_position", ctypes.c_int),
                ("slide", ctypes.c_int)]


AT_FIELDS = ["q_q", "q_s", "q_b", "k_q", "k_s", "k_b", "v_q", "v_s", "v_b", "o_q", "o_s", "o_b", "idx_w",
             "q_norm", "k_norm", "idx_q_norm", "idx_k_norm"]


class QmoeAttnWeights(ctypes.Structure):
    _fields_ = [(f, ctypes.c_void_p) for f in AT_FIELDS]


DN_FIELDS = ["qkv_q", "qkv_s", "qkv_b", "z_q", "z_s", "z_b", "a_w", "b_w", "out_q", "out_s", "out_b",
             "conv_w", "norm_w", "a_log", "dt_bias"]


class QmoeDnWeights(ctypes.Structure):
    _fields_ = [(f, ctypes.c_void_p) for f in DN_FIELDS]


class QmoeGrConfig(ctypes.Structure):
    _fields_ = [(f, ctypes.c_int) for f in ("hidden", "hc_count", "hc_lowrank", "n_slots", "max_tokens")]


class QmoeStTensor(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int), ("ndim", ctypes.c_int), ("shape", ctypes.c_int64 * 8),
                ("file", ctypes.c_int), ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64)]


# safetensors element types (include/qmoe.h QMOE_ST_*)
ST_DTYPES = ["BOOL", "U8", "I8", "U16", "I16", "U32", "I32", "U64", "I64", "F16", "BF16", "F32", "F64"]


# exported symbols and their signatures (must match include/qmoe.h)
_P = ctypes.c_void_p
_I = ctypes.c_int
SIGNATURES = {
    "qmoe_create": (_I, [ctypes.POINTER(_P), ctypes.POINTER(QmoeConfig), ctypes.POINTER(QmoeErr)]),
    "qmoe_destroy": (None, [_P]),
    "qmoe_upload_layer": (_I, [_P, _I, ctypes.POINTER(QmoeLayerWeights), ctypes.POINTER(QmoeErr)]),
    "qmoe_synth_layer": (_I, [_P, _I, ctypes.c_uint64, _I, _P, ctypes.POINTER(QmoeErr)]),
    "qmoe_layer_device_weights": (_I, [_P, _I, ctypes.POINTER(QmoeLayerWeights), ctypes.POINTER(QmoeErr)]),
    "qmoe_synth_fill": (_I, [_P, ctypes.c_size_t, _I, ctypes.c_uint64, ctypes.c_uint32,
                             ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float, _P,
                             ctypes.POINTER(QmoeErr)]),
    "qmoe_router": (_I, [_P, _I, _P, _I, _I, _P, _P, _P, _P, _P, _P, ctypes.POINTER(QmoeErr)]),
    "qmoe_dispatch": (_I, [_P, _P, _I, _P, _P, _P, _P, ctypes.POINTER(QmoeErr)]),
    "qmoe_expert_gateup": (_I, [_P, _I, _P, _I, _I, _P, _P, _P, _P, ctypes.POINTER(QmoeErr)]),
    "qmoe_expert_down": (_I, [_P, _I, _P, _I, _P, _P, _P, ctypes.POINTER(QmoeErr)]),
    "qmoe_expert_gateup_topk": (_I, [_P, _I, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P,
                                     ctypes.POINTER(QmoeErr)]),
    "qmoe_expert_ffn": (_I, [_P, _I, _P, _I, _I, _P, _P, _P, _P, ctypes.POINTER(QmoeErr)]),
    "qmoe_combine": (_I, [_P, _P, _P, _P, _P, _I, _P, _I, _P, _P, ctypes.POINTER(QmoeErr)]),
    "qmoe_layer_forward": (_I, [_P, _I, _P, _I, _I, _P, _I, _P, ctypes.POINTER(QmoeErr)]),
    "qmoe_layer_forward_noalloc": (_I, [ctypes.POINTER(QmoeConfig), ctypes.POINTER(QmoeLayerWeights), _P,
                                        _I, _I, _P, _I, _P, ctypes.POINTER(QmoeErr)]),
    "qmoe_moe_forward_host": (_I, [_P, _I, _P, _I, _P, ctypes.POINTER(QmoeErr)]),
    "qmoe_attn_create": (_I, [ctypes.POINTER(_P), ctypes.POINTER(QmoeAttnConfig), ctypes.POINTER(QmoeErr)]),
    "qmoe_attn_destroy": (None, [_P]),
    "qmoe_attn_upload_layer": (_I, [_P, _I, ctypes.POINTER(QmoeAttnWeights), ctypes.POINTER(QmoeErr)]),
    "qmoe_attn_reset": (_I, [_P, _I, ctypes.POINTER(QmoeErr)]),
    "qmoe_attn_forward": (_I, [_P, _I, _P, _I, _I, _P, _P, ctypes.POINTER(QmoeErr)]),
    "qmoe_attn_forward_inject": (_I, [_P, _I, _P, _I, _I, _P, _P, _P, _I, _P, ctypes.POINTER(QmoeErr)]),
    "qmoe_attn_cache": (_I, [_P, _I, ctypes.POINTER(_P), ctypes.POINTER(_P), ctypes.POINTER(_P),
                             ctypes.POINTER(_I), ctypes.POINTER(QmoeErr)]),
    "qmoe_attn_index_state": (_I, [_P, _I, ctypes.POINTER(_P), ctypes.POINTER(_P), ctypes.POINTER(_I),
                                   ctypes.POINTER(_P), ctypes.POINTER(_I), ctypes.POINTER(QmoeErr)]),
    "qmoe_gr_create": (_I, [ctypes.POINTER(_P), ctypes.POINTER(QmoeGrConfig), ctypes.POINTER(QmoeErr)]),
    "qmoe_gr_destroy": (None, [_P]),
    "qmoe_gr_upload_slot": (_I, [_P, _I, ctypes.POINTER(QmoeHcWeights), ctypes.POINTER(QmoeErr)]),
    "qmoe_gr_mix": (_I, [_P, _I, _P, _I, _P, _P, _P, ctypes.POINTER(QmoeErr)]),
    "qmoe_gr_inject": (_I, [_P, _P, _P, _I, _P, _P, ctypes.POINTER(QmoeErr)]),
    "qmoe_dn_create": (_I, [ctypes.POINTER(_P), ctypes.POINTER(QmoeDnConfig), ctypes.POINTER(QmoeErr)]),
    "qmoe_dn_destroy": (None, [_P]),
    "qmoe_dn_upload_layer": (_I, [_P, _I, ctypes.POINTER(QmoeDnWeights), ctypes.POINTER(QmoeErr)]),
    "qmoe_dn_reset_state": (_I, [_P, _I, _P, ctypes.POINTER(QmoeErr)]),
    "qmoe_dn_forward": (_I, [_P, _I, _P, _I, _P, _P, ctypes.POINTER(QmoeErr)]),
    "qmoe_dn_forward_inject": (_I, [_P, _I, _P, _I, _P, _P, _P, _I, _P, ctypes.POINTER(QmoeErr)]),
    "qmoe_dn_state": (_I, [_P, _I, ctypes.POINTER(_P), ctypes.POINTER(_P), ctypes.POINTER(QmoeErr)]),
    "qmoe_last_routing": (_I, [_P, _I, _P, _P, _P, _P, _P, _P, _P, ctypes.POINTER(QmoeErr)]),
    "qmoe_scratch_bytes": (ctypes.c_size_t, [_P]),
    "qmoe_layer_bytes": (ctypes.c_size_t, [_P]),
    "qmoe_version": (ctypes.c_char_p, []),
    "qmoe_st_open": (_I, [ctypes.POINTER(_P), ctypes.c_char_p, ctypes.POINTER(QmoeErr)]),
    "qmoe_st_close": (None, [_P]),
    "qmoe_st_count": (ctypes.c_size_t, [_P]),
    "qmoe_st_name": (ctypes.c_char_p, [_P, ctypes.c_size_t]),
    "qmoe_st_find": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(QmoeStTensor)]),
    "qmoe_st_read": (_I, [_P, ctypes.c_char_p, _P, ctypes.c_size_t, ctypes.POINTER(QmoeErr)]),
    "qmoe_st_dtype_size": (_I, [_I]),
    "qmoe_st_dtype_name": (ctypes.c_char_p, [_I]),
    "qmoe_upload_layer_st": (_I, [_P, _I, _P, _I, ctypes.POINTER(QmoeErr)]),
    "qmoe_hc_enable": (_I, [_P, _I, _I, ctypes.POINTER(QmoeErr)]),
    "qmoe_hc_upload_layer": (_I, [_P, _I, ctypes.POINTER(QmoeHcWeights), ctypes.POINTER(QmoeErr)]),
    "qmoe_hc_upload_layer_st": (_I, [_P, _I, _P, _I, ctypes.POINTER(QmoeErr)]),
    "qmoe_hc_synth_layer": (_I, [_P, _I, ctypes.c_uint64, ctypes.POINTER(QmoeErr)]),
    "qmoe_hc_device_weights": (_I, [_P, _I, ctypes.POINTER(QmoeHcWeights), ctypes.POINTER(QmoeErr)]),
    "qmoe_hc_mix": (_I, [_P, _I, _P, _I, _P, _P, _P, _P, ctypes.POINTER(QmoeErr)]),
    "qmoe_hc_inject": (_I, [_P, _P, _P, _I, _P, _P, ctypes.POINTER(QmoeErr)]),
    "qmoe_hc_layer_forward": (_I, [_P, _I, _P, _I, _P, _P, ctypes.POINTER(QmoeErr)]),
    "qmoe_stream_enable": (_I, [_P, _I, _I, _I, ctypes.POINTER(QmoeErr)]),
    "qmoe_stream_get_stats": (_I, [_P, ctypes.POINTER(QmoeStreamStats), ctypes.POINTER(QmoeErr)]),
    "qmoe_xcache_create": (_I, [ctypes.POINTER(_P), _I, _I, _I, _I, ctypes.c_uint64,
                                ctypes.POINTER(QmoeErr)]),
    "qmoe_xcache_destroy": (None, [_P]),
    "qmoe_xcache_peek": (_I, [_P, _I, _I]),
    "qmoe_xcache_get": (_I, [_P, _I, _I]),
    "qmoe_xcache_put": (_I, [_P, _I, _I, _I, _I, ctypes.POINTER(_I)]),
    "qmoe_xcache_pin": (_I, [_P, _I, _I, _I]),
    "qmoe_xcache_mark_hot": (_I, [_P, _I, _I, _I]),
    "qmoe_xcache_clear": (None, [_P, _I]),
    "qmoe_xcache_counts": (None, [_P, ctypes.POINTER(ctypes.c_uint64 * 4)]),
}


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    if not os.path.exists(path):
        raise QmoeError(f"{path} is missing: build it with __graft_entry__.build() "
                        f"(make -C qwen3.8-flash-next_amd/csrc)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        _lib = load_library()
    return _lib


def _ptr(t) -> Optional[int]:
    """device pointer of a torch tensor (or None)"""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream) -> Optional[int]:
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def _check(rc: int, err: QmoeErr, what: str):
    if rc != 0:
        raise QmoeError(f"{what}: {err.msg.decode(errors='replace')}")


def _dtype_code(t) -> int:
    import torch
    if t.dtype == torch.bfloat16:
        return BF16
    if t.dtype == torch.float32:
        return F32
    raise QmoeError(f"activation dtype {t.dtype} unsupported (float32 or bfloat16)")


# ---------------------------------------------------------------- workloads

@dataclass(frozen=True)
class Workload:
    """A synthetic MoE-layer workload (shapes, token count, routing bias)."""
    name: str
    hidden: int
    n_experts: int
    top_k: int
    moe_inter: int
    n_tokens: int
    x_bf16: bool
    zipf_s: float = 0.0        # >0: per-expert Zipf(s) log-popularity bias on the router logits
    zipf_scale: float = 1.0
    n_layers: int = 1
    rms_norm: bool = False     # pre-router RMSNorm (weight ones, eps 1e-6) + residual stream
    seed: int = 0
    group_size: int = 64


WORKLOADS = {
    "tiny": Workload("tiny", 256, 8, 2, 128, 4, x_bf16=False),
    "decode": Workload("decode", 2048, 512, 10, 512, 1, x_bf16=True),
    "batched": Workload("batched", 2048, 512, 10, 512, 64, x_bf16=True, zipf_s=1.1),
    "prefill": Workload("prefill", 2048, 512, 10, 512, 4096, x_bf16=True),
    "depth48": Workload("depth48", 2048, 512, 10, 512, 1, x_bf16=False, zipf_s=1.1,
                        n_layers=48, rms_norm=True),
}


# ------------------------------------------------------------------ context

class MoeContext:
    """Owns a qmoe_ctx: resident layers plus device scratch."""

    def __init__(self, hidden, n_experts, top_k, moe_inter, n_layers=1, max_tokens=1,
                 rms_eps=1e-6, group_size=64):
        self.cfg = QmoeConfig(hidden, n_experts, top_k, moe_inter, group_size, n_layers,
                              max_tokens, rms_eps)
        self.H, self.E, self.k, self.I = hidden, n_experts, top_k, moe_inter
        self.n_layers, self.max_tokens = n_layers, max_tokens
        self._h = ctypes.c_void_p()
        err = QmoeErr()
        _check(lib().qmoe_create(ctypes.byref(self._h), ctypes.byref(self.cfg), ctypes.byref(err)),
               err, "qmoe_create")

    @classmethod
    def for_workload(cls, w: Workload, max_tokens: Optional[int] = None, n_layers=None):
        return cls(w.hidden, w.n_experts, w.top_k, w.moe_inter,
                   n_layers=n_layers or w.n_layers, max_tokens=max_tokens or w.n_tokens,
                   group_size=w.group_size)

    @property
    def handle(self):
        return self._h

    def close(self):
        if self._h:
            lib().qmoe_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def scratch_bytes(self) -> int:
        return lib().qmoe_scratch_bytes(self._h)

    def layer_bytes(self) -> int:
        return lib().qmoe_layer_bytes(self._h)

    # -- weights
    def upload_layer(self, layer: int, host: dict):
        """host: dict of numpy arrays in checkpoint layout (keys = WEIGHT_FIELDS)"""
        import numpy as np
        w = QmoeLayerWeights()
        keep = []
        for f in WEIGHT_FIELDS:
            a = host.get(f)
            if a is None:
                setattr(w, f, None)
                continue
            a = np.ascontiguousarray(a)
            keep.append(a)
            setattr(w, f, a.ctypes.data)
        err = QmoeErr()
        _check(lib().qmoe_upload_layer(self._h, layer, ctypes.byref(w), ctypes.byref(err)), err,
               "qmoe_upload_layer")

    def upload_layer_st(self, layer: int, index: "Checkpoint", model_layer: int):
        """MoE tensors of checkpoint layer `model_layer` -> context layer `layer`"""
        err = QmoeErr()
        _check(lib().qmoe_upload_layer_st(self._h, layer, index.handle, model_layer,
                                          ctypes.byref(err)), err, "qmoe_upload_layer_st")

    def synth_layer(self, layer: int, seed: int, with_norm=False, router_bias=None):
        import numpy as np
        rb = None
        if router_bias is not None:
            rb = np.ascontiguousarray(router_bias, dtype=np.float32)
        err = QmoeErr()
        _check(lib().qmoe_synth_layer(self._h, layer, seed, 1 if with_norm else 0,
                                      None if rb is None else rb.ctypes.data, ctypes.byref(err)),
               err, "qmoe_synth_layer")

    def device_weights(self, layer: int) -> dict:
        w = QmoeLayerWeights()
        err = QmoeErr()
        _check(lib().qmoe_layer_device_weights(self._h, layer, ctypes.byref(w), ctypes.byref(err)),
               err, "qmoe_layer_device_weights")
        return {f: getattr(w, f) for f in WEIGHT_FIELDS}

    # -- stages (torch CUDA tensors in, torch CUDA tensors out)
    def router(self, layer, x, want_logits=False, stream=None):
        import torch
        n = x.shape[0]
        dev = x.device
        logits = torch.empty((n, self.E), dtype=torch.float32, device=dev) if want_logits else None
        idx = torch.empty((n, self.k), dtype=torch.int32, device=dev)
        w = torch.empty((n, self.k), dtype=torch.float32, device=dev)
        sg = torch.empty((n,), dtype=torch.float32, device=dev)
        err = QmoeErr()
        _check(lib().qmoe_router(self._h, layer, _ptr(x), _dtype_code(x), n, _ptr(logits),
                                 _ptr(idx), _ptr(w), _ptr(sg), None, _stream(stream),
                                 ctypes.byref(err)), err, "qmoe_router")
        return dict(logits=logits, idx=idx, w=w, shared_gate=sg)

    def router_norm(self, layer, x, want_logits=True, stream=None):
        """router of a layer with a pre-router RMSNorm; also returns the normalised rows"""
        import torch
        n = x.shape[0]
        dev = x.device
        logits = torch.empty((n, self.E), dtype=torch.float32, device=dev) if want_logits else None
        idx = torch.empty((n, self.k), dtype=torch.int32, device=dev)
        w = torch.empty((n, self.k), dtype=torch.float32, device=dev)
        sg = torch.empty((n,), dtype=torch.float32, device=dev)
        xn = torch.empty((n, self.H), dtype=torch.float32, device=dev)
        err = QmoeErr()
        _check(lib().qmoe_router(self._h, layer, _ptr(x), _dtype_code(x), n, _ptr(logits),
                                 _ptr(idx), _ptr(w), _ptr(sg), _ptr(xn), _stream(stream),
                                 ctypes.byref(err)), err, "qmoe_router")
        return dict(logits=logits, idx=idx, w=w, shared_gate=sg, xn=xn)

    def dispatch(self, idx, stream=None):
        import torch
        n = idx.shape[0]
        dev = idx.device
        offsets = torch.empty((self.E + 1,), dtype=torch.int32, device=dev)
        perm = torch.empty((max(1, n * self.k),), dtype=torch.int32, device=dev)
        segments = torch.empty((3 * self.E + 1,), dtype=torch.int32, device=dev)
        err = QmoeErr()
        _check(lib().qmoe_dispatch(self._h, _ptr(idx), n, _ptr(offsets), _ptr(perm),
                                   _ptr(segments), _stream(stream), ctypes.byref(err)), err,
               "qmoe_dispatch")
        return dict(offsets=offsets, perm=perm[: n * self.k], segments=segments)

    def expert_gateup(self, layer, x, d, stream=None, out=None):
        import torch
        n = x.shape[0]
        h = out if out is not None else torch.empty((n * self.k + n, self.I), dtype=torch.float32,
                                                    device=x.device)
        err = QmoeErr()
        _check(lib().qmoe_expert_gateup(self._h, layer, _ptr(x), _dtype_code(x), n, _ptr(d["perm"]),
                                        _ptr(d["segments"]), _ptr(h), _stream(stream),
                                        ctypes.byref(err)), err, "qmoe_expert_gateup")
        return h

    def expert_gateup_topk(self, layer, x, logits, stream=None):
        """one token: top-k of `logits` ([E+1]: router logits, then the
        shared-expert gate logit), dispatch and gate/up in one launch"""
        import torch
        dev = x.device
        k = self.k
        out = dict(idx=torch.empty((1, k), dtype=torch.int32, device=dev),
                   w=torch.empty((1, k), dtype=torch.float32, device=dev),
                   shared_gate=torch.empty((1,), dtype=torch.float32, device=dev),
                   perm=torch.empty((k,), dtype=torch.int32, device=dev),
                   segments=torch.zeros((3 * self.E + 1,), dtype=torch.int32, device=dev),
                   h=torch.empty((k + 1, self.I), dtype=torch.float32, device=dev))
        self.expert_gateup_topk_raw(layer, x, logits, out, stream)
        return out

    def expert_gateup_topk_raw(self, layer, x, logits, out, stream=None):
        """as expert_gateup_topk, into preallocated buffers (graph capture)"""
        err = QmoeErr()
        _check(lib().qmoe_expert_gateup_topk(self._h, layer, _ptr(x), _dtype_code(x), _ptr(logits),
                                             _ptr(out["idx"]), _ptr(out["w"]),
                                             _ptr(out["shared_gate"]), _ptr(out["perm"]),
                                             _ptr(out["segments"]), _ptr(out["h"]),
                                             _stream(stream), ctypes.byref(err)), err,
               "qmoe_expert_gateup_topk")

    def expert_down(self, layer, h, n, d, stream=None, out=None):
        import torch
        y = out if out is not None else torch.empty((n * self.k + n, self.H), dtype=torch.float32,
                                                    device=h.device)
        err = QmoeErr()
        _check(lib().qmoe_expert_down(self._h, layer, _ptr(h), n, _ptr(d["segments"]), _ptr(y),
                                      _stream(stream), ctypes.byref(err)), err, "qmoe_expert_down")
        return y

    def expert_ffn(self, layer, x, d, stream=None):
        import torch
        n = x.shape[0]
        y = torch.empty((n * self.k + n, self.H), dtype=torch.float32, device=x.device)
        err = QmoeErr()
        _check(lib().qmoe_expert_ffn(self._h, layer, _ptr(x), _dtype_code(x), n, _ptr(d["perm"]),
                                     _ptr(d["segments"]), _ptr(y), _stream(stream),
                                     ctypes.byref(err)), err, "qmoe_expert_ffn")
        return y

    def combine(self, y, perm, w, shared_gate, n, x_residual=None, stream=None):
        import torch
        out = torch.empty((n, self.H), dtype=torch.float32, device=y.device)
        err = QmoeErr()
        xd = _dtype_code(x_residual) if x_residual is not None else F32
        _check(lib().qmoe_combine(self._h, _ptr(y), _ptr(perm), _ptr(w), _ptr(shared_gate), n,
                                  _ptr(x_residual), xd, _ptr(out), _stream(stream),
                                  ctypes.byref(err)), err, "qmoe_combine")
        return out

    def layer_forward(self, layer, x, out=None, residual=False, stream=None):
        import torch
        n = x.shape[0]
        if out is None:
            out = torch.empty((n, self.H), dtype=torch.float32, device=x.device)
        err = QmoeErr()
        _check(lib().qmoe_layer_forward(self._h, layer, _ptr(x), _dtype_code(x), n, _ptr(out),
                                        RESIDUAL if residual else 0, _stream(stream),
                                        ctypes.byref(err)), err, "qmoe_layer_forward")
        return out

    def layer_forward_raw(self, layer, x_ptr, x_dtype, n, out_ptr, flags, stream_handle):
        """no-allocation variant for timing loops; returns the rc and message"""
        err = QmoeErr()
        rc = lib().qmoe_layer_forward(self._h, layer, x_ptr, x_dtype, n, out_ptr, flags,
                                      stream_handle, ctypes.byref(err))
        return rc, err.msg.decode(errors="replace")

    def last_routing(self, n, stream=None):
        """routing of the last layer_forward call (device tensors)"""
        import torch
        dev = torch.device("cuda", torch.cuda.current_device())
        r = dict(idx=torch.empty((n, self.k), dtype=torch.int32, device=dev),
                 w=torch.empty((n, self.k), dtype=torch.float32, device=dev),
                 shared_gate=torch.empty((n,), dtype=torch.float32, device=dev),
                 offsets=torch.empty((self.E + 1,), dtype=torch.int32, device=dev),
                 perm=torch.empty((n * self.k,), dtype=torch.int32, device=dev),
                 segments=torch.empty((3 * self.E + 1,), dtype=torch.int32, device=dev))
        err = QmoeErr()
        _check(lib().qmoe_last_routing(self._h, n, _ptr(r["idx"]), _ptr(r["w"]),
                                       _ptr(r["shared_gate"]), _ptr(r["offsets"]), _ptr(r["perm"]),
                                       _ptr(r["segments"]), _stream(stream), ctypes.byref(err)),
               err, "qmoe_last_routing")
        return r

    # -- expert streaming
    def stream_enable(self, slots_per_layer: int, policy: int = CACHE_ADAPTIVE, prefetch: int = 0):
        err = QmoeErr()
        _check(lib().qmoe_stream_enable(self._h, slots_per_layer, policy, prefetch,
                                        ctypes.byref(err)), err, "qmoe_stream_enable")

    def stream_stats(self) -> dict:
        st = QmoeStreamStats()
        err = QmoeErr()
        _check(lib().qmoe_stream_get_stats(self._h, ctypes.byref(st), ctypes.byref(err)), err,
               "qmoe_stream_get_stats")
        return {f: getattr(st, f) for f, _ in QmoeStreamStats._fields_}

    # -- MLP hyper connection around the layer
    def hc_enable(self, hc_count: int, hc_lowrank: int):
        err = QmoeErr()
        _check(lib().qmoe_hc_enable(self._h, hc_count, hc_lowrank, ctypes.byref(err)), err,
               "qmoe_hc_enable")
        self.hc, self.hc_R = hc_count, hc_lowrank

    def hc_upload_layer(self, layer: int, host: dict):
        """host: numpy arrays keyed by HC_FIELDS (hc_norm f32, codes u32, bf16 bits u16)"""
        import numpy as np
        w = QmoeHcWeights()
        keep = []
        for f in HC_FIELDS:
            a = host.get(f)
            if a is not None:
                a = np.ascontiguousarray(a)
                keep.append(a)
            setattr(w, f, None if a is None else a.ctypes.data)
        err = QmoeErr()
        _check(lib().qmoe_hc_upload_layer(self._h, layer, ctypes.byref(w), ctypes.byref(err)), err,
               "qmoe_hc_upload_layer")

    def hc_upload_layer_st(self, layer: int, index: "Checkpoint", model_layer: int):
        err = QmoeErr()
        _check(lib().qmoe_hc_upload_layer_st(self._h, layer, index.handle, model_layer,
                                             ctypes.byref(err)), err, "qmoe_hc_upload_layer_st")

    def hc_synth_layer(self, layer: int, seed: int):
        err = QmoeErr()
        _check(lib().qmoe_hc_synth_layer(self._h, layer, seed, ctypes.byref(err)), err,
               "qmoe_hc_synth_layer")

    def hc_device_weights(self, layer: int) -> dict:
        w = QmoeHcWeights()
        err = QmoeErr()
        _check(lib().qmoe_hc_device_weights(self._h, layer, ctypes.byref(w), ctypes.byref(err)),
               err, "qmoe_hc_device_weights")
        return {f: getattr(w, f) for f in HC_FIELDS}

    def hc_mix(self, layer, hyper, stream=None):
        """gated_residual: hyper [n, hc*H] f32 -> dict(mixed, inject, normed)"""
        import torch
        n = hyper.shape[0]
        dev = hyper.device
        r = dict(mixed=torch.empty((n, self.H), dtype=torch.float32, device=dev),
                 inject=torch.empty((n, self.hc), dtype=torch.float32, device=dev),
                 normed=torch.empty((n, self.hc * self.H), dtype=torch.float32, device=dev))
        err = QmoeErr()
        _check(lib().qmoe_hc_mix(self._h, layer, _ptr(hyper), n, _ptr(r["mixed"]), _ptr(r["inject"]),
                                 _ptr(r["normed"]), _stream(stream), ctypes.byref(err)), err,
               "qmoe_hc_mix")
        return r

    def hc_inject(self, inject, moe_out, hyper, stream=None):
        """hyper[t, j] += inject[t, j] * moe_out[t], in place"""
        err = QmoeErr()
        _check(lib().qmoe_hc_inject(self._h, _ptr(inject), _ptr(moe_out), hyper.shape[0],
                                    _ptr(hyper), _stream(stream), ctypes.byref(err)), err,
               "qmoe_hc_inject")
        return hyper

    def hc_layer_forward(self, layer, hyper, want_out=True, stream=None):
        """mix, the MoE layer and the inject update; hyper is updated in place.
        Returns the MoE output [n, H] (or None)."""
        import torch
        n = hyper.shape[0]
        out = torch.empty((n, self.H), dtype=torch.float32, device=hyper.device) if want_out else None
        err = QmoeErr()
        _check(lib().qmoe_hc_layer_forward(self._h, layer, _ptr(hyper), n, _ptr(out),
                                           _stream(stream), ctypes.byref(err)), err,
               "qmoe_hc_layer_forward")
        return out

    def hc_layer_forward_raw(self, layer, hyper_ptr, n, out_ptr, stream_handle):
        """no-allocation variant for timing loops; returns the rc and message"""
        err = QmoeErr()
        rc = lib().qmoe_hc_layer_forward(self._h, layer, hyper_ptr, n, out_ptr, stream_handle,
                                         ctypes.byref(err))
        return rc, err.msg.decode(errors="replace")

    def forward_host(self, layer, x):
        """moe_forward's host contract: numpy f32 [n,H] in, numpy f32 [n,H] out"""
        import numpy as np
        x = np.ascontiguousarray(x, dtype=np.float32)
        n = x.shape[0]
        out = np.empty((n, self.H), dtype=np.float32)
        err = QmoeErr()
        _check(lib().qmoe_moe_forward_host(self._h, layer, x.ctypes.data, n, out.ctypes.data,
                                           ctypes.byref(err)), err, "qmoe_moe_forward_host")
        return out


class Checkpoint:
    """index over the *.safetensors files of a directory (qmoe_st_*); host only"""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        err = QmoeErr()
        _check(lib().qmoe_st_open(ctypes.byref(h), os.fsencode(path), ctypes.byref(err)), err,
               "qmoe_st_open")
        self._h = h.value

    @property
    def handle(self):
        return self._h

    def close(self):
        if self._h:
            lib().qmoe_st_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def names(self) -> list:
        n = lib().qmoe_st_count(self._h)
        return [lib().qmoe_st_name(self._h, i).decode() for i in range(n)]

    def info(self, name: str) -> Optional[dict]:
        t = QmoeStTensor()
        if not lib().qmoe_st_find(self._h, name.encode(), ctypes.byref(t)):
            return None
        return dict(dtype=ST_DTYPES[t.dtype], shape=tuple(t.shape[:t.ndim]), file=t.file,
                    offset=t.offset, nbytes=t.nbytes)

    def read(self, name: str) -> bytes:
        t = QmoeStTensor()
        if not lib().qmoe_st_find(self._h, name.encode(), ctypes.byref(t)):
            raise QmoeError(f"missing tensor {name}")
        buf = ctypes.create_string_buffer(max(int(t.nbytes), 1))
        err = QmoeErr()
        _check(lib().qmoe_st_read(self._h, name.encode(), buf, len(buf), ctypes.byref(err)), err,
               "qmoe_st_read")
        return buf.raw[:t.nbytes]


class ExpertCache:
    """the library's expert slot cache on its own (host only): partitions of
    `slots` entries over items 0..items-1"""

    def __init__(self, parts, items, slots, policy, entry_bytes):
        self._h = ctypes.c_void_p()
        err = QmoeErr()
        _check(lib().qmoe_xcache_create(ctypes.byref(self._h), parts, items, slots, policy,
                                        entry_bytes, ctypes.byref(err)), err, "qmoe_xcache_create")

    def close(self):
        if self._h:
            lib().qmoe_xcache_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def peek(self, part, item):
        return lib().qmoe_xcache_peek(self._h, part, item)

    def get(self, part, item):
        return lib().qmoe_xcache_get(self._h, part, item)

    def put(self, part, item, pin=False, hot=False):
        ev = ctypes.c_int(-1)
        slot = lib().qmoe_xcache_put(self._h, part, item, int(pin), int(hot), ctypes.byref(ev))
        return slot, ev.value

    def pin(self, part, item, pinned):
        return lib().qmoe_xcache_pin(self._h, part, item, int(pinned))

    def mark_hot(self, part, item, hot):
        return lib().qmoe_xcache_mark_hot(self._h, part, item, int(hot))

    def clear(self, part):
        lib().qmoe_xcache_clear(self._h, part)

    def counts(self):
        out = (ctypes.c_uint64 * 4)()
        lib().qmoe_xcache_counts(self._h, ctypes.byref(out))
        return dict(hits=out[0], misses=out[1], evictions=out[2], rejected=out[3])


class AttentionContext:
    """Owns a qmoe_attn_ctx: the full-attention mixer's resident layers
    (weights, k/v and indexer caches) plus device scratch."""

    def __init__(self, hidden, n_heads, n_kv_heads, head_dim, idx_heads, idx_head_dim, idx_budget,
                 idx_compress, kv_cap=2048, rotary_factor=0.25, rope_theta=1e7, n_layers=1,
                 max_tokens=1, group_size=64, max_position=0, slide=False):
        self.cfg = QmoeAttnConfig(hidden, n_heads, n_kv_heads, head_dim, idx_heads, idx_head_dim,
                                  idx_budget, idx_compress, kv_cap, group_size, rotary_factor,
                                  rope_theta, n_layers, max_tokens, max_position, 1 if slide else 0)
        self.d, self.h, self.kvh, self.hd = hidden, n_heads, n_kv_heads, head_dim
        self.ihd, self.cap = idx_head_dim, kv_cap
        self._h = ctypes.c_void_p()
        err = QmoeErr()
        _check(lib().qmoe_attn_create(ctypes.byref(self._h), ctypes.byref(self.cfg), ctypes.byref(err)),
               err, "qmoe_attn_create")

    def close(self):
        if self._h:
            lib().qmoe_attn_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def upload_layer(self, layer: int, host: dict):
        """host: numpy arrays keyed by AT_FIELDS"""
        import numpy as np
        w = QmoeAttnWeights()
        keep = []
        for f in AT_FIELDS:
            a = host.get(f)
            if a is not None:
                a = np.ascontiguousarray(a)
                keep.append(a)
            setattr(w, f, None if a is None else a.ctypes.data)
        err = QmoeErr()
        _check(lib().qmoe_attn_upload_layer(self._h, layer, ctypes.byref(w), ctypes.byref(err)), err,
               "qmoe_attn_upload_layer")

    def reset(self, layer=-1):
        err = QmoeErr()
        _check(lib().qmoe_attn_reset(self._h, layer, ctypes.byref(err)), err, "qmoe_attn_reset")

    def forward(self, layer, x, offset, out=None, stream=None):
        """x [n, d] f32 CUDA tensor at positions offset.. -> out [n, d]"""
        import torch
        n = x.shape[0]
        if out is None:
            out = torch.empty((n, self.d), dtype=torch.float32, device=x.device)
        err = QmoeErr()
        _check(lib().qmoe_attn_forward(self._h, layer, _ptr(x), n, offset, _ptr(out), _stream(stream),
                                       ctypes.byref(err)), err, "qmoe_attn_forward")
        return out

    def forward_inject(self, layer, x, offset, hyper, inject, out=None, stream=None):
        """forward, then hyper[t, j] += inject[t, j] * out[t] (the gated
        residual's update) in the same launches; hyper [n, hc*d] and inject
        [n, hc] f32 CUDA tensors; out is written only when given"""
        n, hc = x.shape[0], inject.shape[1]
        err = QmoeErr()
        _check(lib().qmoe_attn_forward_inject(self._h, layer, _ptr(x), n, offset,
                                              _ptr(out), _ptr(hyper),
                                              _ptr(inject), hc, _stream(stream), ctypes.byref(err)),
               err, "qmoe_attn_forward_inject")
        return out

    def forward_raw(self, layer, x_ptr, n, offset, out_ptr, stream_handle):
        err = QmoeErr()
        rc = lib().qmoe_attn_forward(self._h, layer, x_ptr, n, offset, out_ptr, stream_handle,
                                     ctypes.byref(err))
        return rc, err.msg.decode(errors="replace")

    def cache(self, layer):
        """device addresses (k, v, indexer keys) and the cached length"""
        k, v, i = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
        ln = ctypes.c_int()
        err = QmoeErr()
        _check(lib().qmoe_attn_cache(self._h, layer, ctypes.byref(k), ctypes.byref(v), ctypes.byref(i),
                                     ctypes.byref(ln), ctypes.byref(err)), err, "qmoe_attn_cache")
        return k.value, v.value, i.value, ln.value

    def index_state(self, layer):
        """device addresses of the indexer's pooled block keys, the last
        masked call's kept-block bitmap and block-score order keys, with the
        bitmap's words and the score keys' row stride"""
        p, k, s = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
        kw, ld = ctypes.c_int(), ctypes.c_int()
        err = QmoeErr()
        _check(lib().qmoe_attn_index_state(self._h, layer, ctypes.byref(p), ctypes.byref(k), ctypes.byref(kw),
                                           ctypes.byref(s), ctypes.byref(ld), ctypes.byref(err)),
               err, "qmoe_attn_index_state")
        return p.value, k.value, kw.value, s.value, ld.value


class DeltaNetContext:
    """Owns a qmoe_dn_ctx: the gated DeltaNet mixer's resident layers (weights
    and conv/recurrent states) plus device scratch."""

    def __init__(self, hidden, n_k_heads, n_v_heads, k_head_dim, v_head_dim, conv_kernel=4,
                 n_layers=1, max_tokens=1, group_size=64):
        self.cfg = QmoeDnConfig(hidden, n_k_heads, n_v_heads, k_head_dim, v_head_dim, conv_kernel,
                                group_size, n_layers, max_tokens)
        self.d, self.hk, self.hv, self.dk, self.dv, self.kc = (hidden, n_k_heads, n_v_heads,
                                                              k_head_dim, v_head_dim, conv_kernel)
        self.conv_dim = 2 * n_k_heads * k_head_dim + n_v_heads * v_head_dim
        self._h = ctypes.c_void_p()
        err = QmoeErr()
        _check(lib().qmoe_dn_create(ctypes.byref(self._h), ctypes.byref(self.cfg), ctypes.byref(err)),
               err, "qmoe_dn_create")

    def close(self):
        if self._h:
            lib().qmoe_dn_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def upload_layer(self, layer: int, host: dict):
        """host: numpy arrays keyed by DN_FIELDS (codes u32, bf16 bits u16, f32)"""
        import numpy as np
        w = QmoeDnWeights()
        keep = []
        for f in DN_FIELDS:
            a = host.get(f)
            if a is not None:
                a = np.ascontiguousarray(a)
                keep.append(a)
            setattr(w, f, None if a is None else a.ctypes.data)
        err = QmoeErr()
        _check(lib().qmoe_dn_upload_layer(self._h, layer, ctypes.byref(w), ctypes.byref(err)), err,
               "qmoe_dn_upload_layer")

    def reset_state(self, layer=-1, stream=None):
        err = QmoeErr()
        _check(lib().qmoe_dn_reset_state(self._h, layer, _stream(stream), ctypes.byref(err)), err,
               "qmoe_dn_reset_state")

    def forward(self, layer, x, out=None, stream=None):
        """x [n, d] f32 CUDA tensor -> out [n, d] f32; the layer's states advance by n tokens"""
        import torch
        n = x.shape[0]
        if out is None:
            out = torch.empty((n, self.d), dtype=torch.float32, device=x.device)
        err = QmoeErr()
        _check(lib().qmoe_dn_forward(self._h, layer, _ptr(x), n, _ptr(out), _stream(stream),
                                     ctypes.byref(err)), err, "qmoe_dn_forward")
        return out

    def forward_inject(self, layer, x, hyper, inject, out=None, stream=None):
        """forward, then hyper[t, j] += inject[t, j] * out[t] (the gated
        residual's update) in the same launches; hyper [n, hc*d] and inject
        [n, hc] f32 CUDA tensors; out is written only when given"""
        n, hc = x.shape[0], inject.shape[1]
        err = QmoeErr()
        _check(lib().qmoe_dn_forward_inject(self._h, layer, _ptr(x), n,
                                            _ptr(out), _ptr(hyper),
                                            _ptr(inject), hc, _stream(stream), ctypes.byref(err)),
               err, "qmoe_dn_forward_inject")
        return out

    def forward_raw(self, layer, x_ptr, n, out_ptr, stream_handle):
        """no-allocation variant for timing loops; returns the rc and message"""
        err = QmoeErr()
        rc = lib().qmoe_dn_forward(self._h, layer, x_ptr, n, out_ptr, stream_handle, ctypes.byref(err))
        return rc, err.msg.decode(errors="replace")

    def state_ptrs(self, layer):
        conv, rec = ctypes.c_void_p(), ctypes.c_void_p()
        err = QmoeErr()
        _check(lib().qmoe_dn_state(self._h, layer, ctypes.byref(conv), ctypes.byref(rec),
                                   ctypes.byref(err)), err, "qmoe_dn_state")
        return conv.value, rec.value

    def state_shapes(self):
        return (self.kc - 1, self.conv_dim), (self.hv, self.dv, self.dk)


class GatedResidualContext:
    """Owns a qmoe_gr_ctx: weight slots of gated_residual for the
    attention-block hyper connections (with inject) and the final mixer
    (without), plus device scratch."""

    def __init__(self, hidden, hc_count, hc_lowrank, n_slots=1, max_tokens=1):
        self.cfg = QmoeGrConfig(hidden, hc_count, hc_lowrank, n_slots, max_tokens)
        self.d, self.hc, self.R = hidden, hc_count, hc_lowrank
        self.has_inject = [False] * n_slots
        self._h = ctypes.c_void_p()
        err = QmoeErr()
        _check(lib().qmoe_gr_create(ctypes.byref(self._h), ctypes.byref(self.cfg), ctypes.byref(err)),
               err, "qmoe_gr_create")

    def close(self):
        if self._h:
            lib().qmoe_gr_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def upload_slot(self, slot: int, host: dict):
        """host: numpy arrays keyed by HC_FIELDS; no "inject_w" (or None)
        makes a slot without inject (the final mixer)"""
        import numpy as np
        w = QmoeHcWeights()
        keep = []
        for f in HC_FIELDS:
            a = host.get(f)
            if a is not None:
                a = np.ascontiguousarray(a)
                keep.append(a)
            setattr(w, f, None if a is None else a.ctypes.data)
        err = QmoeErr()
        _check(lib().qmoe_gr_upload_slot(self._h, slot, ctypes.byref(w), ctypes.byref(err)), err,
               "qmoe_gr_upload_slot")
        self.has_inject[slot] = host.get("inject_w") is not None

    def mix(self, slot, hyper, mixed=None, inject=None, want_inject=None, stream=None):
        """hyper [n, hc*d] f32 CUDA tensor -> (mixed [n, d], inject [n, hc] or None);
        the inject is formed when the slot has inject weights (or want_inject)"""
        import torch
        n = hyper.shape[0]
        if want_inject is None:  # a slot out of range is the library's error to report
            want_inject = 0 <= slot < len(self.has_inject) and self.has_inject[slot]
        if mixed is None:
            mixed = torch.empty((n, self.d), dtype=torch.float32, device=hyper.device)
        if want_inject and inject is None:
            inject = torch.empty((n, self.hc), dtype=torch.float32, device=hyper.device)
        err = QmoeErr()
        _check(lib().qmoe_gr_mix(self._h, slot, _ptr(hyper), n, _ptr(mixed),
                                 _ptr(inject) if want_inject else None, _stream(stream),
                                 ctypes.byref(err)), err, "qmoe_gr_mix")
        return mixed, inject if want_inject else None

    def inject(self, inject, out, hyper, stream=None):
        """hyper[t, j] += inject[t, j] * out[t], in place"""
        err = QmoeErr()
        _check(lib().qmoe_gr_inject(self._h, _ptr(inject), _ptr(out), hyper.shape[0], _ptr(hyper),
                                    _stream(stream), ctypes.byref(err)), err, "qmoe_gr_inject")
        return hyper


def decoder_layer_types(n_layers, full_attention_interval=4):
    """per-layer mixer kinds of the model's text stack: every
    full_attention_interval-th layer full attention, the others gated
    DeltaNet (src/colibri_runtime/model.py:138-143, c/src/model.c:124)"""
    return ["attn" if (l + 1) % full_attention_interval == 0 else "dn" for l in range(n_layers)]


class DecoderStack:
    """The decoder layer loop of model_forward (c/src/model.c:1644-1745) on
    the library's parts, for n tokens of hyper state [n, hc*d] f32 updated
    in place.  Layer l: the attention block's hyper connection (slot l of
    `gr`: gated_residual with inject, model.c:1671-1672), its mixer (gated
    DeltaNet, layer l of `dn`, or full attention with the QSA indexer,
    layer l of `at`, at positions offset..) with the inject update hyper +=
    inject (x) out (model.c:1699-1707) fused into its last launch
    (forward_inject), then the MLP hyper connection, the
    MoE layer and its inject update (layer l of `moe`,
    qmoe_hc_layer_forward, model.c:1710-1731).  After the last layer the
    final mixer (slot len(types) of `gr`, no inject, model.c:1743-1745)
    gives the LM head's input.  Buffers are allocated once, so a HIP graph
    can capture step()."""

    def __init__(self, gr, moe, dn, at, types, n, device="cuda"):
        import torch
        self.gr, self.moe, self.dn, self.at, self.types = gr, moe, dn, at, list(types)
        d, hc = gr.d, gr.hc
        self.mixed = torch.empty((n, d), dtype=torch.float32, device=device)
        self.inject = torch.empty((n, hc), dtype=torch.float32, device=device)
        self.final = torch.empty((n, d), dtype=torch.float32, device=device)

    def step(self, hyper, offset):
        """hyper [n, hc*d] at positions offset.. through every layer; returns
        the final mixer's output [n, d] (a buffer reused by the next step)"""
        L = len(self.types)
        for l, t in enumerate(self.types):
            self.gr.mix(l, hyper, mixed=self.mixed, inject=self.inject, want_inject=True)
            # the mixer with the gated residual's update fused into its last launch
            if t == "dn":
                self.dn.forward_inject(l, self.mixed, hyper, self.inject)
            else:
                self.at.forward_inject(l, self.mixed, offset, hyper, self.inject)
            self.moe.hc_layer_forward(l, hyper, want_out=False)
        self.gr.mix(L, hyper, mixed=self.final, want_inject=False)
        return self.final


def synth_fill(t, kind: int, seed: int, layer: int, tag: int, start=0, stddev=1.0, stream=None):
    """fill a torch CUDA tensor with a synthetic stream (kind 0 bf16 normal, 1 f32 normal, 2 codes)"""
    err = QmoeErr()
    _check(lib().qmoe_synth_fill(_ptr(t), t.numel(), kind, seed, layer, tag, start, stddev,
                                 _stream(stream), ctypes.byref(err)), err, "qmoe_synth_fill")
    return t


def version() -> str:
    return lib().qmoe_version().decode()
