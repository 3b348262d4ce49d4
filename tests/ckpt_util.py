"""Checkpoint writers for the tests: MoE layers in the MLX safetensors layout
(tensor names of c/src/model.c:541-547 and 1902-1912) written with the
safetensors library, and a raw writer for malformed files."""
import json
import os
import struct

import numpy as np

# array key -> (name suffix after "model.layers.<L>.mlp.", shape from (H, E, I, G, GI))
MOE_TENSORS = {
    "router_w": ("gate.weight", lambda H, E, I, G, GI: (E, H)),
    "gate_q": ("switch_mlp.gate_proj.weight", lambda H, E, I, G, GI: (E, I, H // 8)),
    "gate_s": ("switch_mlp.gate_proj.scales", lambda H, E, I, G, GI: (E, I, G)),
    "gate_b": ("switch_mlp.gate_proj.biases", lambda H, E, I, G, GI: (E, I, G)),
    "up_q": ("switch_mlp.up_proj.weight", lambda H, E, I, G, GI: (E, I, H // 8)),
    "up_s": ("switch_mlp.up_proj.scales", lambda H, E, I, G, GI: (E, I, G)),
    "up_b": ("switch_mlp.up_proj.biases", lambda H, E, I, G, GI: (E, I, G)),
    "down_q": ("switch_mlp.down_proj.weight", lambda H, E, I, G, GI: (E, H, I // 8)),
    "down_s": ("switch_mlp.down_proj.scales", lambda H, E, I, G, GI: (E, H, GI)),
    "down_b": ("switch_mlp.down_proj.biases", lambda H, E, I, G, GI: (E, H, GI)),
    "sh_gate_q": ("shared_expert.gate_proj.weight", lambda H, E, I, G, GI: (I, H // 8)),
    "sh_gate_s": ("shared_expert.gate_proj.scales", lambda H, E, I, G, GI: (I, G)),
    "sh_gate_b": ("shared_expert.gate_proj.biases", lambda H, E, I, G, GI: (I, G)),
    "sh_up_q": ("shared_expert.up_proj.weight", lambda H, E, I, G, GI: (I, H // 8)),
    "sh_up_s": ("shared_expert.up_proj.scales", lambda H, E, I, G, GI: (I, G)),
    "sh_up_b": ("shared_expert.up_proj.biases", lambda H, E, I, G, GI: (I, G)),
    "sh_down_q": ("shared_expert.down_proj.weight", lambda H, E, I, G, GI: (H, I // 8)),
    "sh_down_s": ("shared_expert.down_proj.scales", lambda H, E, I, G, GI: (H, GI)),
    "sh_down_b": ("shared_expert.down_proj.biases", lambda H, E, I, G, GI: (H, GI)),
    "sh_gate_w": ("shared_expert_gate.weight", lambda H, E, I, G, GI: (1, H)),
}


# hyper connection: array key -> (suffix after "model.layers.<L>.mlp_hyper_connection.",
# shape from (hc, D=hc*H, R, g)); hc_norm is stored BF16 (mw_load_f32, model.c:275-294)
HC_TENSORS = {
    "hc_norm": ("hc_norm.weight", lambda hc, D, R, g: (D,)),
    "down_q": ("input_mix_weight_down.weight", lambda hc, D, R, g: (R, D // 8)),
    "down_s": ("input_mix_weight_down.scales", lambda hc, D, R, g: (R, D // g)),
    "down_b": ("input_mix_weight_down.biases", lambda hc, D, R, g: (R, D // g)),
    "up_q": ("input_mix_weight_up.weight", lambda hc, D, R, g: (D, R // 8)),
    "up_s": ("input_mix_weight_up.scales", lambda hc, D, R, g: (D, R // g)),
    "up_b": ("input_mix_weight_up.biases", lambda hc, D, R, g: (D, R // g)),
    "inject_w": ("block_inject_weight.weight", lambda hc, D, R, g: (hc, D)),
}


def moe_name(layer, key):
    return f"model.layers.{layer}.mlp.{MOE_TENSORS[key][0]}"


def hc_name(layer, key):
    return f"model.layers.{layer}.mlp_hyper_connection.{HC_TENSORS[key][0]}"


def hc_tensors(arrays, hc, H, R, layer, g=64, drop=()):
    """name -> torch tensor for one layer's hyper connection (hc_norm f32 -> bf16
    bits, exact when the values are bf16-representable)"""
    D = hc * H
    out = {}
    for key, (suffix, shp) in HC_TENSORS.items():
        if key in drop:
            continue
        a = arrays[key]
        if key == "hc_norm":
            a = (np.ascontiguousarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)
        out[hc_name(layer, key)] = _torch_tensor(a, shp(hc, D, R, g))
    return out


def _torch_tensor(a, shape):
    import torch
    a = np.ascontiguousarray(a).reshape(shape)
    if a.dtype == np.uint16:  # bf16 bit patterns
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
    return torch.from_numpy(a.copy())


def write_moe_layer(path, arrays, H, E, I, layer, g=64, shards=2, prefixed_shard=1, drop=(),
                    extra=None, replace=None):
    """writes `arrays` (oracle Layer.arrays() keys) as checkpoint layer
    `layer`, round-robin over `shards` files; names in shard `prefixed_shard`
    get the multimodal "language_model." prefix.  `drop` omits keys,
    `replace` maps name -> torch tensor (after the layer's own), `extra` adds
    unrelated tensors."""
    from safetensors.torch import save_file
    import torch
    os.makedirs(path, exist_ok=True)
    G, GI = H // g, I // g
    tensors = {}
    for key, (suffix, shp) in MOE_TENSORS.items():
        if key in drop:
            continue
        tensors[moe_name(layer, key)] = _torch_tensor(arrays[key], shp(H, E, I, G, GI))
    for nm, t in (replace or {}).items():
        tensors[nm] = t
    if extra is None:
        extra = {
            f"model.layers.{layer}.input_layernorm.weight": torch.ones(H, dtype=torch.bfloat16),
            "model.embed_tokens.weight": torch.zeros((4, H), dtype=torch.bfloat16),
        }
    tensors.update(extra)
    names = sorted(tensors)
    for s in range(shards):
        part = {}
        for i, nm in enumerate(names):
            if i % shards != s:
                continue
            stored = ("language_model." + nm) if s == prefixed_shard else nm
            part[stored] = tensors[nm].contiguous()
        save_file(part, os.path.join(path, f"model-{s + 1:05d}-of-{shards:05d}.safetensors"),
                  metadata={"format": "mlx"})
    return names


def write_raw(path, header, data=b"", header_len=None, pad=0):
    """one safetensors file from a header dict (or a raw JSON string) and data bytes"""
    js = header if isinstance(header, (bytes, str)) else json.dumps(header)
    js = js.encode() if isinstance(js, str) else js
    js = js + b" " * pad
    n = len(js) if header_len is None else header_len
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", n))
        f.write(js)
        f.write(data)
