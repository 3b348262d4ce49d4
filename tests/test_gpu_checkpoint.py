"""Checkpoint upload (qmoe_upload_layer_st) on the GPU: a layer written in
the MLX safetensors layout and uploaded from the file lands in HBM byte for
byte as the same arrays uploaded from memory, and the layer's output on the
golden input is the golden output (and bit-identical to the in-memory
upload); the reference's loader rules hold (model.c:213-272): a missing
.biases reads as zero, a quantized router or shared-expert gate, dense
expert weights, a wrong shape or dtype are refused before any copy."""
import ctypes
import os

import numpy as np
import pytest

from ckpt_util import MOE_TENSORS, moe_name, write_moe_layer
from conftest import load_oracle, load_pkg

orc = load_oracle()
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

pytestmark = pytest.mark.gpu

H, E, K, I = 256, 8, 2, 128
MAX_ABS, REL_L2 = 2e-2, 1e-3


def say(msg):
    print(msg, flush=True)


def device_bytes(ptr, nbytes):
    buf = np.empty(nbytes, np.uint8)
    rc = ctypes.CDLL("libamdhip64.so").hipMemcpy(ctypes.c_void_p(buf.ctypes.data),
                                                 ctypes.c_void_p(ptr), ctypes.c_size_t(nbytes), 2)
    assert rc == 0
    return buf


@pytest.fixture(scope="module")
def torch_dev(gpu):
    import torch
    return torch, gpu


def test_upload_from_checkpoint_matches_memory_upload(torch_dev, tmp_path):
    torch, dev = torch_dev
    pkg = load_pkg()
    say("case: tiny layer written as checkpoint layer 5 (3 shards), uploaded to context layer 1")
    L = orc.Layer(H, E, K, I, seed=0)
    arrays = L.arrays()
    write_moe_layer(str(tmp_path), arrays, H, E, I, layer=5, shards=3, prefixed_shard=2)
    g = np.load(os.path.join(GOLDEN, "tiny_layer.npz"))
    with pkg.Checkpoint(str(tmp_path)) as ck, \
            pkg.MoeContext(H, E, K, I, n_layers=2, max_tokens=4) as ctx:
        ctx.upload_layer_st(1, ck, 5)
        ctx.upload_layer(0, arrays)
        dw1, dw0 = ctx.device_weights(1), ctx.device_weights(0)
        for key in MOE_TENSORS:
            a = np.ascontiguousarray(arrays[key])
            got = device_bytes(dw1[key], a.nbytes)
            assert got.tobytes() == a.tobytes(), key
        assert dw1["router_bias"] is None and dw1["norm_w"] is None
        x = torch.from_numpy(np.array(g["x"])).to(dev)
        out1 = ctx.layer_forward(1, x)
        out0 = ctx.layer_forward(0, x)
        torch.cuda.synchronize()
        o1 = out1.cpu().numpy()
        assert np.array_equal(o1, out0.cpu().numpy())
        err = float(np.abs(o1 - g["out"]).max())
        rel = float(np.linalg.norm(o1 - g["out"]) / np.linalg.norm(g["out"]))
        say(f"checkpoint layer vs golden: max-abs {err:.3e} rel-L2 {rel:.3e}")
        assert err < MAX_ABS and rel < REL_L2


def test_missing_biases_read_as_zero(torch_dev, tmp_path):
    torch, dev = torch_dev
    pkg = load_pkg()
    say("case: checkpoint without switch_mlp.down_proj.biases and shared_expert.up_proj.biases")
    arrays = orc.Layer(H, E, K, I, seed=4).arrays()
    write_moe_layer(str(tmp_path), arrays, H, E, I, layer=0, drop=("down_b", "sh_up_b"))
    zeroed = dict(arrays)
    zeroed["down_b"] = np.zeros_like(arrays["down_b"])
    zeroed["sh_up_b"] = np.zeros_like(arrays["sh_up_b"])
    ref = orc.Layer.from_arrays(H, E, K, I, zeroed)
    x = orc.gen_x(4, H, 11, bf16=False)
    with pkg.Checkpoint(str(tmp_path)) as ck, pkg.MoeContext(H, E, K, I, max_tokens=4) as ctx:
        ctx.synth_layer(0, 77)  # stale contents that the upload must overwrite
        ctx.upload_layer_st(0, ck, 0)
        dw = ctx.device_weights(0)
        assert not device_bytes(dw["down_b"], arrays["down_b"].nbytes).any()
        assert not device_bytes(dw["sh_up_b"], arrays["sh_up_b"].nbytes).any()
        out = ctx.layer_forward(0, torch.from_numpy(x).to(dev))
        torch.cuda.synchronize()
        want = ref.forward(x, False)["out"]
        got = out.cpu().numpy()
        err = float(np.abs(got - want).max())
        say(f"zero-bias checkpoint vs oracle: max-abs {err:.3e}")
        assert err < MAX_ABS


@pytest.mark.parametrize("case,needle", [
    ("quant_router", "must be dense BF16"),
    ("dense_expert", "dense expert weights are not supported"),
    ("wrong_E", "has shape [4,256]"),
    ("scales_f16", "must be BF16 (got F16)"),
    ("missing_layer", "missing tensor model.layers.9.mlp.gate.weight"),
    ("group32", "switch_mlp.gate_proj.scales has shape [8,128,8]"),
])
def test_checkpoint_errors(torch_dev, tmp_path, case, needle):
    torch, dev = torch_dev
    pkg = load_pkg()
    say(f"case: checkpoint error {case}")
    arrays = orc.Layer(H, E, K, I, seed=1).arrays()
    drop, replace, model_layer = (), {}, 0
    if case == "quant_router":
        replace[moe_name(0, "router_w").replace(".weight", ".scales")] = \
            torch.zeros((E, H // 64), dtype=torch.bfloat16)
    elif case == "dense_expert":
        drop = ("gate_s",)
    elif case == "wrong_E":
        replace[moe_name(0, "router_w")] = torch.zeros((4, H), dtype=torch.bfloat16)
    elif case == "scales_f16":
        replace[moe_name(0, "up_s")] = torch.zeros((E, I, H // 64), dtype=torch.float16)
    elif case == "missing_layer":
        model_layer = 9
    elif case == "group32":
        replace[moe_name(0, "gate_s")] = torch.zeros((E, I, H // 32), dtype=torch.bfloat16)
    write_moe_layer(str(tmp_path), arrays, H, E, I, layer=0, drop=drop, replace=replace)
    with pkg.Checkpoint(str(tmp_path)) as ck, pkg.MoeContext(H, E, K, I, max_tokens=4) as ctx:
        with pytest.raises(pkg.QmoeError) as ei:
            ctx.upload_layer_st(0, ck, model_layer)
        assert needle in str(ei.value), str(ei.value)
