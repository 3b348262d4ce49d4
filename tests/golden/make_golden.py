"""Writes the golden fixtures under tests/golden/ from the CPU oracle.

  tiny_layer.npz    the 4-token tiny layer (H=256, E=8, k=2, I=128), f32 x:
                    inputs, router logits, routing, outputs, and SHA-256 of
                    every weight tensor (pins the seeded generator)
  decode_token.npz  one bf16 token through the decode-shape layer (H=2048,
                    E=512, k=10, I=512): routing and output
  hyper_tiny.npz    the tiny layer inside its MLP hyper connection (hc 4, rank
                    128, a non-unit bf16-exact hc_norm): 4 hyper states in,
                    mixed, inject, routing, the MoE output and the updated
                    hyper states out, and SHA-256 of every hc tensor

Run from the repository root:  python tests/golden/make_golden.py
The oracle itself is pinned by tests/test_oracle.py (reference known-answer
vectors, the reference's util.h, float64 and transformers cross-checks).
"""
import hashlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import oracle as orc  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def tiny():
    L = orc.Layer(256, 8, 2, 128, seed=0)
    x = orc.gen_x(4, 256, 0, bf16=False)
    r = L.forward(x, False)
    rt = L.route(x, False)
    hashes = {k: sha(v) for k, v in L.t.items() if v is not None}
    np.savez_compressed(os.path.join(OUT, "tiny_layer.npz"), x=x, logits=rt["logits"],
                        gate_logit=rt["gate_logit"], idx=r["idx"], w=r["w"],
                        shared_gate=r["shared_gate"], out=r["out"],
                        weight_names=np.array(sorted(hashes)),
                        weight_sha256=np.array([hashes[k] for k in sorted(hashes)]))


def decode():
    H, E, k, I = 2048, 512, 10, 512
    x = orc.gen_x(1, H, 0, bf16=True)
    Lr = orc.Layer(H, E, k, I, seed=0, only_experts=[])
    rt = Lr.route(x, True)
    L = orc.Layer(H, E, k, I, seed=0, only_experts=rt["idx"].reshape(-1))
    r = L.forward(x, True)
    assert np.array_equal(r["idx"], rt["idx"])
    np.savez_compressed(os.path.join(OUT, "decode_token.npz"), x=x, logits=rt["logits"],
                        gate_logit=rt["gate_logit"], idx=r["idx"], w=r["w"],
                        shared_gate=r["shared_gate"], out=r["out"])


def hyper_tiny_case():
    """the fixture's layer, hyper-connection weights and input (also used by
    the tests to rebuild the same arrays)"""
    L = orc.Layer(256, 8, 2, 128, seed=0)
    hp = orc.Hyper(4, 256, 128, seed=0, norm_std=0.2)
    a = hp.arrays()
    a["hc_norm"] = orc.bf16_to_f32(orc.f32_to_bf16(a["hc_norm"]))
    hp = orc.Hyper.from_arrays(4, 256, 128, a)
    hyper = orc.gen_hyper(4, 4, 256, seed=0)
    return L, hp, hyper


def hyper_tiny():
    L, hp, hyper = hyper_tiny_case()
    r = hp.layer_forward(L, hyper)
    rt = L.route(r["mixed"], False)
    hashes = {k: sha(v) for k, v in hp.t.items()}
    np.savez_compressed(os.path.join(OUT, "hyper_tiny.npz"), hyper_in=hyper, mixed=r["mixed"],
                        inject=r["inject"], idx=rt["idx"], moe_out=r["moe_out"],
                        hyper_out=r["hyper"], hc_norm=hp.t["hc_norm"],
                        weight_names=np.array(sorted(hashes)),
                        weight_sha256=np.array([hashes[k] for k in sorted(hashes)]))


if __name__ == "__main__":
    tiny()
    decode()
    hyper_tiny()
    print("wrote", sorted(f for f in os.listdir(OUT) if f.endswith(".npz")))
