"""Writes the golden fixtures under tests/golden/ from the CPU oracle.

  tiny_layer.npz    the 4-token tiny layer (H=256, E=8, k=2, I=128), f32 x:
                    inputs, router logits, routing, outputs, and SHA-256 of
                    every weight tensor (pins the seeded generator)
  decode_token.npz  one bf16 token through the decode-shape layer (H=2048,
                    E=512, k=10, I=512): routing and output

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


if __name__ == "__main__":
    tiny()
    decode()
    print("wrote", sorted(f for f in os.listdir(OUT) if f.endswith(".npz")))
