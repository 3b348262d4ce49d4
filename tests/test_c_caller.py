"""The ABI from a C program: tests/c/abi_caller.c includes include/qmoe.h
and links libqmoe.so (built by the library's Makefile), as the reference C
port would call it in place of moe_forward (c/src/model.c:1712)."""
import os
import struct
import subprocess

import numpy as np
import pytest

from conftest import load_oracle

HERE = os.path.dirname(os.path.abspath(__file__))
CALLER = os.path.join(HERE, "c", "abi_caller")
GOLDEN = os.path.join(HERE, "golden")

ORDER = ["router_w", "gate_q", "gate_s", "gate_b", "up_q", "up_s", "up_b", "down_q", "down_s",
         "down_b", "sh_gate_q", "sh_gate_s", "sh_gate_b", "sh_up_q", "sh_up_s", "sh_up_b",
         "sh_down_q", "sh_down_s", "sh_down_b", "sh_gate_w"]


def write_fixture(path, arrays, x, out, idx, H, E, k, I):
    with open(path, "wb") as f:
        f.write(b"QMOEFIX1" + struct.pack("<5i", H, E, k, I, x.shape[0]))
        for a in [arrays[nm] for nm in ORDER] + [x, out, idx]:
            b = np.ascontiguousarray(a).tobytes()
            f.write(struct.pack("<q", len(b)) + b)


def test_c_caller_built_and_linked():
    assert os.path.isfile(CALLER), "tests/c/abi_caller is built by the library's Makefile"
    v = subprocess.run([CALLER, "--version"], capture_output=True, text=True, timeout=60)
    assert v.returncode == 0 and v.stdout.startswith("qmoe"), (v.stdout, v.stderr)
    deps = subprocess.run(["ldd", CALLER], capture_output=True, text=True, timeout=60).stdout
    assert "libqmoe.so" in deps and "not found" not in deps.split("libqmoe.so")[1].split("\n")[0]


@pytest.mark.gpu
def test_c_caller_tiny_layer(gpu, tmp_path):
    orc = load_oracle()
    g = np.load(os.path.join(GOLDEN, "tiny_layer.npz"))
    L = orc.Layer(256, 8, 2, 128, seed=0)
    fx = str(tmp_path / "tiny.bin")
    write_fixture(fx, L.arrays(), g["x"].astype(np.float32), g["out"].astype(np.float32),
                  g["idx"].astype(np.int32), 256, 8, 2, 128)
    print("case: C caller, tiny layer (H=256 E=8 k=2 I=128, n=4)", flush=True)
    r = subprocess.run([CALLER, fx], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0 and "PASSED" in r.stdout
