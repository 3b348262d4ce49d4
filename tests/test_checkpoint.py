"""Checkpoint index (qmoe_st_*, host only, no GPU): files written by the
safetensors library are indexed with the names, dtypes, shapes and bytes the
library wrote; the reference's reader rules hold (c/src/safetensors.c:57-324):
"language_model." dropped from stored names and tried on lookup, and
malformed files (truncated header or JSON, unknown dtype, data range not
matching the shape or past the file, overlapping ranges, duplicate names)
are refused with a message."""
import json
import os

import numpy as np
import pytest

from ckpt_util import moe_name, write_moe_layer, write_raw
from conftest import load_oracle, load_pkg

pytest.importorskip("safetensors")
torch = pytest.importorskip("torch")

H, E, K, I = 256, 8, 2, 128


@pytest.fixture(scope="module")
def layer_arrays():
    orc = load_oracle()
    return orc.Layer(H, E, K, I, seed=0).arrays()


def test_index_matches_the_written_files(tmp_path, layer_arrays):
    pkg = load_pkg()
    names = write_moe_layer(str(tmp_path), layer_arrays, H, E, I, layer=3, shards=3,
                            prefixed_shard=1)
    with pkg.Checkpoint(str(tmp_path)) as ck:
        assert ck.names() == sorted(names)  # prefix dropped, sorted
        info = ck.info(moe_name(3, "gate_q"))
        assert info["dtype"] == "U32" and info["shape"] == (E, I, H // 8)
        assert info["nbytes"] == E * I * H // 8 * 4
        info = ck.info(moe_name(3, "down_s"))
        assert info["dtype"] == "BF16" and info["shape"] == (E, H, I // 64)
        assert ck.info(moe_name(3, "sh_gate_w"))["shape"] == (1, H)
        for key in ("router_w", "gate_q", "down_b", "sh_down_q", "sh_gate_w"):
            got = ck.read(moe_name(3, key))
            assert got == np.ascontiguousarray(layer_arrays[key]).tobytes(), key
        assert ck.info("model.layers.3.mlp.nothing.weight") is None
        assert ck.info(moe_name(2, "gate_q")) is None


def test_files_are_indexed_in_name_order(tmp_path, layer_arrays):
    pkg = load_pkg()
    write_moe_layer(str(tmp_path), layer_arrays, H, E, I, layer=0, shards=2, prefixed_shard=-1)
    open(os.path.join(str(tmp_path), "README.md"), "w").write("not a tensor file")
    with pkg.Checkpoint(str(tmp_path)) as ck:
        files = {ck.info(n)["file"] for n in ck.names()}
        assert files == {0, 1}
        # model-00001-of-00002 sorts first and holds the first name round-robin
        assert ck.info(ck.names()[0])["file"] == 0


def test_prefixed_lookup_fallback(tmp_path):
    """a name stored with the prefix twice keeps one after indexing; the
    lookup of model.X then finds language_model.model.X (safetensors.c:316-324)"""
    pkg = load_pkg()
    data = np.arange(6, dtype=np.float32).tobytes()
    hdr = {"language_model.language_model.model.norm.weight":
           {"dtype": "F32", "shape": [6], "data_offsets": [0, 24]}}
    write_raw(os.path.join(str(tmp_path), "a.safetensors"), hdr, data)
    with pkg.Checkpoint(str(tmp_path)) as ck:
        assert ck.names() == ["language_model.model.norm.weight"]
        assert ck.read("model.norm.weight") == data
        assert ck.info("lm_head.weight") is None


def test_header_json_forms(tmp_path):
    """escapes, unicode, nested metadata, whitespace and padding"""
    pkg = load_pkg()
    a = np.array([1, 2, 3], dtype=np.int32).tobytes()
    b = np.array([0x3F80, 0x4000], dtype=np.uint16).tobytes()
    js = ('{ "__metadata__" : {"format":"mlx", "nested": {"list": [1, 2.5e3, -4, true, null]}},\n'
          ' "w\\u00e9ight\\\\x\\"q" : {"dtype":"I32","shape":[3],"data_offsets":[0,12]},\t'
          ' "\\ud83d\\ude00.b" : {"shape":[2],"dtype":"BF16","data_offsets":[12,16]} }')
    write_raw(os.path.join(str(tmp_path), "x.safetensors"), js, a + b, pad=7)
    with pkg.Checkpoint(str(tmp_path)) as ck:
        names = ck.names()
        assert names == sorted(['wéight\\x"q', "\U0001F600.b"], key=lambda s: s.encode())
        assert ck.read('wéight\\x"q') == a
        assert ck.info("\U0001F600.b")["dtype"] == "BF16"
        assert ck.read("\U0001F600.b") == b


def test_empty_tensor_and_scalar(tmp_path):
    pkg = load_pkg()
    hdr = {"e": {"dtype": "F32", "shape": [0, 4], "data_offsets": [0, 0]},
           "s": {"dtype": "F64", "shape": [], "data_offsets": [0, 8]}}
    write_raw(os.path.join(str(tmp_path), "x.safetensors"), hdr, np.float64(2.5).tobytes())
    with pkg.Checkpoint(str(tmp_path)) as ck:
        assert ck.info("e")["nbytes"] == 0 and ck.info("e")["shape"] == (0, 4)
        assert ck.info("s")["shape"] == () and ck.read("s") == np.float64(2.5).tobytes()


def _open_error(path):
    pkg = load_pkg()
    with pytest.raises(pkg.QmoeError) as ei:
        pkg.Checkpoint(path)
    return str(ei.value)


@pytest.mark.parametrize("case,needle", [
    ("short", "shorter than the 8-byte header length field"),
    ("hlen_past_end", "header length runs past the end of the file"),
    ("bad_json", "header is not a JSON object"),
    ("trailing", "trailing bytes after the header object"),
    ("not_object", "top level is not an object"),
    ("bad_dtype", "element type F8_E4M3 is not supported"),
    ("no_offsets", "entry lacks dtype, shape or data_offsets"),
    ("float_offset", "data_offsets must be two ordered non-negative integers"),
    ("range_vs_shape", "byte range disagrees with the shape"),
    ("past_end", "byte range disagrees with the shape or leaves the file"),
    ("neg_dim", "shape entries must be non-negative integers"),
    ("overlap", "data overlaps another tensor of the file"),
    ("dup_prefix", "a: tensor name given twice"),
])
def test_malformed_files_are_refused(tmp_path, case, needle):
    p = os.path.join(str(tmp_path), "m.safetensors")
    d16 = bytes(16)
    ok = {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}
    if case == "short":
        open(p, "wb").write(b"\x01\x02\x03")
    elif case == "hlen_past_end":
        write_raw(p, {"a": ok}, d16, header_len=10 ** 6)
    elif case == "bad_json":
        write_raw(p, '{"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]', d16)
    elif case == "trailing":
        write_raw(p, json.dumps({"a": ok}) + " x", d16)
    elif case == "not_object":
        write_raw(p, "[1, 2]", d16)
    elif case == "bad_dtype":
        write_raw(p, {"a": {"dtype": "F8_E4M3", "shape": [16], "data_offsets": [0, 16]}}, d16)
    elif case == "no_offsets":
        write_raw(p, {"a": {"dtype": "F32", "shape": [4]}}, d16)
    elif case == "float_offset":
        write_raw(p, {"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16.0]}}, d16)
    elif case == "range_vs_shape":
        write_raw(p, {"a": {"dtype": "F32", "shape": [3], "data_offsets": [0, 16]}}, d16)
    elif case == "past_end":
        write_raw(p, {"a": {"dtype": "F32", "shape": [8], "data_offsets": [0, 32]}}, d16)
    elif case == "neg_dim":
        write_raw(p, {"a": {"dtype": "F32", "shape": [-4], "data_offsets": [0, 16]}}, d16)
    elif case == "overlap":
        write_raw(p, {"a": ok, "b": {"dtype": "F32", "shape": [2], "data_offsets": [8, 16]}}, d16)
    elif case == "dup_prefix":
        write_raw(p, {"a": ok, "language_model.a": {"dtype": "F32", "shape": [0],
                                                     "data_offsets": [16, 16]}}, d16)
    msg = _open_error(str(tmp_path))
    assert needle in msg, msg


def test_duplicate_across_files_and_empty_dir(tmp_path):
    d16 = bytes(16)
    ok = {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}
    assert "no .safetensors file in the directory" in _open_error(str(tmp_path))
    assert "checkpoint directory cannot be listed" in _open_error(os.path.join(str(tmp_path), "missing"))
    write_raw(os.path.join(str(tmp_path), "a.safetensors"), {"model.x": ok}, d16)
    write_raw(os.path.join(str(tmp_path), "b.safetensors"), {"language_model.model.x": ok}, d16)
    assert "model.x: tensor name given twice" in _open_error(str(tmp_path))


def test_read_errors(tmp_path):
    pkg = load_pkg()
    write_raw(os.path.join(str(tmp_path), "a.safetensors"),
              {"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}, bytes(16))
    with pkg.Checkpoint(str(tmp_path)) as ck:
        with pytest.raises(pkg.QmoeError, match="missing tensor b"):
            ck.read("b")
        import ctypes
        buf = ctypes.create_string_buffer(8)
        err = pkg.QmoeErr()
        assert pkg.lib().qmoe_st_read(ck.handle, b"a", buf, 8, ctypes.byref(err)) == -1
        assert b"too small" in err.msg
