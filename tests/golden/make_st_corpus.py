"""Writes tests/golden/st_corpus/: small safetensors files, valid and
malformed, for the sanitizer run of the checkpoint index
(tests/test_sanitize.py).  The malformed cases follow the reference's own
(c/tests/test_safetensors.c:110-176: truncated header length, bad dtype,
overlapping ranges, offsets beyond the file, mismatched size, duplicate
names after the language_model. prefix, invalid JSON) and add parser edge
cases (deep nesting, bad escapes, huge or negative numbers, shape products
that overflow, more than 8 dims, trailing bytes, empty header).  ok_* and
edge_* files index; bad_* files are refused.  Run from
the repository root: python tests/golden/make_st_corpus.py"""
import json
import os
import struct

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "st_corpus")


def st_bytes(header, data=b"", hlen=None):
    h = header if isinstance(header, bytes) else header.encode()
    n = len(h) if hlen is None else hlen
    return struct.pack("<Q", n) + h + data


def obj(**tensors):
    return json.dumps(tensors)


F32x4 = {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}
DATA16 = bytes(range(16))
CASES = {
    # valid files
    "ok_one_f32": st_bytes(obj(t=F32x4), DATA16),
    "ok_two_and_meta": st_bytes(json.dumps({"__metadata__": {"format": "mlx"},
                                            "a": {"dtype": "BF16", "shape": [2, 2], "data_offsets": [0, 8]},
                                            "language_model.b": {"dtype": "U32", "shape": [2],
                                                                 "data_offsets": [8, 16]}}), DATA16),
    "ok_scalar_and_empty": st_bytes(json.dumps({"s": {"dtype": "F32", "shape": [], "data_offsets": [0, 4]},
                                                "e": {"dtype": "F32", "shape": [0, 3], "data_offsets": [4, 4]}}),
                                    DATA16[:4]),
    "ok_escapes_in_name": st_bytes(json.dumps({"a\\u00e9\\n\"b": F32x4}).replace("\\\\", "\\"), DATA16),
    # the reference's malformed cases
    "bad_header_len_past_file": struct.pack("<Q", 10000),
    "bad_dtype_size": st_bytes('{"t":{"dtype":"F16","shape":[4],"data_offsets":[0,16]}}', DATA16),
    "bad_overlap": st_bytes('{"a":{"dtype":"F32","shape":[4],"data_offsets":[0,16]},'
                            '"b":{"dtype":"F32","shape":[4],"data_offsets":[8,24]}}', DATA16 * 2),
    "bad_offsets_past_file": st_bytes('{"t":{"dtype":"F32","shape":[4],"data_offsets":[0,100]}}', DATA16),
    "bad_size_mismatch": st_bytes('{"t":{"dtype":"F32","shape":[4],"data_offsets":[0,8]}}', DATA16),
    "bad_duplicate_after_prefix": st_bytes('{"t":{"dtype":"F32","shape":[4],"data_offsets":[0,16]},'
                                           '"language_model.t":{"dtype":"F32","shape":[4],'
                                           '"data_offsets":[16,32]}}', DATA16 * 2),
    "bad_json": st_bytes("{not json", DATA16),
    # parser and arithmetic edge cases
    "bad_empty_file": b"",
    "bad_short_length": b"\x01\x02\x03",
    "bad_header_len_zero": st_bytes("", b""),
    "bad_header_len_huge": struct.pack("<Q", (1 << 64) - 1) + b"{}",
    "bad_not_object": st_bytes("[1,2,3]"),
    "bad_deep_nesting": st_bytes("[" * 5000 + "]" * 5000),
    "bad_deep_object": st_bytes('{"a":' * 3000 + "1" + "}" * 3000),
    "bad_unterminated_string": st_bytes('{"t":{"dtype":"F32'),
    "bad_escape": st_bytes('{"t\\u12":{"dtype":"F32","shape":[4],"data_offsets":[0,16]}}', DATA16),
    "bad_escape_end": st_bytes('{"t\\', DATA16),
    "bad_control_char": st_bytes('{"t\x01":{"dtype":"F32","shape":[4],"data_offsets":[0,16]}}', DATA16),
    "bad_unknown_dtype": st_bytes('{"t":{"dtype":"Q4","shape":[4],"data_offsets":[0,16]}}', DATA16),
    "bad_missing_dtype": st_bytes('{"t":{"shape":[4],"data_offsets":[0,16]}}', DATA16),
    "bad_shape_not_array": st_bytes('{"t":{"dtype":"F32","shape":4,"data_offsets":[0,16]}}', DATA16),
    "bad_shape_negative": st_bytes('{"t":{"dtype":"F32","shape":[-4],"data_offsets":[0,16]}}', DATA16),
    "bad_shape_fraction": st_bytes('{"t":{"dtype":"F32","shape":[4.5],"data_offsets":[0,16]}}', DATA16),
    "bad_shape_overflow": st_bytes('{"t":{"dtype":"F32","shape":[4294967296,4294967296,16],'
                                   '"data_offsets":[0,16]}}', DATA16),
    "bad_shape_huge_number": st_bytes('{"t":{"dtype":"F32","shape":[1e400],"data_offsets":[0,16]}}', DATA16),
    "bad_nine_dims": st_bytes('{"t":{"dtype":"U8","shape":[1,1,1,1,1,1,1,1,16],"data_offsets":[0,16]}}',
                              DATA16),
    "bad_offsets_reversed": st_bytes('{"t":{"dtype":"F32","shape":[4],"data_offsets":[16,0]}}', DATA16),
    "bad_offsets_three": st_bytes('{"t":{"dtype":"F32","shape":[4],"data_offsets":[0,8,16]}}', DATA16),
    "bad_offsets_huge": st_bytes('{"t":{"dtype":"F32","shape":[4],'
                                 '"data_offsets":[18446744073709551600,18446744073709551616]}}', DATA16),
    "bad_trailing_garbage": st_bytes('{"t":{"dtype":"F32","shape":[4],"data_offsets":[0,16]}} xyz', DATA16),
    "edge_metadata_not_object": st_bytes('{"__metadata__":[1],"t":{"dtype":"F32","shape":[4],'
                                        '"data_offsets":[0,16]}}', DATA16),
    "bad_tensor_not_object": st_bytes('{"t":"F32"}', DATA16),
    "edge_long_name": st_bytes(json.dumps({"n" * 20000: F32x4}), DATA16),
    "bad_many_tensors_overlap": st_bytes(json.dumps({f"t{i}": {"dtype": "U8", "shape": [16],
                                                               "data_offsets": [i, i + 16]}
                                                     for i in range(300)}), DATA16 * 20),
}


def main():
    os.makedirs(OUT, exist_ok=True)
    for f in os.listdir(OUT):
        if f.endswith(".safetensors"):
            os.remove(os.path.join(OUT, f))
    for name, data in CASES.items():
        with open(os.path.join(OUT, name + ".safetensors"), "wb") as fh:
            fh.write(data)
    print(f"{len(CASES)} files in {OUT}")


if __name__ == "__main__":
    main()
