"""The checkpoint index (qmoe_st.c, which parses headers of untrusted
files) and the expert slot cache (qmoe_cache.c) built with
AddressSanitizer and UndefinedBehaviorSanitizer into a host-only driver
(tests/c/st_fuzz.c), then run over

* the corpus tests/golden/st_corpus/ (tests/golden/make_st_corpus.py): the
  malformed cases of the reference's own safetensors test
  (c/tests/test_safetensors.c:110-176) and parser edge cases -- bad_* files
  must be refused with a message, ok_* and edge_* files must index, and
  every indexed tensor must read back;
* 600 mutants of valid files (seeded byte flips, truncations, header
  lengths and JSON splices), which must be refused or index cleanly;
* random sequences of cache operations over several shapes and the three
  policies (a pinned entry is never evicted; results stay in range).

Any sanitizer report fails the test.  CPU only.
"""
import os
import random
import shutil
import struct
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "qwen3.8-flash-next_amd", "csrc")
CORPUS = os.path.join(ROOT, "tests", "golden", "st_corpus")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    gcc = shutil.which("gcc")
    if not gcc:
        pytest.skip("gcc is not available")
    out = str(tmp_path_factory.mktemp("san") / "st_fuzz")
    cmd = [gcc, "-std=c11", "-O1", "-g", *SAN, "-Wall", "-Wextra", "-Wno-unused-parameter",
           "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", "-I" + os.path.join(ROOT, "include"), "-I" + CSRC,
           os.path.join(ROOT, "tests", "c", "st_fuzz.c"), os.path.join(CSRC, "qmoe_st.c"),
           os.path.join(CSRC, "qmoe_cache.c"), "-o", out, "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode and ("asan" in r.stderr.lower() or "sanitizer" in r.stderr.lower()):
        pytest.skip("the sanitizer runtime is not available: " + r.stderr[-300:])
    assert r.returncode == 0, r.stderr
    return out


def run(driver, args):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([driver, *args], capture_output=True, text=True, errors="replace", env=env, timeout=300)
    assert "Sanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-4000:]
    assert r.returncode == 0, (r.returncode, r.stderr[-2000:])
    return r.stdout.splitlines()


def one_per_dir(root, files):
    """each (name, bytes) in its own directory; returns the directories"""
    dirs = []
    for name, data in files:
        d = os.path.join(root, name)
        os.makedirs(d, exist_ok=True)
        with open(os.path.join(d, name + ".safetensors"), "wb") as f:
            f.write(data)
        dirs.append(d)
    return dirs


def corpus():
    out = []
    for f in sorted(os.listdir(CORPUS)):
        if f.endswith(".safetensors"):
            with open(os.path.join(CORPUS, f), "rb") as fh:
                out.append((f[:-len(".safetensors")], fh.read()))
    return out


def test_corpus(driver, tmp_path):
    files = corpus()
    assert len(files) >= 30
    dirs = one_per_dir(str(tmp_path), files)
    lines = run(driver, dirs)
    assert len(lines) == len(files)
    for (name, _), line in zip(files, lines):
        if name.startswith("bad_"):
            assert line.startswith("refused ") and len(line) > 10, (name, line)
        else:
            assert line.startswith("ok "), (name, line)


def mutants(files, count, seed):
    rng = random.Random(seed)
    valid = [d for n, d in files if n.startswith("ok_")]
    tokens = [b"{", b"}", b"[", b"]", b",", b":", b'"', b"\\", b"-", b"1e999", b"18446744073709551617",
              b'"dtype"', b'"shape"', b'"data_offsets"', b"null", b"true", b"\x00", b"\xff"]
    out = []
    for i in range(count):
        data = bytearray(rng.choice(valid))
        hlen = struct.unpack("<Q", bytes(data[:8]))[0]
        kind = rng.randrange(5)
        if kind == 0:  # byte flips in the header
            for _ in range(rng.randint(1, 6)):
                j = rng.randrange(8, 8 + hlen)
                data[j] = rng.randrange(256)
        elif kind == 1:  # truncation
            data = data[:rng.randrange(len(data))]
        elif kind == 2:  # another header length
            data[:8] = struct.pack("<Q", rng.choice([0, 1, hlen - 1, hlen + 1, len(data), 1 << 40,
                                                     rng.randrange(1 << 16)]))
        elif kind == 3:  # a JSON token spliced into the header, the length kept consistent
            j = rng.randrange(8, 8 + hlen)
            t = rng.choice(tokens)
            data[j:j] = t
            data[:8] = struct.pack("<Q", hlen + len(t))
        else:  # a header byte deleted
            j = rng.randrange(8, 8 + hlen)
            del data[j]
            data[:8] = struct.pack("<Q", hlen - 1)
        out.append((f"m{i:04d}", bytes(data)))
    return out


def test_mutants(driver, tmp_path):
    files = mutants(corpus(), 600, seed=0)
    dirs = one_per_dir(str(tmp_path), files)
    lines = run(driver, dirs)
    assert len(lines) == len(files)
    assert all(l.startswith("ok ") or l.startswith("refused ") for l in lines)
    refused = sum(l.startswith("refused ") for l in lines)
    assert 100 < refused < len(lines), refused  # both outcomes are exercised


@pytest.mark.parametrize("seed", [1, 2])
def test_cache_operations(driver, seed):
    assert run(driver, ["--cache", str(seed), "20000"]) == ["cache ok"]
