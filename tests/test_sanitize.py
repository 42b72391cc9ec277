"""The host code under AddressSanitizer and UndefinedBehaviorSanitizer, on
the CPU: the .safetensors reader (weights_hip.cpp) on malformed files, the
C-ABI status -> exception shim and the host API's argument checks
(tensor_hip.cpp, sd_hip.hpp, against the no-GPU stub backend_stub.cpp), and
the CPU oracle (sd_oracle.c). The sanitized build is g++/gcc only (no device
code): tests/cpp/sanitize_host.cpp drives it. Any sanitizer finding aborts
the driver, which fails the test; so does a malformed file that is not
rejected with the loader's own error, or an exception of the wrong type.

The reference's failure handling is exceptions on bad shapes, devices and
files (tensor.cpp:97-99, :733, :891; safetensors.cpp:81-200; the stub
backend_cuda_stub.cpp:14-56); these tests hold the host side of this
library to the same, with no memory errors or undefined behaviour on any
input.
"""
import json
import os
import random
import shutil
import struct
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "stablediffusion-cpp_amd")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:exitcode=99",
           UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1:exitcode=98")


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    if not (shutil.which("g++") and shutil.which("gcc")):
        pytest.skip("no host compiler")
    out = tmp_path_factory.mktemp("sanitize")
    inc = ["-I", os.path.join(ROOT, "include"), "-I", os.path.join(PKG, "host"), "-I", os.path.join(ROOT, "oracle")]
    objs = []

    def cc(tool, src, std):
        obj = str(out / (os.path.basename(src) + ".o"))
        subprocess.run([tool, std, *SAN, *inc, "-c", src, "-o", obj], check=True, capture_output=True, text=True)
        objs.append(obj)

    cc("gcc", os.path.join(ROOT, "oracle", "sd_oracle.c"), "-std=c11")
    for src in (os.path.join(PKG, "host", "tensor_hip.cpp"), os.path.join(PKG, "host", "weights_hip.cpp"),
                os.path.join(PKG, "csrc", "backend_stub.cpp"), os.path.join(ROOT, "tests", "cpp", "sanitize_host.cpp")):
        cc("g++", src, "-std=c++17")
    exe = str(out / "sanitize_host")
    subprocess.run(["g++", *SAN, *objs, "-o", exe, "-lpthread", "-lm"], check=True, capture_output=True, text=True)
    return exe


def run(driver, *args):
    p = subprocess.run([driver, *args], capture_output=True, text=True, env=ENV, timeout=300)
    assert "Sanitizer" not in p.stderr and "runtime error" not in p.stderr, p.stderr[-4000:]
    assert p.returncode == 0, (p.returncode, p.stdout[-2000:], p.stderr[-2000:])
    return p.stdout.splitlines()


def safetensors(header, data=b"", hlen=None):
    h = header if isinstance(header, bytes) else json.dumps(header).encode()
    return struct.pack("<Q", len(h) if hlen is None else hlen) + h + data


VALID_HEADER = {
    "a": {"dtype": "F32", "shape": [2, 3], "data_offsets": [0, 24]},
    "b": {"dtype": "BF16", "shape": [4], "data_offsets": [24, 32]},
    "c": {"dtype": "F16", "shape": [2, 2], "data_offsets": [32, 40]},
    "i": {"dtype": "I64", "shape": [1], "data_offsets": [40, 48]},
    "__metadata__": {"format": "pt", "note": "caf\\u00e9 \\ud83d\\ude00"},
}
VALID_DATA = bytes(range(48))


def malformed():
    good = json.dumps(VALID_HEADER).encode()
    cases = {
        "empty": b"",
        "short": b"\x01\x02",
        "length past end": safetensors(good, VALID_DATA, hlen=len(good) + 10**6),
        "length 2^63": safetensors(good, VALID_DATA, hlen=1 << 63),
        "not an object": safetensors(b"[1, 2]"),
        "empty header": safetensors(b""),
        "trailing characters": safetensors(good + b"}", VALID_DATA),
        "deep arrays": safetensors(b"[" * 200000),
        "deep objects": safetensors(b'{"a":' * 50000),
        "unterminated string": safetensors(b'{"a'),
        "bad escape": safetensors(b'{"a\\q": 1}'),
        "short unicode escape": safetensors(b'{"\\u12'),
        "bad surrogate": safetensors(b'{"\\ud83d\\u0041": 1}'),
        "nul in number": safetensors(b'{"a": {"dtype": "F32", "shape": [1\x00], "data_offsets": [0, 4]}}', b"\0" * 4),
        "number overflow": safetensors(b'{"a": {"dtype": "F32", "shape": [1e999], "data_offsets": [0, 4]}}', b"\0" * 4),
        "bad number": safetensors(b'{"a": {"dtype": "F32", "shape": [1-2], "data_offsets": [0, 4]}}', b"\0" * 4),
        "negative dim": safetensors({"a": {"dtype": "F32", "shape": [-1, 4], "data_offsets": [0, 16]}}, b"\0" * 16),
        "fractional dim": safetensors({"a": {"dtype": "F32", "shape": [1.5], "data_offsets": [0, 4]}}, b"\0" * 4),
        "count overflow": safetensors({"a": {"dtype": "F32", "shape": [2**62, 8], "data_offsets": [0, 0]}}),
        "size mismatch": safetensors({"a": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}, b"\0" * 8),
        "offsets reversed": safetensors({"a": {"dtype": "F32", "shape": [1], "data_offsets": [8, 4]}}, b"\0" * 8),
        "offsets past data": safetensors({"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}, b"\0" * 8),
        "missing offsets": safetensors({"a": {"dtype": "F32", "shape": [1]}}, b"\0" * 4),
        "string shape": safetensors({"a": {"dtype": "F32", "shape": ["1"], "data_offsets": [0, 4]}}, b"\0" * 4),
    }
    for cut in range(0, len(good) + 8, 7):
        cases[f"truncated at {cut}"] = safetensors(good, VALID_DATA)[:cut]
    rnd = random.Random(1234)
    base = safetensors(good, VALID_DATA)
    for i in range(300):
        b = bytearray(base)
        for _ in range(rnd.randint(1, 4)):
            b[rnd.randrange(8, 8 + len(good))] = rnd.randrange(256)
        cases[f"flipped {i}"] = bytes(b)
    return cases


def test_weights_reader_on_malformed_files(driver, tmp_path):
    ok = tmp_path / "valid.safetensors"
    ok.write_bytes(safetensors(VALID_HEADER, VALID_DATA))
    cases = malformed()
    paths = [str(ok)]
    for i, blob in enumerate(cases.values()):
        p = tmp_path / f"case{i}.safetensors"
        p.write_bytes(blob)
        paths.append(str(p))
    lines = run(driver, "weights", *paths)
    assert lines[-1] == "ok"
    outcome = lines[:-1]
    assert len(outcome) == len(paths)
    # the valid file parses completely and stops only at the upload (no device on the stub)
    assert outcome[0].startswith("device"), outcome[0]
    names = ["valid"] + list(cases)
    expected_rejected = [n for n in cases if not n.startswith("flipped")]
    for name, line in zip(names[1:], outcome[1:]):
        if name in expected_rejected:
            assert line.startswith("rejected"), f"{name}: {line}"
        else:
            assert line.startswith(("rejected", "device")), f"{name}: {line}"
    reasons = {n: l for n, l in zip(names, outcome)}
    assert "nesting too deep" in reasons["deep arrays"] and "nesting too deep" in reasons["deep objects"]
    assert "bad surrogate pair" in reasons["bad surrogate"]


def test_shim_and_host_argument_checks(driver):
    assert run(driver, "shim")[-1] == "ok"


def test_oracle_routines(driver):
    assert run(driver, "oracle")[-1] == "ok"
