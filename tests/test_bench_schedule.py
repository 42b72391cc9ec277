"""CPU test: bench.py's model of run_gn's schedule choice (gn_dispatches,
used to find each GroupNorm workload's kernels in a rocprofv3 trace) agrees
with the library's rule, whose thresholds it reads from the source: single
kernel up to kSmallResidentMin floats per segment, the resident schedule
from 64 MB of x, else the split schedule with split_chunk's chunk (the
largest of 8192, 4096, 2048 floats giving 768 workgroups per pass)."""
import importlib.util
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GN_SRC = os.path.join(ROOT, "stablediffusion-cpp_amd", "csrc", "k_groupnorm.hip")


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_thresholds_match_the_library_source():
    src = open(GN_SRC).read()
    assert re.search(r"constexpr int64_t kSmallResidentMin = 24576;", src)
    assert re.search(r"nseg \* L \* 4 >= \(int64_t\(64\) << 20\)", src)
    assert re.search(r"if \(nseg \* \(\(L \+ c - 1\) / c\) >= 768\) return c;", src)
    assert "{int64_t(8192), int64_t(4096)}" in src and "return 2048;" in src


def test_config_shapes():
    b = _bench()
    assert b.gn_dispatches((2, 1280, 8, 8)) == [("k_gn_single", 64 * 256)]           # 4d
    assert b.gn_dispatches((2, 320, 64, 64)) == [("k_gn_partial", 81920), ("k_gn_apply", 81920)]  # 4c: 2048
    assert b.gn_dispatches((1, 512, 128, 128)) == [("k_gn_partial", 262144), ("k_gn_apply", 262144)]  # 4a: 8192
    assert b.gn_dispatches((1, 128, 1024, 1024))[0][0] == "k_gn_resident_pipe<"   # 4b
    assert b.gn_dispatches((2, 640, 64, 64)) == [("k_gn_partial", 64 * 20 * 64), ("k_gn_apply", 64 * 20 * 64)]


def test_split_chunk_rule():
    b = _bench()
    assert b.gn_split_chunk(32, 262144) == 8192      # 1024 workgroups
    assert b.gn_split_chunk(32, 230400) == 8192      # 928 workgroups
    assert b.gn_split_chunk(64, 81920) == 4096       # 640 at 8192, 1280 at 4096
    assert b.gn_split_chunk(64, 40960) == 2048
    assert b.gn_split_chunk(1, 100) == 2048
