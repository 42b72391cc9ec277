"""CPU test: bench.py's model of run_gn's schedule choice (gn_dispatches,
used to find each GroupNorm workload's kernels in a rocprofv3 trace) agrees
with the library's rule, whose thresholds it reads from the source: single
kernel up to kSmallResidentMin floats per segment, the pipelined schedule
for segments of whole 4096-float chunks within one channel (at most 64 per
segment, launches of at most 2^17 chunks), the resident schedule from 64 MB
of x, else the split schedule
with split_chunk's chunk (the largest of 8192, 4096, 2048 floats giving 768
workgroups per pass)."""
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
    assert "constexpr int kPipeChunk = kPipeTPB * 4 * kPipeCV;  // 4096 floats" in src
    assert "constexpr int kPipeTPB = 256, kPipeCV = 4;" in src
    assert "static constexpr int kPipeMaxChunks = 1 << 17;" in src
    assert "if (HW % kPipeChunk != 0 || L % kPipeChunk != 0) return false;" in src
    assert "if (cps < 1 || cps > 64) return false;" in src
    assert "const int64_t sb_max = kPipeMaxChunks / cps;" in src
    assert "const unsigned grid = (unsigned)(2 * sb * cps);" in src


def test_config_shapes():
    b = _bench()
    assert b.gn_dispatches((2, 1280, 8, 8)) == [("k_gn_single", 64 * 256)]           # 4d
    assert b.gn_dispatches((2, 320, 64, 64)) == [("k_gn_pipe", 2 * 64 * 10 * 256)]   # 4c: 10 chunks a segment
    assert b.gn_dispatches((1, 512, 128, 128)) == [("k_gn_pipe", 2 * 32 * 64 * 256)]  # 4a: 64 chunks a segment
    assert b.gn_dispatches((1, 128, 1024, 1024))[0][0] == "k_gn_resident_pipe<"   # 4b
    assert b.gn_dispatches((2, 640, 64, 64)) == [("k_gn_pipe", 2 * 64 * 20 * 256)]
    assert b.gn_dispatches((8, 512, 128, 128)) == [("k_gn_pipe", 2 * 256 * 64 * 256)]  # 128 MB of x
    assert b.gn_dispatches((80, 512, 128, 128)) == [("k_gn_pipe", 2 * 2048 * 64 * 256)]  # first of two launches
    # chunks that would cross channels, or more than 64 a segment: the split schedule
    assert b.gn_dispatches((2, 1280, 32, 32)) == [("k_gn_partial", 64 * 20 * 64), ("k_gn_apply", 64 * 20 * 64)]  # 2048-float chunks
    assert b.gn_dispatches((1, 64, 384, 384))[0][0] == "k_gn_partial"      # 72 chunks a segment, 38 MB


def test_split_chunk_rule():
    b = _bench()
    assert b.gn_split_chunk(32, 262144) == 8192      # 1024 workgroups
    assert b.gn_split_chunk(32, 230400) == 8192      # 928 workgroups
    assert b.gn_split_chunk(64, 81920) == 4096       # 640 at 8192, 1280 at 4096
    assert b.gn_split_chunk(64, 40960) == 2048
    assert b.gn_split_chunk(1, 100) == 2048
