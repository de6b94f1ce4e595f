"""The host-side slot runs of the span decode kernel (chunk_runs in
nh_forward.hip) against the per-key mapping the kernel's gather path uses
(slot_of(span_key(...)), infer.rs:1749-1756,1770-1826), on random spans,
rings, windows and chunk sizes: every key of every chunk must get the same
slot through its run, by the kernel's own rule (the last run starting at or
before the key).  The functions are compiled from the library's source with
g++ (host code only)."""
import os
import re
import shutil
import subprocess

import pytest

SRC = os.path.join(os.path.dirname(__file__), "..", "needle-rs_amd", "csrc", "nh_forward.hip")


def _grab(src: str, start: str, end: str = "\n}\n") -> str:
    a = src.index(start)
    return src[a:src.index(end, a) + len(end)]


def _constant(src: str, name: str) -> str:
    m = re.search(r"constexpr int %s = ([^;]+);" % name, src)
    assert m, name
    return "constexpr int %s = %s;\n" % (name, m.group(1))


HARNESS = r"""
int main() {
    std::mt19937 rng(7);
    long keys = 0, fitting = 0;
    for (int it = 0; it < 20000; ++it) {
        Dims D{(int)(rng() % 200), 1 + (int)(rng() % 400)};
        const int p0 = (int)(rng() % 900);
        KeySpan K{};
        K.end = p0 + 1;
        int pos = 0;
        const int want_runs = 1 + (int)(rng() % 4);
        for (int r = 0; r < want_runs && pos < K.end; ++r) {
            const int lo = pos + (int)(rng() % 40);
            if (lo >= K.end) break;
            const int hi = std::min(K.end, lo + 1 + (int)(rng() % 500));
            K.lo[K.nrun] = lo; K.hi[K.nrun] = hi; ++K.nrun; pos = hi;
        }
        if (K.nrun == 0 || K.hi[K.nrun - 1] != K.end) {
            K.lo[K.nrun] = std::max(pos, K.end - 1); K.hi[K.nrun] = K.end;
            if (K.lo[K.nrun] < K.hi[K.nrun]) ++K.nrun;
        }
        const int lo = rng() % 3 == 0 ? std::max(0, p0 + 1 - 256) : 0;
        int alo, ahi, blo, bhi;
        span_ranges(D, K, lo, p0, alo, ahi, blo, bhi);
        int n = 0;
        for (int r = 0; r < K.nrun; ++r)
            n += span_overlap(K.lo[r], K.hi[r], alo, ahi) + span_overlap(K.lo[r], K.hi[r], blo, bhi);
        if (n < 1) continue;
        const int chunk = 16 * (1 + (int)(rng() % 16)), count = (n + chunk - 1) / chunk;
        ChunkRuns R{};
        if (!chunk_runs(D, K, lo, p0, n, count, chunk, R)) continue;
        ++fitting;
        for (int k = 0; k < n; ++k) {
            const int want = slot_of(D, span_key(K, alo, ahi, blo, bhi, k));
            const int c = k / chunk, j = k - c * chunk;
            int got = R.slot0[c][0] + (j - R.key0[c][0]);
            for (int r = 1; r < DC_RUNS; ++r)
                if (j >= R.key0[c][r]) got = R.slot0[c][r] + (j - R.key0[c][r]);
            if (got != want) { std::printf("case %d key %d: run slot %d, key slot %d\n", it, k, got, want); return 1; }
            ++keys;
        }
    }
    std::printf("fitting %ld keys %ld ok\n", fitting, keys);
    return fitting > 1000 ? 0 : 2;
}
"""


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_chunk_runs_match_key_slots(tmp_path):
    src = open(SRC).read()
    code = "".join([
        "#include <algorithm>\n#include <cstdio>\n#include <random>\nusing std::min; using std::max;\n",
        _constant(src, "DC_RUNS"), _constant(src, "DC_RUN_CHUNKS"), _constant(src, "RUN_NONE"),
        _constant(src, "RUN_CHUNK"),
        "constexpr int SPAN_RUNS = 24;\n",
        "struct Dims { int sink, ring; };\n",
        "struct KeySpan { int end; int nrun; int lo[SPAN_RUNS], hi[SPAN_RUNS]; };\n",
        _grab(src, "struct ChunkRuns {", "\n};\n"),
        _grab(src, "__host__ __device__ inline void span_ranges("),
        _grab(src, "__host__ __device__ inline int span_overlap("),
        _grab(src, "__device__ __forceinline__ int span_key("),
        _grab(src, "__device__ __forceinline__ int slot_of("),
        _grab(src, "static bool chunk_runs("),
        HARNESS,
    ]).replace("__host__ __device__ inline", "inline").replace("__device__ __forceinline__", "inline")
    # the kernel-side SPAN_RUNS must match the harness's KeySpan
    assert "constexpr int SPAN_RUNS = 24;" in open(os.path.join(os.path.dirname(SRC), "nh_forward.h")).read()
    cpp = tmp_path / "runs.cpp"
    cpp.write_text(code)
    exe = tmp_path / "runs"
    subprocess.run(["g++", "-O1", "-std=c++17", str(cpp), "-o", str(exe)], check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ok" in r.stdout
