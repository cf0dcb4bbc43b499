"""CPU unit tests of host-library pieces that need no GPU.

The copy-pool partition (csrc/fa_copy_parts.h) decides which bytes of a
host-slice upload or download each host thread copies.  A partition that
leaves a gap sends stale bytes of the pinned ring to the device, so every
byte count -- in particular the odd 16-bit ones, 2 * (128m + 1) -- must be
covered exactly once.  The header is compiled here with g++ on its own.

Also the arithmetic behind one 16-bit GPU test input (f16 probabilities in
the subnormal range).
"""
from __future__ import annotations

import os
import subprocess

import numpy as np

from fa_testutil import long_row_f16_case

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "flash-attention-cpu_amd", "csrc")

CHECK = r"""
#include <cstdio>
#include <cstdlib>
#include <vector>
#include "fa_copy_parts.h"

// Every byte of [0, n) covered by exactly one part, parts in order, each
// part starting on a 64-byte boundary.
static int check(size_t n, int parts) {
    size_t next = 0;
    for (int id = 0; id < parts; ++id) {
        size_t b, len;
        fa_copy_part_range(n, parts, id, &b, &len);
        if (len == 0) continue;
        if (b != next || b % 64 != 0 || b + len > n) {
            std::printf("bad part n=%zu parts=%d id=%d b=%zu len=%zu next=%zu\n", n, parts, id, b, len, next);
            return 1;
        }
        next = b + len;
    }
    if (next != n) {
        std::printf("gap n=%zu parts=%d covered=%zu\n", n, parts, next);
        return 1;
    }
    return 0;
}

int main() {
    int bad = 0;
    std::vector<size_t> ns = {0, 1, 2, 63, 64, 65, 255, 256, 257, 1053954, 8388614, (size_t)16 << 20};
    // n = 256m + r for r = 1, 2, 3 (odd 16-bit element counts give r = 2),
    // small m and m around the 1 MiB threading cut and the 16 MiB chunk.
    for (size_t m : {1ul, 2ul, 3ul, 100ul, 4095ul, 4096ul, 4117ul, 4118ul, 65535ul, 65536ul})
        for (size_t r : {1ul, 2ul, 3ul}) ns.push_back(256 * m + r);
    for (size_t n = 0; n < 4096; ++n) ns.push_back(n);
    for (size_t n : ns)
        for (int parts = 1; parts <= 8; ++parts) bad |= check(n, parts);
    std::printf(bad ? "FAIL\n" : "OK\n");
    return bad;
}
"""


def test_copy_pool_partition_covers_every_byte(tmp_path):
    src = tmp_path / "check_parts.cpp"
    exe = tmp_path / "check_parts"
    src.write_text(CHECK)
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-I", CSRC, str(src), "-o", str(exe)],
                   check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.strip().endswith("OK"), r.stdout


def test_long_row_f16_case_breaks_the_bound_without_scaling():
    """CPU check of fa_testutil.long_row_f16_case (run on the GPU by
    test_gpu_lp.py): the small probability as the 16-bit kernel forms it
    (exp2((s - m) c) in f32), rounded to f16 directly, misses the 16-bit
    bound; rounded as 2^7 p, as the kernel now does, it stays inside."""
    q, k, v, sq, sk, d = long_row_f16_case()
    c = np.float32(np.float32(1.0 / np.sqrt(np.float32(d))) * np.float32(1.4426950408889634))
    s1 = np.float32(4.0) * np.float32(k[d])   # q . k_j for j >= 1
    t = np.exp2((s1 - np.float32(48.0)) * c, dtype=np.float32)
    assert np.float32(2.0 ** -24) < t < np.float32(2.0 ** -14)   # subnormal in f16
    n = sk - 1

    def out(p):   # O column with every p_j = p (key 0: p = 1), V = -1 / +1
        return (-1.0 + n * p) / (1.0 + n * p)

    exact = out(float(t))
    u = 2.0 ** -11
    bound = u / (1.0 - u) + 2e-5   # the 16-bit bar at max|V| = 1
    direct = out(float(np.float16(t)))
    scaled = out(float(np.float16(t * np.float32(128.0))) / 128.0)
    assert abs(direct - exact) > 2.5 * bound
    assert abs(scaled - exact) < 0.5 * bound
