"""The stream split's index arithmetic, checked on the CPU.

The prefill kernel (prefill_body in csrc/fa_kernels.hip) cuts the key stages
of every (slice, query block) into equal runs, one per workgroup, and each
run into segments; fa_merge finds the partials of a shared block again.
This test walks the same arithmetic in Python for many shapes and checks the
invariants the kernels rely on, against brute-force enumeration:

* every (slice, block, stage) unit is processed exactly once, and the
  per-block stage counts equal ceil(block key end / SK) (causal: the block's
  last row + 1, capped at seq_k; the reference's causal tile skip,
  src/v2.rs:208-212);
* the closed-form block lookup (with its float square-root estimate) agrees
  with a linear search;
* a block touched by one workgroup is written directly; the partial slots
  (workgroup + global block) are unique and below the slot count the host
  allocates, and the merge's slots for a block are exactly those written;
* the workgroups sharing one block never exceed the host's slot bound.

The key split's compact grid (map_block_split) is checked the same way: the
splits whose workgroups store a partial of a block are exactly the splits
fa_merge reads for its rows.
"""
from __future__ import annotations

import math

import numpy as np
import pytest


def geom(sk, bq, skk, causal, nqb=None):
    # the kernel clamps bf to the block count (no block past the last query block exists)
    bf = sk // bq if nqb is None else min(sk // bq, nqb)
    return {"R": bq // skk, "nsf": -(-sk // skk), "bf": bf, "causal": causal}


def prefix(g, b):
    if not g["causal"]:
        return b * g["nsf"]
    if b <= g["bf"]:
        return g["R"] * (b * (b + 1) // 2)
    return g["R"] * (g["bf"] * (g["bf"] + 1) // 2) + (b - g["bf"]) * g["nsf"]


def stages(g, b):
    return g["R"] * (b + 1) if (g["causal"] and b < g["bf"]) else g["nsf"]


def block_of(g, r):
    if not g["causal"]:
        return r // g["nsf"]
    tri = g["R"] * (g["bf"] * (g["bf"] + 1) // 2)
    if r >= tri:
        return g["bf"] + (r - tri) // g["nsf"]
    b = int((np.sqrt(np.float32(8.0) * np.float32(r // g["R"]) + np.float32(1.0)) - np.float32(1.0))
            * np.float32(0.5))
    while b > 0 and prefix(g, b) > r:
        b -= 1
    while prefix(g, b + 1) <= r:
        b += 1
    return b


def plan(bh, sq, sk, bq, skk, causal, want):
    """Host side (make_plan's stream_fit)."""
    nqb = -(-sq // bq)
    g = geom(sk, bq, skk, causal, nqb)
    u_head = prefix(g, nqb)
    utot = bh * u_head
    per = max(4, -(-utot // want))
    wgs = -(-utot // per)
    max_st = -(-(min(sk, nqb * bq) if causal else sk) // skk)
    segs = -(-max_st // per) + 1
    slots = wgs + bh * nqb - 1
    return g, nqb, u_head, per, wgs, segs, slots


CASES = [
    # bh, sq, sk, rows per block, stage keys, causal, workgroups wanted
    (16, 1000, 1000, 128, 16, True, 256), (16, 1000, 1000, 128, 32, True, 256), (3, 300, 300, 64, 16, True, 256),
    (1, 256, 256, 128, 64, False, 256), (4, 2048, 2048, 128, 64, True, 256), (2, 2000, 700, 128, 64, True, 100),
    (5, 77, 5000, 32, 16, True, 7), (7, 129, 129, 128, 64, True, 3), (1, 5000, 130, 128, 64, True, 256),
    (2, 1000, 1000, 128, 16, False, 1000), (9, 640, 1000, 64, 16, True, 256), (1, 1, 1, 128, 64, True, 256),
]


def _random_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        bq, skk = [(128, 64), (128, 32), (128, 16), (64, 16), (32, 16)][rng.integers(0, 5)]
        out.append((int(rng.integers(1, 9)), int(rng.integers(1, 3000)), int(rng.integers(1, 3000)), bq, skk,
                    bool(rng.integers(0, 2)), int(rng.integers(1, 600))))
    return out


@pytest.mark.parametrize("case", CASES + _random_cases(60, 2024))
def test_stream_split_covers_every_unit_once(case):
    bh, sq, sk, bq, skk, causal, want = case
    g, nqb, u_head, per, wgs, segs, slots = plan(bh, sq, sk, bq, skk, causal, want)
    for b in range(nqb):   # stage counts and prefix sums against brute force
        kend = min(sk, (b + 1) * bq) if causal else sk
        assert stages(g, b) == -(-kend // skk)
        assert prefix(g, b) == sum(stages(g, x) for x in range(b))
    for r in range(u_head):
        b = max(x for x in range(nqb) if prefix(g, x) <= r)
        assert block_of(g, r) == b, r
    seen = np.zeros(bh * u_head, np.int32)
    written = {}           # (h, b) -> list of slots, or "direct"
    used_slots = set()
    for wg in range(wgs):
        u, uend = wg * per, min(wg * per + per, bh * u_head)
        while u < uend:
            h, r = divmod(u, u_head)
            b = block_of(g, r)
            s0 = r - prefix(g, b)
            cnt = min(stages(g, b) - s0, uend - u)
            ub = h * u_head + prefix(g, b)
            first, last = ub // per, (ub + stages(g, b) - 1) // per
            seen[u:u + cnt] += 1
            if first == last:
                assert s0 == 0 and cnt == stages(g, b)
                written[(h, b)] = "direct"
            else:
                slot = wg + h * nqb + b
                assert 0 <= slot < slots and slot not in used_slots
                used_slots.add(slot)
                written.setdefault((h, b), []).append(slot)
                assert last - first + 1 <= segs
            u += cnt
    assert np.all(seen == 1)
    for h in range(bh):
        for b in range(nqb):
            ub = h * u_head + prefix(g, b)
            first, last = ub // per, (ub + stages(g, b) - 1) // per
            if first == last:
                assert written[(h, b)] == "direct"
            else:   # fa_merge's slots: first + j + h * nqb + b, j < last - first + 1
                assert sorted(written[(h, b)]) == [first + j + h * nqb + b for j in range(last - first + 1)]


def _key_split_cases():
    rng = np.random.default_rng(77)
    cases = [(16, 1000, 1000, 256, True, 3), (1, 300, 700, 64, False, 3), (1, 300, 700, 64, True, 6),
             (4, 1000, 1000, 512, True, 0), (2, 100, 700, 1024, False, 3), (3, 700, 200, 128, True, 5)]
    for _ in range(40):
        cases.append((int(rng.integers(1, 5)), int(rng.integers(1, 1500)), int(rng.integers(1, 3000)),
                      int(rng.choice([32, 64, 100, 128, 256, 300, 512, 1024])), bool(rng.integers(0, 2)),
                      int(rng.integers(2, 12))))
    return cases


@pytest.mark.parametrize("variant", (1, 3))
@pytest.mark.parametrize("case", _key_split_cases())
def test_key_split_writers_match_merged_splits(case, variant):
    """map_block_split's compact grid: split y holds every block whose key
    range reaches y * split_len (causal v2/v3: blocks qb >= floor(y *
    split_len / rows); v1 visits every key, so every block).  For each block,
    the splits listed (the partials written) must be the splits fa_merge
    reads: the first min(num_splits, ceil(block key end / split_len))."""
    import flash_attention_amd as fa
    bh, sq, sk, d, causal, splits = case
    skip_future = causal and variant != 1   # v1: no causal skip (src/v1.rs:209-216)
    try:
        s = fa.describe_launch(variant, 1, bh, sq, sk, d, causal, fa.PATH_PREFILL, splits)
    except fa.FaError:
        pytest.skip("plan refused")
    if "split_len=" not in s or "stream_per" in s:
        pytest.skip("no key split for this shape")
    nks = int(s.split("splits=")[1].split()[0])
    split_len = int(s.split("split_len=")[1].split()[0])
    grid = int(s.split("grid=")[1].split("x")[0])
    rows = {512: 64, 1024: 32}.get(max(32, 1 << (d - 1).bit_length()), 128)
    nqb = -(-sq // rows)
    writers = [0] * nqb
    listed = 0
    for y in range(nks):
        cnt = nqb - (y * split_len) // rows if skip_future else nqb
        for rank in range(max(cnt, 0)):
            writers[nqb - 1 - rank if causal else rank] += 1
        listed += max(cnt, 0) * bh
    assert listed == grid, s
    for qb in range(nqb):
        kend = min(sk, (qb + 1) * rows) if skip_future else sk
        assert writers[qb] == min(nks, -(-kend // split_len)), (qb, s)


@pytest.mark.parametrize("case", CASES[:6] + _random_cases(20, 7))
def test_v1_stream_split_counts_every_key(case):
    """v1 visits every key of every block, causal or not: its stream split
    is planned on the non-causal unit geometry (each block nsf stages), which
    test_stream_split_covers_every_unit_once checks; here the host's plan for
    v1 must match that geometry's run length and workgroup count."""
    import flash_attention_amd as fa
    bh, sq, sk, bq, skk, causal, want = case
    d = {64: 64, 32: 256}.get(skk) if bq == 128 else None
    if d is None:
        pytest.skip("v1 stages of 128-row blocks: 64 keys at d <= 128, 32 at d = 256")
    try:
        s = fa.describe_launch(1, 1, bh, sq, sk, d, causal, fa.PATH_STREAM, want)
    except fa.FaError:
        pytest.skip("plan refused")
    g, nqb, u_head, per, wgs, segs, slots = plan(bh, sq, sk, bq, skk, False, want)
    assert f"stream_per={per}" in s and f"grid={wgs}x1x1" in s, (s, per, wgs)
