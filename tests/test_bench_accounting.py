"""bench.py's accounting, checked on the CPU.

* Algorithmic FLOP (4 * d * visible pairs * heads, causal counting j <= i)
  and bytes (Q, K, V read once, O written once, f32) for every benchmark
  configuration, against the figures stated for them independently of this
  code (34.377 GFLOP and 134.2 MB for the headline, ...).
* The launch-size parser used to key traffic entries.
* The traffic table refuses a figure measured on other kernel sources.
"""
from __future__ import annotations

import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from flash_attention_amd import traffic  # noqa: E402

STATED = {   # name: (GFLOP, bytes)
    "config1": (0.01678, 262144),
    "config2": (34.377, 134217728),
    "config3": (549.79, 268435456),
    "config4a": (0.537, 1073774592),
    "config4b": (8.590, 1074266112),
    "config5": (68.719, 167772160),
    "config5c": (8.200, 65536000),
    # 4 * d * 2048 * 2049 / 2 * heads; Q, K, V, O of heads x 2048 x d f32
    "wide_d512": (68.753, 268435456),
    "wide_d1024": (68.753, 268435456),
    # 4 * 128 * 2048 * 768; 4 * 768 * 128 * (2 * 1 + 2 * 2048)
    "decode_batched": (0.80531, 1611399168),
}


@pytest.mark.parametrize("cfg", bench.CONFIGS, ids=[c[0] for c in bench.CONFIGS])
def test_algorithmic_flop_and_bytes(cfg):
    name, bh, sq, sk, d, causal = cfg[:6]
    gflop, nbytes = STATED[name]
    assert bench.flops_of(bh, sq, sk, d, causal) / 1e9 == pytest.approx(gflop, rel=2e-3)
    assert bench.bytes_of(bh, sq, sk, d) == nbytes


def test_visible_pairs_brute_force():
    for sq, sk in ((1, 1), (5, 3), (3, 5), (17, 17), (40, 10), (10, 40)):
        brute = sum(1 for i in range(sq) for j in range(sk) if j <= i)
        assert bench.visible_pairs(sq, sk, True) == brute
        assert bench.visible_pairs(sq, sk, False) == sq * sk


def test_grid_threads_parses_describe_launch():
    assert bench.grid_threads("fa_prefill_v3_d128_2 grid=256x1x1 block=512 two_blocks") == 131072
    s = ("fa_decode_rows_d128_q1 grid=16x1x32 block=256; fa_merge_d128 grid=32x1x1 block=64; "
         "splits=16 split_len=2048 workspace=4259840")
    assert bench.grid_threads(s) == 16 * 32 * 256


def test_traffic_lookup_requires_matching_kernel_sources(tmp_path):
    path = tmp_path / "traffic.json"
    ent = {"kernel": "fa_x", "grid_threads": 64, "hbm_bytes_per_launch": 123,
           "kernel_source_sha256": traffic.kernel_source_hash()}
    path.write_text(json.dumps({"fa_x@64": ent}))
    assert traffic.lookup(str(path), "fa_x", 64) == (123, "ok")
    assert traffic.lookup(str(path), "fa_x", 128)[0] is None
    ent["kernel_source_sha256"] = "0" * 16
    path.write_text(json.dumps({"fa_x@64": ent}))
    assert traffic.lookup(str(path), "fa_x", 64) == (None, "profiled on other kernel sources")


def test_bench_rows_have_distinct_launch_keys():
    """profiles/ key kernel figures by (kernel, launch size): two bench rows
    whose launches share a key would have their counters averaged.  The one
    shared key is v1 of configs 4a and 4b, the same kernel over the same 32
    prefill blocks and the same K / V bytes."""
    import flash_attention_amd as fa
    use = {}
    for (name, bh, sq, sk, d, causal, *_rest) in bench.CONFIGS:
        plans = [fa.describe_launch(v, 1, bh, sq, sk, d, causal) for v in (1, 2, 3)]
        if name in ("config2", "config3", "config4a", "config5"):
            plans += [fa.describe_launch(3, 1, bh, sq, sk, d, causal, dtype=t) for t in (fa.DTYPE_BF16, fa.DTYPE_F16)]
        for plan in plans:
            for part in plan.split("; "):
                if "grid=" in part:
                    use.setdefault((part.split()[0], bench.grid_threads(part)), set()).add(name)
    shared = {k: v for k, v in use.items() if len(v) > 1}
    assert shared == {("fa_prefill_v1_d128_1", 16384): {"config4a", "config4b"}}, shared

