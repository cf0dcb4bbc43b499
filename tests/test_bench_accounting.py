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
    "wide_d2048": (68.753, 268435456),
    "wide_d4096": (68.753, 268435456),
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
    whose launches share a key would have their counters averaged."""
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
    assert shared == {}, shared



def _fake_configs():
    """An extra.configs dict shaped as bench.py builds it, every config and variant present."""
    configs = {}
    for (name, bh, sq, sk, d, causal, _s, _u, kind) in bench.CONFIGS:
        e = {"shape": "x" * 60, "flop": bench.flops_of(bh, sq, sk, d, causal), "bytes": bench.bytes_of(bh, sq, sk, d)}
        for var in ("v1", "v2", "v3"):
            ent = {"us": 12345.6}
            if kind == "prefill":
                ent.update(tflops=123.45, pct_peak=78.5, mfma_busy=81.2, lds_conflicts=0, hbm_mb=199.4,
                           fetch_gbs=612.3)
            else:
                ent.update(gbs=6620.4, pct_hbm=82.8, hbm_mb=1074.2, fetch_gbs=6600.1, mfma_busy=3.1,
                           lds_conflicts=0)
            e[var] = ent
        if name in ("config2", "config3", "config4a", "config5"):
            for t in ("bf16", "f16"):
                e[t] = {"us": 46.2, "tflops": 744.1, "pct_peak16": 29.8, "mfma_busy": 29.5, "lds_conflicts": 0}
        e["cpu_v2"] = {"ms": 23800.123, "calls": 200, "threads": 16, "gflops": 1444.44}
        e["parity"] = {"v1": [1.19e-6, 5.75e-7], "v2": [1.19e-6, 5.75e-7], "v3": [1.19e-6, 5.75e-7], "ok": True}
        configs[name] = e
    return configs


def test_summary_survives_a_2000_character_tail():
    """The driver keeps the last few KB of stderr: the closing summary (one
    line per config, every variant with time, rate, % of peak and parity)
    must fit in 2000 characters."""
    lines = bench.summary_lines(_fake_configs())
    text = "\n".join(lines)
    assert len(lines) == 1 + len(bench.CONFIGS)
    assert len(text) < 2000, len(text)
    c2 = next(line for line in lines if line.startswith("config2:"))
    assert "v3 12345.6us 123.5TF 78.5% m81" in c2 and "bf16 46.2us 744.1TF 29.8% m30" in c2
    assert c2.endswith("; 1.2e-06/5.8e-07 ok")
    c4 = next(line for line in lines if line.startswith("config4a:"))
    assert "v2 12345.6us 6620GB/s 82.8% |" in c4


def test_json_line_stays_compact():
    """The one stdout JSON line (every config's figures in extra.configs) stays
    well inside the driver's 16 KB stdout tail."""
    import json as _json
    line = _json.dumps({"metric": bench.METRIC, "extra": {"configs": _fake_configs()}}, separators=(",", ":"))
    assert len(line) < 9000, len(line)


def test_pmc_table_from_counter_runs(tmp_path):
    """build_pmc_table joins the two PMC passes per (kernel, launch size) and
    derives MFMA busy %, VALU per MFMA, wait share and LDS conflicts."""
    hdr = "Kernel_Name,Grid_Size,Counter_Name,Counter_Value\n"
    a = tmp_path / "a" / "x"
    b = tmp_path / "b" / "x"
    a.mkdir(parents=True)
    b.mkdir(parents=True)
    rows_a = [("SQ_VALU_MFMA_BUSY_CYCLES", 553648128), ("SQ_INSTS_MFMA", 17301504), ("SQ_INSTS_VALU", 23087104),
              ("SQ_WAVE_CYCLES", 322.0e6), ("SQ_WAIT_INST_ANY", 190.8e6), ("GRBM_GUI_ACTIVE", 5327934),
              ("SQ_BUSY_CYCLES", 1.0)]
    rows_b = [("SQ_LDS_BANK_CONFLICT", 0), ("SQ_LDS_IDX_ACTIVE", 17301504), ("SQ_INSTS_LDS", 4325376),
              ("GRBM_GUI_ACTIVE", 5327934)]
    (a / "run_counter_collection.csv").write_text(
        hdr + "".join(f"fa_k,131072,{c},{v}\n" for c, v in rows_a) + "other_kernel,64,GRBM_GUI_ACTIVE,5\n")
    (b / "run_counter_collection.csv").write_text(hdr + "".join(f"fa_k,131072,{c},{v}\n" for c, v in rows_b))
    table = traffic.build_pmc_table(str(tmp_path / "a"), str(tmp_path / "b"))
    assert list(table) == ["fa_k@131072"]
    e = table["fa_k@131072"]
    # 553.6 M busy cycles over (5,327,934 / 8 XCDs) x 1024 SIMDs
    assert e["mfma_busy_pct"] == pytest.approx(81.2, abs=0.05)
    assert e["valu_per_mfma"] == pytest.approx((23087104 - 17301504) / 17301504, abs=0.005)
    assert e["wait_pct"] == pytest.approx(59.3, abs=0.05)
    assert e["lds_bank_conflicts"] == 0 and e["kernel_source_sha256"] == traffic.kernel_source_hash()
    path = tmp_path / "pmc.json"
    path.write_text(json.dumps(table))
    assert traffic.lookup_entry(str(path), "fa_k", 131072)["mfma_busy_pct"] == e["mfma_busy_pct"]
    assert traffic.lookup_entry(str(path), "fa_k", 64) is None


def test_profile_report_covers_every_bench_launch(tmp_path):
    """profile_report plans every benchmark call (f32 variants and 16-bit
    forms) and lists each (kernel, launch size) of the committed tables
    under the workloads that launch it; every prefill / decode kernel of the
    bench has a row in both committed tables (profiles/ measured on the
    current kernel sources)."""
    from flash_attention_amd import profile_report as pr
    calls = pr.workload_launches()
    labels = {c["label"] for c in calls}
    for (name, *_rest) in bench.CONFIGS:
        assert {f"{name} v1", f"{name} v2", f"{name} v3"} <= labels
    assert {"config2 bf16", "config2 f16", "config3 bf16", "config4a bf16", "config5 f16"} <= labels
    traffic_t = json.load(open(os.path.join(ROOT, "profiles", "traffic.json")))
    pmc_t = json.load(open(os.path.join(ROOT, "profiles", "pmc.json")))
    src = traffic.kernel_source_hash()
    for c in calls:
        for k, g in c["launches"]:
            for t in (traffic_t, pmc_t):
                e = t.get(f"{k}@{g}")
                assert e is not None, (c["label"], k, g)
                assert e["kernel_source_sha256"] == src, (c["label"], k)
    md = pr.counters_markdown(pmc_t, calls)
    assert "| fa_prefill_v3_d128_2 | 131072 | config2 v3 |" in md
    md = pr.traffic_markdown(traffic_t, calls)
    assert "| fa_prefill_v3_d128_2 | 131072 | config2 v3 |" in md and "134.2 MB" in md
