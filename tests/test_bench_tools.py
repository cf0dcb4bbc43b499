"""Benchmark-history tools: bench_quick's CSV rows and bench_compare's join.

The CPU tests cover the schema and the comparison logic of
examples/bench_compare.rs (join on everything but the timings, last two
distinct commits by default, prefix match, concatenated headers, malformed
rows skipped, the 3 % markers), including rows in the reference's own
10-column format.  The GPU test runs bench_quick --csv end to end and feeds
its output back through bench_compare.
"""
from __future__ import annotations

import io
import os
from contextlib import redirect_stdout

import pytest

from flash_attention_amd import bench_compare as bc
from flash_attention_amd import bench_quick as bq

REF_HEADER = "timestamp,commit,os,arch,threads,variant,causal,seq_len,d_head,time_ms"


def _gpu_row(commit, variant, causal, seq, d, t, dt):
    return bq.csv_row(1800000000, commit, "linux", "x86_64", 256, variant, causal, seq, d, t, "gfx950", dt)


def test_csv_row_schema():
    row = _gpu_row("abc1234", "v2", True, 1024, 128, 1.23456, 0.0123456)
    assert row == "1800000000,abc1234,linux,x86_64,256,v2,true,1024,128,1.2346,gfx950,0.0123"
    assert bq.HEADER.split(",")[:10] == REF_HEADER.split(",")
    (r,) = bc.parse_csv(bq.HEADER + "\n" + row)
    assert r.key == bc.Key("linux", "x86_64", "gfx950", 256, "v2", True, 1024, 128)
    assert r.time_ms == pytest.approx(1.2346) and r.device_ms == pytest.approx(0.0123)


def test_shapes_and_runs_follow_bench_quick():
    # examples/bench_quick.rs: five shapes, naive + three variants x {non-causal, causal}
    assert bq.SHAPES == ((256, 64), (512, 64), (1024, 64), (2048, 64), (1024, 128))
    assert [(r[0], r[2]) for r in bq.RUNS] == [("naive", False), ("v1", False), ("v2", False), ("v3", False),
                                               ("v1", True), ("v2", True), ("v3", True)]


def test_commit_resolution_prefers_env(monkeypatch):
    monkeypatch.setenv("BENCH_COMMIT", "deadbee")
    assert bq.resolve_commit() == "deadbee"


def test_parse_reference_rows_and_skip_malformed():
    text = "\n".join([
        REF_HEADER,
        "1783478131,90d04f4,macos,aarch64,10,naive,false,256,64,1.5852",
        "1783478131,90d04f4,macos,aarch64,10,v1,true,256,64,0.1350",
        "garbage,row",
        "1783478131,90d04f4,macos,aarch64,ten,v1,true,256,64,0.1350",
        REF_HEADER,                      # concatenated per-target CSVs repeat the header
        "1783478200,90d04f4,linux,x86_64,4,v2,false,512,64,2.5",
    ])
    warnings = []
    rows = bc.parse_csv(text, warn=warnings.append)
    assert len(rows) == 3 and len(warnings) == 2
    assert rows[0].key.device == "cpu" and rows[0].device_ms is None
    assert bc.commits_in_order(rows) == ["90d04f4"]


def test_compare_joins_only_identical_targets():
    rows = bc.parse_csv("\n".join([
        bq.HEADER,
        _gpu_row("aaa1111", "v2", False, 1024, 64, 10.0, 1.00),
        _gpu_row("aaa1111", "v3", False, 1024, 64, 10.0, 1.00),
        _gpu_row("aaa1111", "v1", True, 1024, 64, 10.0, 1.00),     # not re-measured in bbb
        "1,aaa1111,linux,x86_64,8,v2,false,1024,64,50.0",          # a CPU row: never joined to GPU rows
        _gpu_row("bbb2222", "v2", False, 1024, 64, 9.0, 1.02),
        _gpu_row("bbb2222", "v3", False, 1024, 64, 10.5, 0.90),
        _gpu_row("bbb2222", "naive", False, 1024, 64, 30.0, 3.0),  # new shape/variant
    ]))
    assert bc.commits_in_order(rows) == ["aaa1111", "bbb2222"]
    lines, only_old, only_new = bc.compare(rows, "aaa1111", "bbb2222")
    text = "\n".join(lines)
    assert only_old == 2 and only_new == 1
    v2 = next(line for line in lines if " v2 " in line and "gfx950" in line)
    assert "-10.0% faster" in v2 and "+2.0% ~" in v2
    v3 = next(line for line in lines if " v3 " in line)
    assert "+5.0% SLOWER" in v3 and "-10.0% faster" in v3
    assert "new" in next(line for line in lines if "naive" in line)
    assert "linux/x86_64 " not in text.split("\n", 3)[3]   # the CPU-only row has no partner


def test_main_defaults_and_prefix_match(tmp_path):
    path = tmp_path / "history.csv"
    path.write_text("\n".join([bq.HEADER, _gpu_row("aaa1111", "v2", True, 256, 64, 2.0, 0.2),
                               _gpu_row("bbb2222", "v2", True, 256, 64, 1.0, 0.1),
                               _gpu_row("ccc3333", "v2", True, 256, 64, 4.0, 0.4)]) + "\n")
    buf = io.StringIO()
    with redirect_stdout(buf):
        assert bc.main(["--file", str(path)]) == 0
    assert buf.getvalue().startswith("comparing bbb2222 -> ccc3333")
    buf = io.StringIO()
    with redirect_stdout(buf):
        assert bc.main(["--file", str(path), "aaa", "bbb"]) == 0
    assert "comparing aaa1111 -> bbb2222" in buf.getvalue() and "-50.0% faster" in buf.getvalue()
    with pytest.raises(SystemExit):
        bc.main(["--file", str(path), "zzz", "bbb"])


def test_committed_history_parses():
    assert os.path.exists(bc.DEFAULT_HISTORY)
    with open(bc.DEFAULT_HISTORY, encoding="utf-8") as fh:
        text = fh.read()
    rows = bc.parse_csv(text, warn=lambda m: pytest.fail(m))
    assert rows and all(r.key.device.startswith("gfx") and r.device_ms is not None for r in rows)
    assert text.startswith(bq.HEADER)


@pytest.mark.gpu
def test_bench_quick_csv_end_to_end(tmp_path):
    buf = io.StringIO()
    with redirect_stdout(buf):
        assert bq.main(["--csv", "--iters", "2", "--dev-iters", "3"]) == 0
    lines = buf.getvalue().strip().splitlines()
    assert lines[0] == bq.HEADER_EXT and len(lines) == 1 + len(bq.SHAPES) * len(bq.RUNS)
    rows = bc.parse_csv(buf.getvalue(), warn=lambda m: pytest.fail(m))
    assert all(r.time_ms > 0 and r.device_ms > 0 and r.key.threads > 0 for r in rows)
    for line in lines[1:]:   # the GPU columns: algorithmic TFLOP/s and GB/s are always filled
        f = line.split(",")
        assert len(f) == 22 and f[12] == "" and float(f[15]) > 0 and float(f[17]) > 0, line
    # fed back twice under two commits, everything joins
    c1 = buf.getvalue().replace(f",{rows[0].commit},", ",old0001,")
    c2 = buf.getvalue().replace(f",{rows[0].commit},", ",new0002,")
    lines, only_old, only_new = bc.compare(bc.parse_csv(c1 + c2), "old0001", "new0002")
    assert only_old == 0 and only_new == 0 and len(lines) == 3 + len(rows)


def _ext_row(commit, workload, variant, sq, sk, heads, d, wall, dev, **cols):
    return bq.csv_row(1800000000, commit, "linux", "x86_64", 256, variant, True, sq, d, wall, "gfx950", dev,
                      workload=workload, seq_len_k=sk, heads=heads, **cols)


def test_extended_row_schema_and_gpu_columns():
    assert bq.HEADER_EXT.split(",")[:12] == bq.HEADER.split(",")
    assert bq.HEADER_EXT.split(",")[12:] == ["workload", "seq_len_k", "heads", "tflops", "pct_peak", "gbps",
                                             "pct_hbm", "mfma_busy", "lds_bank_conflicts", "fetch_gbps"]
    row = _ext_row("abc1234", "config2", "v3", 2048, 2048, 32, 128, 0.2712, 0.2704, tflops=127.1234,
                   pct_peak=80.81, mfma_busy=81.2, lds_bank_conflicts=0, fetch_gbps=612.34)
    assert row.split(",")[12:] == ["config2", "2048", "32", "127.123", "80.8", "", "", "81.2", "0", "612.3"]
    (r,) = bc.parse_csv(bq.HEADER_EXT + "\n" + row)
    assert r.key == bc.Key("linux", "x86_64", "gfx950", 256, "v3", True, 2048, 128, "config2", 2048, 32)
    assert r.rate == "127.1TF" and r.device_ms == pytest.approx(0.2704)
    dec = _ext_row("abc1234", "config4a", "v2", 1, 32768, 32, 128, 0.17, 0.16, gbps=6620.4, pct_hbm=82.8)
    (r,) = bc.parse_csv(dec)
    assert r.rate == "6620GB/s" and r.key.seq_len_k == 32768
    with pytest.raises(TypeError):
        bq.csv_row(1, "c", "linux", "x86_64", 1, "v1", False, 1, 1, 1.0, "gfx950", 1.0, bogus=1)


def test_gpu_columns_of_a_quick_row():
    # 1024^2 d64 non-causal in 0.1 ms: 4 * 64 * 1024^2 FLOP, 4 * 64 * 4 * 1024 bytes
    cols = bq.gpu_columns(0, 1024, 64, False, 0.1)
    assert cols["tflops"] == pytest.approx(4 * 64 * 1024 ** 2 / 1e-4 / 1e12)
    assert cols["pct_peak"] == pytest.approx(100 * cols["tflops"] / 157.3)
    assert cols["gbps"] == pytest.approx(4 * 64 * 4 * 1024 / 1e-4 / 1e9)
    causal = bq.gpu_columns(0, 1024, 64, True, 0.1)
    assert causal["tflops"] == pytest.approx(cols["tflops"] * 1025 / 2048)


def test_compare_keeps_workloads_apart_and_mixes_row_forms():
    rows = bc.parse_csv("\n".join([
        bq.HEADER,
        _gpu_row("aaa1111", "v2", True, 2048, 128, 3.0, 0.30),           # 12-column quick row
        bq.HEADER_EXT,
        _ext_row("aaa1111", "config2", "v2", 2048, 2048, 32, 128, 0.29, 0.29, tflops=118.0),
        _ext_row("aaa1111", "config3", "v2", 16384, 16384, 8, 128, 4.3, 4.3, tflops=127.0),
        _ext_row("bbb2222", "", "v2", 2048, 2048, 1, 128, 2.7, 0.27, tflops=20.0),   # same quick key
        _ext_row("bbb2222", "config2", "v2", 2048, 2048, 32, 128, 0.25, 0.25, tflops=137.0),
        _ext_row("bbb2222", "config3", "v2", 16384, 16384, 8, 128, 4.5, 4.5, tflops=122.0),
    ]))
    lines, only_old, only_new = bc.compare(rows, "aaa1111", "bbb2222")
    assert only_old == 0 and only_new == 0
    c2 = next(line for line in lines if "config2" in line)
    assert "-13.8% faster" in c2 and "118.0TF -> 137.0TF" in c2
    c3 = next(line for line in lines if "config3" in line)
    assert "SLOWER" in c3
    quick = [line for line in lines if "gfx950 " in line and "config" not in line]
    assert len(quick) == 1 and "-10.0% faster" in quick[0]
