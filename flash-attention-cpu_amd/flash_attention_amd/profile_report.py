"""Markdown reports of the rocprofv3 figures behind bench.py, one row per kernel launch.

Every benchmark workload (bench.CONFIGS, each f32 variant and the 16-bit
forms) is planned with fa_describe_launch, which names the kernels and grids
a call launches; the profile tables (profiles/traffic.json from FETCH_SIZE /
WRITE_SIZE runs, profiles/pmc.json from the two SQ counter passes, both
built by flash_attention_amd.traffic) are keyed by kernel name and launch
size, so each row lists the workloads that launch it.

    python -m flash_attention_amd.profile_report --traffic ../profiles/traffic.json \\
        --pmc ../profiles/pmc.json --out-dir ../profiles [--trace <kernel-trace run dir>]

writes pmc_traffic_bench_all_configs.md (HBM bytes per launch against the
algorithmic bytes of the call), pmc_counters_bench_all_configs.md (MFMA busy
%, non-MFMA VALU per MFMA, wait share, LDS bank conflicts) and, given a
kernel-trace run, kernel_stats_bench_default.md (durations per launch size).
Runs on the CPU (planning needs no GPU).
"""
from __future__ import annotations

import argparse
import json
import os
import sys

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROOT = os.path.dirname(_PKG_DIR)

PMC_COMMANDS = """rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CYCLES SQ_INSTS_VALU SQ_INSTS_MFMA SQ_WAVE_CYCLES SQ_WAIT_INST_ANY GRBM_GUI_ACTIVE -d gpurun_out/pmcA -o run -f csv -- python3 bench.py --steps 3 --warmup 1 --no-cpu-baseline
rocprofv3 --pmc SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_INSTS_LDS SQ_WAIT_INST_LDS SQ_LDS_ADDR_CONFLICT GRBM_GUI_ACTIVE -d gpurun_out/pmcB -o run -f csv -- python3 bench.py --steps 3 --warmup 1 --no-cpu-baseline
cd flash-attention-cpu_amd && python3 -m flash_attention_amd.traffic --pmc-a ../gpurun_out/pmcA --pmc-b ../gpurun_out/pmcB --out ../profiles/pmc.json"""

TRAFFIC_COMMANDS = """rocprofv3 --pmc FETCH_SIZE -d gpurun_out/tr_fetch -o run -f csv -- python3 bench.py --no-cpu-baseline --steps 5 --warmup 1
rocprofv3 --pmc WRITE_SIZE -d gpurun_out/tr_write -o run -f csv -- python3 bench.py --no-cpu-baseline --steps 5 --warmup 1
rocprofv3 --pmc FETCH_SIZE -d gpurun_out/tr_cf -o run -f csv -- python3 bench.py --calibrate-copy-mib 1024
rocprofv3 --pmc WRITE_SIZE -d gpurun_out/tr_cw -o run -f csv -- python3 bench.py --calibrate-copy-mib 1024
cd flash-attention-cpu_amd && python3 -m flash_attention_amd.traffic --fetch ../gpurun_out/tr_fetch \\
    --write ../gpurun_out/tr_write --copy-fetch ../gpurun_out/tr_cf --copy-write ../gpurun_out/tr_cw \\
    --copy-mib 1024 --out ../profiles/traffic.json"""

TRACE_COMMANDS = """rocprofv3 --kernel-trace --stats -d gpurun_out/ks -o run -f csv -- python3 bench.py --no-cpu-baseline"""

REPORT_COMMAND = ("cd flash-attention-cpu_amd && python3 -m flash_attention_amd.profile_report "
                  "--traffic ../profiles/traffic.json --pmc ../profiles/pmc.json --out-dir ../profiles")


def _bench():
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    import bench   # the repository's bench.py: workloads and their algorithmic bytes
    return bench


def _launches(plan: str) -> list[tuple[str, int]]:
    out = []
    for part in plan.split(";"):
        f = part.split()
        if len(f) >= 3 and f[1].startswith("grid=") and f[2].startswith("block="):
            g = [int(x) for x in f[1].split("=")[1].split("x")]
            out.append((f[0], g[0] * g[1] * g[2] * int(f[2].split("=")[1])))
    return out


def workload_launches() -> list[dict]:
    """One entry per benchmark call: label, its launches (kernel, grid threads)
    in order, its algorithmic bytes and FLOP, and whether it is a decode shape."""
    from . import DTYPE_BF16, DTYPE_F16, describe_launch

    bench = _bench()
    calls = []
    for (name, bh, sq, sk, d, causal, _sig, _vu, kind) in bench.CONFIGS:
        for var in (1, 2, 3):
            plan = describe_launch(var, 1, bh, sq, sk, d, causal)
            calls.append({"label": f"{name} v{var}", "launches": _launches(plan), "kind": kind,
                          "bytes": bench.bytes_of(bh, sq, sk, d), "flop": bench.flops_of(bh, sq, sk, d, causal)})
        if name in ("config2", "config3", "config4a", "config5"):
            for tname, dt in (("bf16", DTYPE_BF16), ("f16", DTYPE_F16)):
                if name == "config3" and tname == "f16":
                    continue
                plan = describe_launch(3, 1, bh, sq, sk, d, causal, dtype=dt)
                calls.append({"label": f"{name} {tname}", "launches": _launches(plan), "kind": kind,
                              "bytes": bh * d * (2 * sq + 4 * sk + 4 * sq), "flop": bench.flops_of(bh, sq, sk, d, causal)})
    return calls


def _users(calls):
    users: dict[tuple[str, int], list[str]] = {}
    for c in calls:
        for i, key in enumerate(c["launches"]):
            users.setdefault(key, []).append(c["label"] + (" (merge)" if i > 0 else ""))
    return users


def _load(path):
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


def traffic_markdown(traffic: dict, calls) -> str:
    users = _users(calls)
    src = next(iter(traffic.values()))["kernel_source_sha256"] if traffic else "-"
    fs = next(iter(traffic.values()))["fetch_scale"] if traffic else 0
    ws = next(iter(traffic.values()))["write_scale"] if traffic else 0
    lines = [
        "# HBM traffic per launch, every benchmark workload (rocprofv3 FETCH_SIZE / WRITE_SIZE)", "",
        f"Kernel sources sha256 `{src}` (`flash_attention_amd.traffic.kernel_source_hash()`); bench.py reports",
        "`roofline.traffic` and each config's `hbm_mb` / `fetch_gbs` from `profiles/traffic.json` only while the",
        "sources hash the same.", "",
        "Commands (one MI355X, repo root; each counter in its own run, then the same counters on a plain",
        "1 GiB device copy, `__amd_rocclr_copyBuffer`, to calibrate them), then this report:", "", "```",
        TRAFFIC_COMMANDS, REPORT_COMMAND, "```", "",
        f"Calibration: the copy reads and writes 1 GiB per dispatch; FETCH_SIZE x {fs:.4f} and WRITE_SIZE x "
        f"{ws:.4f} give the bytes moved.  Means per dispatch (KiB, raw; dispatches include bench.py's untimed "
        "clock-ramp calls).  Entries are keyed by kernel and launch size (threads in the grid).  The call ratio "
        "divides all of a call's launches (kernel + merge) by its algorithmic bytes (Q, K, V read once, O written "
        "once; 16-bit inputs at 2 bytes).", "",
        "| Kernel | Grid threads | Workloads | FETCH_SIZE | WRITE_SIZE | HBM bytes (scaled) | Algorithmic bytes | Call ratio |",
        "|---|---|---|---|---|---|---|---|",
    ]
    for c in calls:
        first = c["launches"][0] if c["launches"] else None
        ent = traffic.get(f"{first[0]}@{first[1]}") if first else None
        if ent is None or ent.get("_listed"):
            continue
        call_bytes = sum(traffic.get(f"{k}@{g}", {}).get("hbm_bytes_per_launch", 0) for k, g in c["launches"])
        for i, (k, g) in enumerate(c["launches"]):
            e = traffic.get(f"{k}@{g}")
            if e is None or e.get("_listed"):
                continue
            e["_listed"] = True
            ratio = f"{call_bytes / c['bytes']:.3f}" if i == 0 else "—"
            alg = f"{c['bytes'] / 1e6:.1f} MB" if i == 0 else "—"
            lines.append(f"| {k} | {g} | {', '.join(users.get((k, g), []))} | {e['fetch_kib_raw']:,.0f} | "
                         f"{e['write_kib_raw']:,.0f} | {e['hbm_bytes_per_launch'] / 1e6:.1f} MB | {alg} | {ratio} |")
    for e in traffic.values():
        e.pop("_listed", None)
    return "\n".join(lines) + "\n"


def counters_markdown(pmc: dict, calls) -> str:
    users = _users(calls)
    src = next(iter(pmc.values()))["kernel_source_sha256"] if pmc else "-"
    lines = [
        "# MFMA utilisation, VALU, waits and LDS conflicts per kernel launch, every benchmark workload (rocprofv3 PMC)",
        "",
        f"Kernel sources sha256 `{src}`; bench.py reports each config's `mfma_busy` / `lds_conflicts` from",
        "`profiles/pmc.json` only while the sources hash the same.", "",
        "Commands (one MI355X, repo root; the two counter passes in runs of their own), then this report:", "",
        "```", PMC_COMMANDS, REPORT_COMMAND, "```", "",
        "Columns, per dispatch (means over every dispatch at that launch size, bench.py's clock-ramp calls",
        "included): **MFMA busy** = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 XCDs x 1024 SIMDs), the share",
        "of SIMD cycles issuing MFMA while the GPU was active (for a launch-bound kernel the active time includes",
        "dispatch); **VALU / MFMA** = (SQ_INSTS_VALU - SQ_INSTS_MFMA) / SQ_INSTS_MFMA; **waiting** =",
        "SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES; **LDS bank conflicts** = SQ_LDS_BANK_CONFLICT cycles per launch and",
        "their share of SQ_LDS_IDX_ACTIVE.  The decode and merge kernels are HBM-bound (their MFMA busy is",
        "naturally low); the prefill kernels are MFMA-bound.", "",
        "| Kernel | Grid threads | Workloads | MFMA busy | MFMA insts | VALU / MFMA | Waiting | LDS bank conflicts | LDS insts |",
        "|---|---|---|---|---|---|---|---|---|",
    ]
    seen = set()
    for c in calls:
        for (k, g) in c["launches"]:
            e = pmc.get(f"{k}@{g}")
            if e is None or (k, g) in seen:
                continue
            seen.add((k, g))
            busy = "—" if e["mfma_busy_pct"] is None else f"{e['mfma_busy_pct']:.1f} %"
            vpm = "—" if e["valu_per_mfma"] is None else f"{e['valu_per_mfma']:.2f}"
            wait = "—" if e["wait_pct"] is None else f"{e['wait_pct']:.0f} %"
            lines.append(f"| {k} | {g} | {', '.join(users.get((k, g), []))} | {busy} | {e['mfma_insts']:,} | {vpm} | "
                         f"{wait} | {e['lds_bank_conflicts']:,} ({e['lds_conflict_pct']:.2f} %) | {e['lds_insts']:,} |")
    return "\n".join(lines) + "\n"


def trace_markdown(run_dir: str, calls, src: str) -> str:
    from .traffic import trace_table

    users = _users(calls)
    rows = sorted(trace_table(run_dir).items(), key=lambda kv: -kv[1]["avg_us"] * kv[1]["calls"])
    lines = [
        "# Kernel durations per workload: bench.py default run (rocprofv3 kernel trace)", "",
        f"Kernel sources sha256 `{src}`.  Commands (one MI355X, repo root):", "", "```",
        TRACE_COMMANDS,
        "cd flash-attention-cpu_amd && python3 -m flash_attention_amd.profile_report --traffic ../profiles/traffic.json "
        "--pmc ../profiles/pmc.json --out-dir ../profiles --trace ../gpurun_out/ks",
        "```", "",
        "The name-keyed `run_kernel_stats.csv` mixes launch sizes (one kernel serves several configs), so this",
        "table is the kernel trace grouped by kernel and launch size; library kernels only.  Call counts include",
        "bench.py's untimed clock-ramp calls (0.3 s of the same call before every measurement), its warm-ups and",
        "the host-slice calls, so averages sit at or slightly above bench.py's HIP-event figures.", "",
        "| Kernel | Grid threads | Workloads | Calls | Average (us) | Min (us) | Max (us) |",
        "|---|---|---|---|---|---|---|",
    ]
    for (name, grid), r in rows:
        other = ["peak probe (bench.py measure_peaks)"] if name.startswith("fa_probe_") else ["(other)"]
        lines.append(f"| {name} | {grid} | {', '.join(users.get((name, grid), other))} | {r['calls']} | "
                     f"{r['avg_us']:.1f} | {r['min_us']:.1f} | {r['max_us']:.1f} |")
    return "\n".join(lines) + "\n"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--traffic", required=True)
    ap.add_argument("--pmc", required=True)
    ap.add_argument("--out-dir", required=True)
    ap.add_argument("--trace", help="kernel-trace run dir: also write kernel_stats_bench_default.md")
    a = ap.parse_args(argv)
    calls = workload_launches()
    traffic, pmc = _load(a.traffic), _load(a.pmc)
    written = []
    if traffic:
        p = os.path.join(a.out_dir, "pmc_traffic_bench_all_configs.md")
        with open(p, "w") as f:
            f.write(traffic_markdown(traffic, calls))
        written.append(p)
    if pmc:
        p = os.path.join(a.out_dir, "pmc_counters_bench_all_configs.md")
        with open(p, "w") as f:
            f.write(counters_markdown(pmc, calls))
        written.append(p)
    if a.trace:
        from .traffic import kernel_source_hash
        p = os.path.join(a.out_dir, "kernel_stats_bench_default.md")
        with open(p, "w") as f:
            f.write(trace_markdown(a.trace, calls, kernel_source_hash()))
        written.append(p)
    print("wrote " + ", ".join(written) if written else "nothing to write (no tables)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
