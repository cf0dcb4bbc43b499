"""HBM traffic per kernel launch from rocprofv3 counter runs.

``roofline.traffic`` in bench.py is the HBM bytes one launch of the headline
kernel moves, measured with two rocprofv3 ``--pmc`` passes (FETCH_SIZE, then
WRITE_SIZE; each counter in a run of its own) and calibrated by the same
counters on a plain device copy of known size:

    rocprofv3 --pmc FETCH_SIZE -d <dir_f> -o run -f csv -- python3 bench.py --no-cpu-baseline --steps 5 --warmup 1
    rocprofv3 --pmc WRITE_SIZE -d <dir_w> -o run -f csv -- python3 bench.py --no-cpu-baseline --steps 5 --warmup 1
    rocprofv3 --pmc FETCH_SIZE -d <dir_cf> -o run -f csv -- python3 bench.py --calibrate-copy-mib 1024
    rocprofv3 --pmc WRITE_SIZE -d <dir_cw> -o run -f csv -- python3 bench.py --calibrate-copy-mib 1024
    python -m flash_attention_amd.traffic --fetch <dir_f> --write <dir_w> \\
        --copy-fetch <dir_cf> --copy-write <dir_cw> --copy-mib 1024 --out profiles/traffic.json

``--trace <dir>`` prints per-launch-size kernel durations of a
``rocprofv3 --kernel-trace`` run as a markdown table.

``--pmc-a <dir> --pmc-b <dir> --out profiles/pmc.json`` builds the per-kernel
counter table (MFMA busy %, non-MFMA VALU per MFMA, wait share, LDS bank
conflicts) from two rocprofv3 ``--pmc`` runs over bench.py, one per counter
pass (PMC_PASS_A, PMC_PASS_B below):

    rocprofv3 --pmc <PMC_PASS_A> -d <dir_a> -o run -f csv -- python3 bench.py --no-cpu-baseline --steps 3 --warmup 1
    rocprofv3 --pmc <PMC_PASS_B> -d <dir_b> -o run -f csv -- python3 bench.py --no-cpu-baseline --steps 3 --warmup 1

Entries are keyed by kernel name and launch size (threads in the grid), so
the same kernel on two workloads keeps two figures, and each entry carries a
hash of the kernel sources it was measured on: bench.py reports a figure only
while the sources still hash the same, so an edited kernel never inherits an
old measurement.
"""
from __future__ import annotations

import argparse
import csv
import glob
import hashlib
import json
import os
import sys
from collections import defaultdict

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(_PKG_DIR, "csrc")
COPY_KERNEL = "__amd_rocclr_copyBuffer"


def kernel_source_files() -> list[str]:
    """The files the gfx950 code object is built from (kernels, includes, parameter block)."""
    files = [os.path.join(CSRC, "fa_kernels.hip"), os.path.join(CSRC, "fa_params.h")]
    files += sorted(glob.glob(os.path.join(CSRC, "*.inc")))
    return files


def kernel_source_hash() -> str:
    """sha256 (first 16 hex digits) over the kernel source files' names and bytes."""
    h = hashlib.sha256()
    for path in kernel_source_files():
        h.update(os.path.basename(path).encode())
        with open(path, "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def counter_means(run_dir: str, counter: str) -> dict[tuple[str, int], tuple[float, int]]:
    """{(kernel name, grid threads): (mean counter value in KiB, dispatches)} over a run's CSV files."""
    sums: dict[tuple[str, int], list[float]] = defaultdict(lambda: [0.0, 0])
    paths = glob.glob(os.path.join(run_dir, "**", "*counter_collection.csv"), recursive=True)
    if not paths:
        raise FileNotFoundError(f"no *counter_collection.csv under {run_dir}")
    csv.field_size_limit(1 << 24)
    for path in paths:
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                if row.get("Counter_Name") != counter:
                    continue
                key = (row["Kernel_Name"], int(row["Grid_Size"]))
                sums[key][0] += float(row["Counter_Value"])
                sums[key][1] += 1
    return {k: (s / n, n) for k, (s, n) in sums.items() if n}


def copy_scale(run_dir: str, counter: str, copy_mib: int) -> float:
    """Bytes per counter KiB, from the copy kernel that moves copy_mib MiB each way per dispatch."""
    means = counter_means(run_dir, counter)
    best = max((v for (name, _g), v in means.items() if COPY_KERNEL in name), key=lambda v: v[0], default=None)
    if best is None:
        raise ValueError(f"no {COPY_KERNEL} dispatch with {counter} under {run_dir}")
    return copy_mib * 1024.0 / best[0]


def build_table(fetch_dir, write_dir, copy_fetch_dir, copy_write_dir, copy_mib, prefix="fa_"):
    fs = copy_scale(copy_fetch_dir, "FETCH_SIZE", copy_mib)
    ws = copy_scale(copy_write_dir, "WRITE_SIZE", copy_mib)
    fetch = counter_means(fetch_dir, "FETCH_SIZE")
    write = counter_means(write_dir, "WRITE_SIZE")
    src = kernel_source_hash()
    table = {}
    for key in sorted(set(fetch) & set(write)):
        name, grid = key
        if not name.startswith(prefix):
            continue
        f_kib, nf = fetch[key]
        w_kib, nw = write[key]
        table[f"{name}@{grid}"] = {
            "kernel": name, "grid_threads": grid, "dispatches": [nf, nw],
            "fetch_kib_raw": round(f_kib, 1), "write_kib_raw": round(w_kib, 1),
            "fetch_scale": round(fs, 4), "write_scale": round(ws, 4),
            "fetch_bytes_per_launch": int(round(f_kib * fs * 1024)),
            "hbm_bytes_per_launch": int(round(f_kib * fs * 1024 + w_kib * ws * 1024)),
            "kernel_source_sha256": src,
        }
    return table


# PMC passes behind the per-kernel counter table (each pass in a run of its
# own: one rocprofv3 --pmc run may hold at most 8 SQ and 2 GRBM counters).
PMC_PASS_A = ("SQ_VALU_MFMA_BUSY_CYCLES", "SQ_BUSY_CYCLES", "SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_WAVE_CYCLES",
              "SQ_WAIT_INST_ANY", "GRBM_GUI_ACTIVE")
PMC_PASS_B = ("SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE", "SQ_INSTS_LDS", "SQ_WAIT_INST_LDS", "SQ_LDS_ADDR_CONFLICT",
              "GRBM_GUI_ACTIVE")
SIMDS = 1024   # MI355X: 256 CUs x 4 SIMDs
XCDS = 8


def all_counter_means(run_dir: str, prefix: str = "fa_") -> dict[tuple[str, int], dict[str, float]]:
    """{(kernel name, grid threads): {counter: mean per dispatch}} over a run's CSV files."""
    sums: dict[tuple[str, int, str], list[float]] = defaultdict(lambda: [0.0, 0])
    paths = glob.glob(os.path.join(run_dir, "**", "*counter_collection.csv"), recursive=True)
    if not paths:
        raise FileNotFoundError(f"no *counter_collection.csv under {run_dir}")
    csv.field_size_limit(1 << 24)
    for path in paths:
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                if not row["Kernel_Name"].startswith(prefix):
                    continue
                k = (row["Kernel_Name"], int(row["Grid_Size"]), row["Counter_Name"])
                sums[k][0] += float(row["Counter_Value"])
                sums[k][1] += 1
    out: dict[tuple[str, int], dict[str, float]] = {}
    for (name, grid, ctr), (s, n) in sums.items():
        out.setdefault((name, grid), {})[ctr] = s / n
        out[(name, grid)].setdefault("_dispatches", n)
    return out


def pmc_figures(a: dict[str, float], b: dict[str, float]) -> dict:
    """Derived figures of one kernel launch size from the two passes' means.

    mfma_busy_pct: SQ_VALU_MFMA_BUSY_CYCLES (summed over the SIMDs) over the
    SIMD-cycles the GPU was active (GRBM_GUI_ACTIVE summed over the XCDs / 8
    per XCD x 1024 SIMDs); valu_per_mfma: non-MFMA VALU instructions per MFMA;
    wait_pct: SQ_WAIT_INST_ANY share of the wave cycles; lds_bank_conflicts:
    SQ_LDS_BANK_CONFLICT cycles per launch, and their share of the LDS
    unit's active cycles."""
    active = a["GRBM_GUI_ACTIVE"] / XCDS
    mfma = a.get("SQ_INSTS_MFMA", 0.0)
    valu = a.get("SQ_INSTS_VALU", 0.0)
    fig = {
        "gui_active_cycles_per_xcd": int(round(active)),
        "mfma_busy_pct": round(100.0 * a["SQ_VALU_MFMA_BUSY_CYCLES"] / (active * SIMDS), 1) if active else None,
        "mfma_insts": int(round(mfma)),
        "valu_per_mfma": round((valu - mfma) / mfma, 2) if mfma else None,
        "valu_insts_non_mfma": int(round(valu - mfma)),
        "wait_pct": round(100.0 * a["SQ_WAIT_INST_ANY"] / a["SQ_WAVE_CYCLES"], 1) if a.get("SQ_WAVE_CYCLES") else None,
        "lds_bank_conflicts": int(round(b.get("SQ_LDS_BANK_CONFLICT", 0.0))),
        "lds_conflict_pct": (round(100.0 * b["SQ_LDS_BANK_CONFLICT"] / b["SQ_LDS_IDX_ACTIVE"], 2)
                             if b.get("SQ_LDS_IDX_ACTIVE") else 0.0),
        "lds_insts": int(round(b.get("SQ_INSTS_LDS", 0.0))),
        "dispatches": [int(a.get("_dispatches", 0)), int(b.get("_dispatches", 0))],
    }
    return fig


def build_pmc_table(dir_a: str, dir_b: str, prefix: str = "fa_") -> dict:
    pa, pb = all_counter_means(dir_a, prefix), all_counter_means(dir_b, prefix)
    src = kernel_source_hash()
    table = {}
    for key in sorted(set(pa) & set(pb)):
        name, grid = key
        if "GRBM_GUI_ACTIVE" not in pa[key] or "SQ_VALU_MFMA_BUSY_CYCLES" not in pa[key]:
            continue
        ent = {"kernel": name, "grid_threads": grid}
        ent.update(pmc_figures(pa[key], pb[key]))
        ent["kernel_source_sha256"] = src
        table[f"{name}@{grid}"] = ent
    return table


def trace_table(run_dir: str, prefix: str = "fa_") -> dict[tuple[str, int], dict]:
    """Per (kernel name, grid threads): calls and mean / min / max duration (us)
    from a ``rocprofv3 --kernel-trace`` run's *kernel_trace.csv.  The name-keyed
    ``--stats`` table mixes launch sizes; this keeps each workload apart."""
    acc: dict[tuple[str, int], list[float]] = {}
    paths = glob.glob(os.path.join(run_dir, "**", "*kernel_trace.csv"), recursive=True)
    if not paths:
        raise FileNotFoundError(f"no *kernel_trace.csv under {run_dir}")
    csv.field_size_limit(1 << 24)
    for path in paths:
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                name = row["Kernel_Name"]
                if not name.startswith(prefix):
                    continue
                grid = int(row["Grid_Size_X"]) * int(row["Grid_Size_Y"]) * int(row["Grid_Size_Z"])
                us = (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3
                a = acc.setdefault((name, grid), [0, 0.0, float("inf"), 0.0])
                a[0] += 1
                a[1] += us
                a[2] = min(a[2], us)
                a[3] = max(a[3], us)
    return {k: {"calls": a[0], "avg_us": a[1] / a[0], "min_us": a[2], "max_us": a[3]} for k, a in acc.items()}


def trace_markdown(run_dir: str) -> str:
    rows = sorted(trace_table(run_dir).items(), key=lambda kv: -kv[1]["avg_us"] * kv[1]["calls"])
    out = ["| Kernel | Grid threads | Calls | Average (us) | Min (us) | Max (us) |", "|---|---|---|---|---|---|"]
    for (name, grid), r in rows:
        out.append(f"| {name} | {grid} | {r['calls']} | {r['avg_us']:.1f} | {r['min_us']:.1f} | {r['max_us']:.1f} |")
    return "\n".join(out)


def lookup_entry(table_path: str, kernel: str, grid_threads: int):
    """The table's entry for (kernel, grid) when measured on these kernel sources, else None."""
    try:
        with open(table_path) as f:
            table = json.load(f)
    except (OSError, ValueError):
        return None
    ent = table.get(f"{kernel}@{grid_threads}")
    if not ent or ent.get("kernel_source_sha256") != kernel_source_hash():
        return None
    if "fetch_kib_raw" in ent and "fetch_bytes_per_launch" not in ent:
        ent["fetch_bytes_per_launch"] = int(round(ent["fetch_kib_raw"] * ent["fetch_scale"] * 1024))
    return ent


def lookup(table_path: str, kernel: str, grid_threads: int):
    """HBM bytes per launch for (kernel, grid), or (None, reason) when absent or measured on other sources."""
    try:
        with open(table_path) as f:
            table = json.load(f)
    except (OSError, ValueError):
        return None, "no traffic table"
    ent = table.get(f"{kernel}@{grid_threads}")
    if not ent:
        return None, "kernel not profiled"
    if ent.get("kernel_source_sha256") != kernel_source_hash():
        return None, "profiled on other kernel sources"
    return ent["hbm_bytes_per_launch"], "ok"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--trace", help="print the per-launch-size table of a --kernel-trace run and exit")
    ap.add_argument("--fetch")
    ap.add_argument("--write")
    ap.add_argument("--copy-fetch")
    ap.add_argument("--copy-write")
    ap.add_argument("--copy-mib", type=int, default=1024)
    ap.add_argument("--pmc-a", help="run dir of the first PMC pass (PMC_PASS_A counters)")
    ap.add_argument("--pmc-b", help="run dir of the second PMC pass (PMC_PASS_B counters)")
    ap.add_argument("--out")
    a = ap.parse_args(argv)
    if a.trace:
        print(trace_markdown(a.trace))
        return 0
    if a.pmc_a or a.pmc_b:
        if not (a.pmc_a and a.pmc_b and a.out):
            ap.error("--pmc-a, --pmc-b and --out go together")
        table = build_pmc_table(a.pmc_a, a.pmc_b)
        with open(a.out, "w") as f:
            json.dump(table, f, indent=1, sort_keys=True)
            f.write("\n")
        print(f"wrote {len(table)} kernel entries to {a.out}")
        return 0
    if not (a.fetch and a.write and a.copy_fetch and a.copy_write and a.out):
        ap.error("--fetch, --write, --copy-fetch, --copy-write and --out are required")
    table = build_table(a.fetch, a.write, a.copy_fetch, a.copy_write, a.copy_mib)
    with open(a.out, "w") as f:
        json.dump(table, f, indent=1, sort_keys=True)
        f.write("\n")
    print(f"wrote {len(table)} kernel entries to {a.out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
