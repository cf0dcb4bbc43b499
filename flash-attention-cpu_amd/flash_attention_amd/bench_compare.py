"""Compare two commits' rows of a benchmark history CSV.

Mirrors the reference's examples/bench_compare.rs: rows are joined on every
field except the timings (os, arch, threads, variant, causal, seq_len,
d_head -- plus ``device`` here) so measurements from different targets are
never compared by accident; with no arguments the last two distinct commits
(in order of first appearance, i.e. chronological for an appended file) are
compared, otherwise two commit prefixes.  A change of 3 % or more is marked
``faster`` / ``SLOWER``.

Accepts the reference's 10-column rows (device "cpu", no device_ms), the
12-column GPU rows and the 22-column rows with GPU columns that
bench_quick --csv and bench.py --csv write (the workload name, key length
and slice count join the key, so bench.py's BASELINE configurations are
compared config by config; their TFLOP/s or GB/s are shown next to the
timings); repeated header lines are skipped (concatenated CSVs), malformed
rows are reported and skipped.  For GPU rows both timings are compared:
time_ms (host-slice call for bench_quick rows, wall time of a
device-resident call for bench.py rows) and device_ms (kernels only).

Run: ``python -m flash_attention_amd.bench_compare [--file history.csv] [old new]``.
"""
from __future__ import annotations

import argparse
import os
import sys
from dataclasses import dataclass

DEFAULT_HISTORY = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "benches",
                               "history.csv")


@dataclass(frozen=True, order=True)
class Key:
    os: str
    arch: str
    device: str
    threads: int
    variant: str
    causal: bool
    seq_len: int
    d_head: int
    workload: str = ""
    seq_len_k: int = 0    # 0: seq_len (a square shape)
    heads: int = 1

    def __post_init__(self):
        if self.seq_len_k == 0:
            object.__setattr__(self, "seq_len_k", self.seq_len)


@dataclass
class Row:
    commit: str
    key: Key
    time_ms: float
    device_ms: float | None
    rate: str = ""        # "127.1TF" / "6620GB/s" from the GPU columns, when present


def _bool(s: str) -> bool:
    if s == "true":
        return True
    if s == "false":
        return False
    raise ValueError(s)


def parse_csv(text: str, warn=lambda msg: print(msg, file=sys.stderr)) -> list[Row]:
    rows = []
    for line in text.splitlines():
        if not line or line.startswith("timestamp,"):
            continue
        f = line.split(",")
        if len(f) not in (10, 12, 22):
            warn(f"skipping malformed row: {line}")
            continue
        try:
            device = f[10] if len(f) >= 12 else "cpu"
            device_ms = float(f[11]) if len(f) >= 12 else None
            seq_len = int(f[7])
            workload, seq_len_k, heads, rate = "", seq_len, 1, ""
            if len(f) == 22:
                workload, seq_len_k, heads = f[12], int(f[13]), int(f[14])
                if f[15] and not f[17]:
                    rate = f"{float(f[15]):.1f}TF"
                elif f[17]:
                    rate = f"{float(f[17]):.0f}GB/s"
            key = Key(f[2], f[3], device, int(f[4]), f[5], _bool(f[6]), seq_len, int(f[8]), workload,
                      seq_len_k, heads)
            rows.append(Row(f[1], key, float(f[9]), device_ms, rate))
        except ValueError:
            warn(f"skipping malformed row: {line}")
    return rows


def commits_in_order(rows: list[Row]) -> list[str]:
    seen: list[str] = []
    for r in rows:
        if r.commit not in seen:
            seen.append(r.commit)
    return seen


def resolve(commits: list[str], arg: str) -> str:
    for c in commits:
        if c == arg or c.startswith(arg):
            return c
    raise SystemExit(f"no data for commit matching {arg!r}; known commits: {commits}")


def _change(old: float, new: float) -> tuple[float, str]:
    pct = (new - old) / old * 100.0 if old else 0.0
    return pct, "faster" if pct <= -3.0 else ("SLOWER" if pct >= 3.0 else "~")


def compare(rows: list[Row], old: str, new: str) -> tuple[list[str], int, int]:
    """Report lines, and the counts of keys only in `old` / only in `new`."""
    old_map = {r.key: r for r in rows if r.commit == old}
    new_map = {r.key: r for r in rows if r.commit == new}
    lines = [f"comparing {old} -> {new}", "",
             f"{'target':<16} {'thr':>5} {'var':>5} {'causal':>6} {'seq':>5} {'d':>5} | {'old_ms':>10} "
             f"{'new_ms':>10} {'change':>8}        | {'old_dev':>10} {'new_dev':>10} {'change':>8}"]
    only_old = only_new = 0
    for key in sorted(set(old_map) | set(new_map)):
        target = f"{key.os}/{key.arch}" + ("" if key.device == "cpu" else f"/{key.device}")
        if key.workload:
            target += f" {key.workload}"
        head = (f"{target:<16} {key.threads:>5} {key.variant:>5} {str(key.causal).lower():>6} {key.seq_len:>5} "
                f"{key.d_head:>5} |")
        o, n = old_map.get(key), new_map.get(key)
        if o and n:
            pct, mark = _change(o.time_ms, n.time_ms)
            line = f"{head} {o.time_ms:>10.4f} {n.time_ms:>10.4f} {pct:>+7.1f}% {mark:<6} |"
            if o.device_ms is not None and n.device_ms is not None:
                dp, dm = _change(o.device_ms, n.device_ms)
                line += f" {o.device_ms:>10.4f} {n.device_ms:>10.4f} {dp:>+7.1f}% {dm:<6}"
            if o.rate or n.rate:
                line += f" | {o.rate or '-'} -> {n.rate or '-'}"
            lines.append(line.rstrip())
        elif n:
            only_new += 1
            dev = f" {'-':>10} {n.device_ms:>10.4f}" if n.device_ms is not None else ""
            lines.append(f"{head} {'-':>10} {n.time_ms:>10.4f} {'new':>9}        |{dev}")
        else:
            only_old += 1
    if only_old:
        lines.append(f"\n{only_old} measurement(s) present only in {old}, not in {new} "
                     "(target/shape not re-measured)")
    if only_new:
        lines.append(f"{only_new} measurement(s) present only in {new}, not in {old} "
                     "(new target/shape, printed above as \"new\")")
    return lines, only_old, only_new


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--file", default=DEFAULT_HISTORY)
    ap.add_argument("commits", nargs="*", help="old and new commit (prefix match); default: the last two")
    args = ap.parse_args(argv)
    try:
        with open(args.file, encoding="utf-8") as fh:
            rows = parse_csv(fh.read())
    except OSError as e:
        raise SystemExit(f"couldn't read {args.file}: {e}")
    if not rows:
        print(f"no usable rows in {args.file}", file=sys.stderr)
        return 1
    commits = commits_in_order(rows)
    if len(args.commits) == 2:
        old, new = resolve(commits, args.commits[0]), resolve(commits, args.commits[1])
    elif len(args.commits) == 0 and len(commits) >= 2:
        old, new = commits[-2], commits[-1]
    elif len(args.commits) == 0:
        print(f"only one commit ({commits[0]}) in {args.file} so far -- nothing to compare yet. Run "
              "bench_quick --csv again after a change and append it to add a second one.")
        return 0
    else:
        ap.error("give two commits or none")
    lines, _, _ = compare(rows, old, new)
    print("\n".join(lines))
    return 0


if __name__ == "__main__":
    sys.exit(main())
