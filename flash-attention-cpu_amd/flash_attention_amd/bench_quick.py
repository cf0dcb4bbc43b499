"""Quick benchmark table / history rows for the GPU library.

Mirrors the reference's examples/bench_quick.rs: the same shapes
((256, 64), (512, 64), (1024, 64), (2048, 64), (1024, 128)), the same inputs
(U(-1, 1), seeds 1/2/3), naive plus v1/v2/v3 non-causal and causal, one
warm-up call and the mean of N calls.  Two timings per row:

* ``time_ms``   -- the drop-in host-slice call (fa_v1/v2/v3, fa_naive_attention),
  i.e. what a caller of the crate's API sees, PCIe copies included;
* ``device_ms`` -- the same computation on device-resident buffers
  (fa_device_ex / fa_naive_device), kernels only, timed with HIP events.

``--csv`` prints rows in the history schema of benches/history.csv
(examples/bench_quick.rs:170-176) followed by GPU columns::

    timestamp,commit,os,arch,threads,variant,causal,seq_len,d_head,time_ms,device,device_ms,
    workload,seq_len_k,heads,tflops,pct_peak,gbps,pct_hbm,mfma_busy,lds_bank_conflicts,fetch_gbps

``threads`` is the GPU's compute-unit count (the reference records rayon's
thread count), ``device`` its gfx architecture.  The commit comes from
BENCH_COMMIT, else ``git rev-parse --short HEAD``, else "unknown"
(examples/bench_quick.rs:22-41).  The last ten columns: the workload name
(empty for these shapes; bench.py --csv writes its BASELINE configurations
as config1 .. config5c), the key length and slice count when they differ
from seq_len and 1, algorithmic TFLOP/s and % of the FP32-MFMA peak (% of
the 16-bit peak for bf16 / f16 rows), algorithmic GB/s and % of 8 TB/s,
and -- where profiles/ holds counters for the kernel at that launch size,
measured on the current kernel sources -- MFMA busy %, LDS bank-conflict
cycles per launch and the FETCH_SIZE rate in GB/s (empty otherwise).  Rows
of the earlier 12-column form stay readable (bench_compare).

Run: ``python -m flash_attention_amd.bench_quick [--csv] [--iters N]`` with
flash-attention-cpu_amd/ on sys.path.
"""
from __future__ import annotations

import argparse
import os
import platform
import subprocess
import sys
import time

import numpy as np

SHAPES = ((256, 64), (512, 64), (1024, 64), (2048, 64), (1024, 128))
HEADER = "timestamp,commit,os,arch,threads,variant,causal,seq_len,d_head,time_ms,device,device_ms"
GPU_COLUMNS = ("workload", "seq_len_k", "heads", "tflops", "pct_peak", "gbps", "pct_hbm", "mfma_busy",
               "lds_bank_conflicts", "fetch_gbps")
HEADER_EXT = HEADER + "," + ",".join(GPU_COLUMNS)
PEAK_TFLOPS = 157.3   # MI355X dense FP32 MFMA
PEAK_GBS = 8000.0     # MI355X HBM3E
# (variant label, flash variant or 0 for naive, causal) in the reference's column order
RUNS = (("naive", 0, False), ("v1", 1, False), ("v2", 2, False), ("v3", 3, False),
        ("v1", 1, True), ("v2", 2, True), ("v3", 3, True))


def random_vec(n: int, seed: int) -> np.ndarray:
    """U(-1, 1) f32 (examples/bench_quick.rs:8-11 draws from rand's StdRng)."""
    return np.random.default_rng(seed).uniform(-1.0, 1.0, n).astype(np.float32)


def resolve_commit() -> str:
    c = os.environ.get("BENCH_COMMIT")
    if c:
        return c
    try:
        r = subprocess.run(["git", "rev-parse", "--short", "HEAD"], capture_output=True, text=True, timeout=10)
        if r.returncode == 0 and r.stdout.strip():
            return r.stdout.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return "unknown"


def _opt(x, fmt: str) -> str:
    return "" if x is None else format(x, fmt)


def csv_row(timestamp: int, commit: str, os_name: str, arch: str, threads: int, variant: str, causal: bool,
            seq_len: int, d_head: int, time_ms: float, device: str, device_ms: float, **gpu) -> str:
    """One history row: the 12-column form, or with any of GPU_COLUMNS given
    as keywords the 22-column form (missing figures left empty)."""
    row = (f"{timestamp},{commit},{os_name},{arch},{threads},{variant},{str(causal).lower()},{seq_len},{d_head},"
           f"{time_ms:.4f},{device},{device_ms:.4f}")
    if not gpu:
        return row
    unknown = set(gpu) - set(GPU_COLUMNS)
    if unknown:
        raise TypeError(f"unknown history columns {sorted(unknown)}")
    ext = [gpu.get("workload") or "", str(gpu.get("seq_len_k") or seq_len), str(gpu.get("heads") or 1),
           _opt(gpu.get("tflops"), ".3f"), _opt(gpu.get("pct_peak"), ".1f"), _opt(gpu.get("gbps"), ".1f"),
           _opt(gpu.get("pct_hbm"), ".1f"), _opt(gpu.get("mfma_busy"), ".1f"),
           _opt(gpu.get("lds_bank_conflicts"), "d"), _opt(gpu.get("fetch_gbps"), ".1f")]
    return row + "," + ",".join(ext)


def gpu_columns(variant: int, seq_len: int, d_head: int, causal: bool, device_ms: float) -> dict:
    """tflops / pct_peak / gbps / pct_hbm of one device-resident call, and
    the counters of its first kernel where profiles/ holds them for the
    current kernel sources (variant 0: the naive kernels)."""
    from . import describe_launch
    from . import traffic as trf

    pairs = seq_len * (seq_len + 1) // 2 if causal else seq_len * seq_len
    flop = 4 * d_head * pairs
    nbytes = 4 * d_head * 4 * seq_len
    sec = device_ms * 1e-3
    cols = {"tflops": flop / sec / 1e12, "pct_peak": 100 * flop / sec / 1e12 / PEAK_TFLOPS,
            "gbps": nbytes / sec / 1e9, "pct_hbm": 100 * nbytes / sec / 1e9 / PEAK_GBS}
    if variant:
        plan = describe_launch(variant, 1, 1, seq_len, seq_len, d_head, causal)
        first = plan.split(";")[0].split()
        dims = [int(x) for x in first[1].split("=")[1].split("x")]
        grid = dims[0] * dims[1] * dims[2] * int(first[2].split("=")[1])
        profiles = os.path.join(os.path.dirname(trf._PKG_DIR), "profiles")   # the repository's
        pent = trf.lookup_entry(os.path.join(profiles, "pmc.json"), first[0], grid)
        if pent is not None:
            cols.update(mfma_busy=pent["mfma_busy_pct"], lds_bank_conflicts=pent["lds_bank_conflicts"])
        tent = trf.lookup_entry(os.path.join(profiles, "traffic.json"), first[0], grid)
        if tent is not None:
            cols["fetch_gbps"] = tent["fetch_bytes_per_launch"] / sec / 1e9
    return cols


def time_host(f, iters: int) -> float:
    """One warm-up call, then the mean wall time of `iters` calls, in ms."""
    f()
    t0 = time.perf_counter()
    for _ in range(iters):
        f()
    return (time.perf_counter() - t0) / iters * 1000.0


def measure(iters: int, dev_iters: int):
    """[(variant, causal, seq_len, d_head, time_ms, device_ms)] over SHAPES x RUNS."""
    import torch

    from . import (FlashAttentionConfig, NAIVE_F32, VARIANTS, attention_device, init, naive_attention,
                   naive_device)

    init()
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream()
    rows = []
    for seq_len, d_head in SHAPES:
        n = seq_len * d_head
        q, k, v = random_vec(n, 1), random_vec(n, 2), random_vec(n, 3)
        out = np.zeros(n, dtype=np.float32)
        tq, tk, tv = (torch.from_numpy(a).to(dev) for a in (q, k, v))
        to = torch.empty(n, device=dev)
        for label, variant, causal in RUNS:
            if variant == 0:
                host = lambda: naive_attention(q, k, v, seq_len, seq_len, d_head, causal, out)   # noqa: E731
                dcall = lambda: naive_device(tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), 1, 1,   # noqa: E731
                                             seq_len, seq_len, d_head, causal, to.data_ptr(),
                                             stream.cuda_stream, NAIVE_F32)
            else:
                cfg = FlashAttentionConfig(causal=causal)
                host = lambda: VARIANTS[variant](q, k, v, seq_len, seq_len, d_head, cfg, out)   # noqa: E731
                dcall = lambda: attention_device(variant, tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), 1, 1,  # noqa
                                                 seq_len, seq_len, d_head, causal, to.data_ptr(), stream.cuda_stream)
            t_host = time_host(host, iters)
            dcall()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(dev_iters):
                dcall()
            e1.record(stream)
            torch.cuda.synchronize()
            rows.append((label, causal, seq_len, d_head, t_host, e0.elapsed_time(e1) / dev_iters))
    return rows


def device_info():
    import torch
    props = torch.cuda.get_device_properties(0)
    arch = getattr(props, "gcnArchName", "") or props.name
    return arch.split(":")[0], int(props.multi_processor_count)


def print_table(rows, key: int, title: str) -> None:
    print(title)
    print(f"{'seq':>7} {'d':>5} | {'naive_ms':>9} | {'v1_ms':>8} {'v2_ms':>8} {'v3_ms':>8} | "
          f"{'v1c_ms':>8} {'v2c_ms':>8} {'v3c_ms':>8}")
    for seq_len, d_head in SHAPES:
        t = {(r[0], r[1]): r[key] for r in rows if r[2] == seq_len and r[3] == d_head}
        print(f"{seq_len:>7} {d_head:>5} | {t[('naive', False)]:>9.3f} | {t[('v1', False)]:>8.3f} "
              f"{t[('v2', False)]:>8.3f} {t[('v3', False)]:>8.3f} | {t[('v1', True)]:>8.3f} "
              f"{t[('v2', True)]:>8.3f} {t[('v3', True)]:>8.3f}")


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--csv", action="store_true", help="print history rows instead of tables")
    ap.add_argument("--iters", type=int, default=20, help="timed host-slice calls per row (after one warm-up)")
    ap.add_argument("--dev-iters", type=int, default=50, help="timed device-resident calls per row")
    args = ap.parse_args(argv)
    rows = measure(args.iters, args.dev_iters)
    device, cus = device_info()
    if args.csv:
        ts, commit = int(time.time()), resolve_commit()
        os_name, arch = platform.system().lower(), platform.machine()
        print(HEADER_EXT)
        for label, causal, seq_len, d_head, t_host, t_dev in rows:
            variant = 0 if label == "naive" else int(label[1])
            cols = gpu_columns(variant, seq_len, d_head, causal, t_dev)
            print(csv_row(ts, commit, os_name, arch, cus, label, causal, seq_len, d_head, t_host, device, t_dev,
                          workload="", **cols))
        return 0
    print_table(rows, 4, f"host-slice calls (time_ms; {device}, {cus} CUs, PCIe copies included)")
    print()
    print_table(rows, 5, "device-resident calls (device_ms; kernels only)")
    seq = 4096
    print(f"\nAt seq_len={seq}: naive score-matrix allocation = {seq * seq * 4 / 2**20:.1f} MB; the flash kernels "
          f"keep scores in registers and K/V stages in LDS (at most 160 KB per CU), independent of seq_len")
    return 0


if __name__ == "__main__":
    sys.exit(main())
