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
(examples/bench_quick.rs:170-176) followed by two GPU columns::

    timestamp,commit,os,arch,threads,variant,causal,seq_len,d_head,time_ms,device,device_ms

``threads`` is the GPU's compute-unit count (the reference records rayon's
thread count), ``device`` its gfx architecture.  The commit comes from
BENCH_COMMIT, else ``git rev-parse --short HEAD``, else "unknown"
(examples/bench_quick.rs:22-41).

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


def csv_row(timestamp: int, commit: str, os_name: str, arch: str, threads: int, variant: str, causal: bool,
            seq_len: int, d_head: int, time_ms: float, device: str, device_ms: float) -> str:
    return (f"{timestamp},{commit},{os_name},{arch},{threads},{variant},{str(causal).lower()},{seq_len},{d_head},"
            f"{time_ms:.4f},{device},{device_ms:.4f}")


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
        print(HEADER)
        for label, causal, seq_len, d_head, t_host, t_dev in rows:
            print(csv_row(ts, commit, os_name, arch, cus, label, causal, seq_len, d_head, t_host, device, t_dev))
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
