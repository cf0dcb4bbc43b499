#!/usr/bin/env python3
"""Benchmark: FlashAttention forward on one MI355X, every configuration.

Headline (the metric's configuration): 32 heads x 2048 x 2048, d_head 128,
causal, f32, v3, inputs resident in HBM.  A "step" is one attention call over
that batch.  ``value`` is whole-job TFLOP/s (algorithmic FLOP
4*d*visible_pairs*heads over wall time between synchronisations); the
``roofline`` object prices the prefill kernel's own duration (HIP events on
the launch stream) against the FP32-MFMA peak, and ``roofline.traffic`` is
the kernel's measured HBM bytes per launch (rocprofv3 counters, reported only
while the kernel sources match the ones profiled).

Every other configuration (1, 3, 4a, 4b, 5, 5c; v1/v2/v3), and four shapes
beyond BASELINE.json (wide heads of d_head 512, 1024 and 2048, and a batched
decode step of 768 slices), is timed the same way into
``extra.configs`` -- TFLOP/s and % of the FP32-MFMA peak for
prefill shapes, GB/s and % of 8 TB/s for decode shapes -- next to a CPU
baseline on the same inputs: the oracle's v2 (oracle/, a C restatement of the
reference crate's rayon + AVX-512/AVX2 path, src/v2.rs:160-385) on all host
cores, time-boxed, ms/call and GFLOP/s (GB/s for decode) as
examples/bench_quick.rs:13-21 reports them.  The CPU v2 output is also the
parity reference: every GPU output timed here is compared with it (max-abs,
relative L2; north_star bar 2e-5 / 1e-5), and the headline's figures are the
top-level ``parity`` object.

Before the configurations, peak probes (fa_probe_launch: back-to-back f32 and
bf16 MFMA streams on every CU, a 1 GiB device copy) measure the ceilings the
data-sheet peaks stand for on this GPU (``extra.measured_peaks``; the roofline
itself keeps the data-sheet denominators).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--variant 3]
                       [--quick | --configs config2,config4a,...]
                       [--no-cpu-baseline] [--no-peaks] [--cpu-seconds S] [--csv PATH]
Prints exactly one JSON line on stdout (compact: per config and variant the
kernel time, throughput, % of peak, counters where profiled, and parity);
progress goes to stderr, which ends with a one-line-per-config summary.
--csv appends one benchmark-history row per config and variant to PATH
(flash_attention_amd.bench_quick's schema, compared by bench_compare).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "flash-attention-cpu_amd"))

METRIC = "attention TFLOP/s f32 (32h×2048×d128 causal) + % FP32-MFMA peak; decode GB/s"
PEAK_TFLOPS = 157.3     # MI355X dense FP32 MFMA
PEAK_GBS = 8000.0       # MI355X HBM3E
PEAK_TFLOPS_16 = 2500.0  # MI355X dense bf16 / f16 MFMA
MAX_ABS_TOL, REL_L2_TOL = 2e-5, 1e-5   # north_star parity bar against CPU v2

# name, heads, seq_q, seq_k, d_head, causal, Q/K std, V ~ U(-1, 1), kind
CONFIGS = [
    ("config1", 1, 256, 256, 64, False, 1.0, False, "prefill"),
    ("config2", 32, 2048, 2048, 128, True, 1.0, False, "prefill"),
    ("config3", 8, 16384, 16384, 128, True, 1.0, False, "prefill"),
    ("config4a", 32, 1, 32768, 128, False, 1.0, False, "decode"),
    ("config4b", 32, 16, 32768, 128, False, 1.0, False, "decode"),
    ("config5", 16, 4096, 1024, 256, False, 3.0, True, "prefill"),
    ("config5c", 16, 1000, 1000, 256, True, 3.0, True, "prefill"),
    # not BASELINE.json configs: heads wider than 256 on the column-group
    # flash kernels (the crate's flash path takes any d_head)
    ("wide_d512", 16, 2048, 2048, 512, True, 1.0, False, "prefill"),
    ("wide_d1024", 8, 2048, 2048, 1024, True, 1.0, False, "prefill"),
    ("wide_d2048", 4, 2048, 2048, 2048, True, 1.0, False, "prefill"),
    # wider than 2048: the any-width kernels (O accumulated in the output)
    ("wide_d4096", 2, 2048, 2048, 4096, True, 1.0, False, "prefill"),
    # batched decode step: 768 (sequence, head) slices of one query over
    # 2048 keys, the split-KV row kernel whatever the grid size (launch
    # sizes of its own for every variant: profiles key kernels by name and
    # launch size)
    ("decode_batched", 768, 1, 2048, 128, False, 1.0, False, "decode"),
]
HEADLINE = "config2"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def visible_pairs(sq: int, sk: int, causal: bool) -> int:
    if not causal:
        return sq * sk
    # key j visible to query i iff j <= i (top-left aligned)
    n = min(sq, sk)
    return n * (n + 1) // 2 + max(0, sq - sk) * sk


def flops_of(bh, sq, sk, d, causal) -> int:
    return 4 * d * visible_pairs(sq, sk, causal) * bh


def bytes_of(bh, sq, sk, d) -> int:
    return 4 * bh * d * (2 * sq + 2 * sk)


class Workload:
    def __init__(self, torch, name, bh, sq, sk, d, causal, qk_sigma=1.0, v_uniform=False, kind="prefill"):
        self.name, self.bh, self.sq, self.sk, self.d, self.causal = name, bh, sq, sk, d, causal
        self.kind = kind
        dev = torch.device("cuda", 0)
        gens = []
        for seed in (1, 2, 3):   # seeds Q=1, K=2, V=3
            g = torch.Generator(device=dev)
            g.manual_seed(seed)
            gens.append(g)
        self.q = torch.randn(bh * sq * d, device=dev, generator=gens[0]) * qk_sigma
        self.k = torch.randn(bh * sk * d, device=dev, generator=gens[1]) * qk_sigma
        if v_uniform:
            self.v = torch.rand(bh * sk * d, device=dev, generator=gens[2]) * 2.0 - 1.0
        else:
            self.v = torch.randn(bh * sk * d, device=dev, generator=gens[2])
        self.o = torch.empty(bh * sq * d, device=dev)
        self.flops = flops_of(bh, sq, sk, d, causal)
        self.bytes = bytes_of(bh, sq, sk, d)

    def describe(self):
        dist = "N(0,1)" if self.kind == "decode" or self.d != 256 else "Q,K ~ N(0,3^2), V ~ U(-1,1)"
        return (f"{self.name}: {self.bh}h x {self.sq} x {self.sk}, d{self.d}, "
                f"{'causal' if self.causal else 'non-causal'}, {dist}")


RAMP_SECONDS = 0.3   # untimed sustained work before each measurement (clock ramp)

# Peak probes (fa_probe_launch): kind, label, iterations per launch (about 4 ms
# of MFMA work each at the data-sheet rate), data-sheet peak, unit.
PROBES = (
    ("fp32_mfma_32x32x2", 0, 5000, PEAK_TFLOPS, "TFLOP/s"),
    ("fp32_mfma_16x16x4", 1, 5000, PEAK_TFLOPS, "TFLOP/s"),
    ("bf16_mfma_16x16x32", 2, 5000, PEAK_TFLOPS_16, "TFLOP/s"),
    ("bf16_mfma_32x32x16", 4, 5000, PEAK_TFLOPS_16, "TFLOP/s"),
    ("hbm_copy", 3, 0, PEAK_GBS, "GB/s"),
    ("hbm_read", 5, 0, PEAK_GBS, "GB/s"),
)
PROBE_COPY_BYTES = 2 << 30   # 1 GiB copied onto another 1 GiB


def measure_peaks(torch, fa) -> dict:
    """The machine's own ceilings next to the data-sheet peaks the roofline
    divides by: back-to-back MFMA streams on every CU (FLOP per launch from
    fa_probe_launch), a 1 GiB device copy (bytes read + written) and a 1 GiB
    read-only stream, each the best of 5 launches after a clock ramp, timed with HIP
    events on the launch stream."""
    stream = torch.cuda.current_stream()
    buf = torch.empty(PROBE_COPY_BYTES // 4, dtype=torch.float32, device="cuda")
    out = {}
    for label, kind, iters, peak, unit in PROBES:
        def call():
            return fa.probe_launch(kind, stream.cuda_stream, buf.data_ptr(), PROBE_COPY_BYTES, iters)
        t_ramp = time.perf_counter()
        while time.perf_counter() - t_ramp < RAMP_SECONDS:
            call()
            torch.cuda.synchronize()
        best = None
        for _ in range(5):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            work = call()
            e1.record(stream)
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1)
            best = ms if best is None else min(best, ms)
        rate = work / (best * 1e-3) / (1e12 if unit == "TFLOP/s" else 1e9)
        out[label] = {"value": round(rate, 1), "unit": unit, "datasheet": peak,
                      "frac_of_datasheet": round(rate / peak, 4), "ms": round(best, 3)}
        log(f"[bench] peak probe {label}: {rate:.1f} {unit} ({rate / peak * 100:.1f} % of the data sheet's {peak:g})")
    del buf
    torch.cuda.empty_cache()
    return out


def time_calls(torch, call, steps: int, warmup: int):
    """Clock ramp, W warm-up calls, then K timed calls between synchronisations.

    An MI355X coming out of idle runs its first ~10-20 ms of work at a lower
    clock (measured: the first calls of a run are 10-15 % slower than the
    steady state), so every measurement first repeats the same call, untimed,
    for RAMP_SECONDS.  Returns (wall ms per step, kernel-stream ms per step
    from HIP events on the launch stream)."""
    stream = torch.cuda.current_stream()
    t_ramp = time.perf_counter()
    while True:
        for _ in range(8):
            call()
        torch.cuda.synchronize()
        if time.perf_counter() - t_ramp >= RAMP_SECONDS:
            break
    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        call()
    e1.record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    return (t1 - t0) * 1e3 / steps, e0.elapsed_time(e1) / steps


def f32_call(torch, fa, wl: Workload, variant: int):
    handle = torch.cuda.current_stream().cuda_stream

    def call():
        fa.attention_device(variant, wl.q.data_ptr(), wl.k.data_ptr(), wl.v.data_ptr(), 1, wl.bh, wl.sq,
                            wl.sk, wl.d, wl.causal, wl.o.data_ptr(), handle)
    return call


def auto_steps(torch, call, cap: int, target_ms: float = 40.0) -> int:
    """Timed calls for about target_ms of GPU time (at least 3, at most cap)."""
    call()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    call()
    torch.cuda.synchronize()
    one = (time.perf_counter() - t0) * 1e3
    return int(max(3, min(cap, target_ms / max(one, 1e-3))))


def time_host_slice(fa, wl: Workload, variant: int, calls: int) -> float:
    """The drop-in host-slice call (fa_multihead_vN: copy in, run, copy out),
    ms per call after one warm-up.  PCIe-inclusive; never the headline."""
    import numpy as np

    q, k, v = wl.q.cpu().numpy(), wl.k.cpu().numpy(), wl.v.cpu().numpy()
    out = np.empty(wl.bh * wl.sq * wl.d, dtype=np.float32)
    cfg = fa.FlashAttentionConfig(causal=wl.causal)
    f = fa.MULTIHEAD_VARIANTS[variant]
    f(q, k, v, 1, wl.bh, wl.sq, wl.sk, wl.d, cfg, out)
    t0 = time.perf_counter()
    for _ in range(calls):
        f(q, k, v, 1, wl.bh, wl.sq, wl.sk, wl.d, cfg, out)
    return (time.perf_counter() - t0) * 1e3 / calls


def grid_threads(describe: str) -> int:
    """Threads in the first launch of a fa_describe_launch string ("name grid=AxBxC block=T ...")."""
    first = describe.split(";")[0].split()
    g = [int(x) for x in first[1].split("=")[1].split("x")]
    return g[0] * g[1] * g[2] * int(first[2].split("=")[1])


def host_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def cpu_v2(inputs, wl: Workload, budget_s: float, threads: int):
    """Oracle v2 (C restatement of the crate's CPU v2) on the same inputs:
    one warm-up call, then calls until budget_s (at least one).  Returns
    (output of the last call, seconds per call, calls)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle   # test infrastructure: the timed CPU baseline and the checker only

    q, k, v = inputs
    out = oracle.run(2, q, k, v, wl.bh, wl.sq, wl.sk, wl.d, wl.causal, 64, 128, nthreads=threads)   # warm-up
    n, t0 = 0, time.perf_counter()
    while True:
        oracle.run(2, q, k, v, wl.bh, wl.sq, wl.sk, wl.d, wl.causal, 64, 128, nthreads=threads, out=out)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 200:
            break
    return out, el / n, n


def parity(got, want) -> dict:
    import numpy as np

    g = np.asarray(got, np.float64)
    w = np.asarray(want, np.float64)
    ma = float(np.max(np.abs(g - w))) if g.size else 0.0
    den = float(np.linalg.norm(w))
    rl = float(np.linalg.norm(g - w)) / (den if den > 0 else 1.0)
    return {"max_abs": float(f"{ma:.3g}"), "rel_l2": float(f"{rl:.3g}"),
            "within_bar": bool(np.all(np.isfinite(g)) and ma < MAX_ABS_TOL and rl < REL_L2_TOL)}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--variant", type=int, default=3, choices=(1, 2, 3))
    ap.add_argument("--quick", "--only-config2", action="store_true", dest="quick",
                    help="time only the headline workload's f32 variants (profiling runs)")
    ap.add_argument("--configs", default="",
                    help="comma-separated subset of " + ",".join(c[0] for c in CONFIGS) + " (the headline always runs)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-peaks", action="store_true", help="skip the MFMA / copy peak probes")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU budget of the headline baseline")
    ap.add_argument("--cpu-seconds-other", type=float, default=2.5, help="CPU budget of each other config")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="only run 5 plain device copies of N MiB (rocprofv3 PMC scale reference) and exit")
    ap.add_argument("--csv", default="", metavar="PATH",
                    help="append one history row per config and variant to PATH (bench_quick's schema)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build measures one MI355X; "
              "heads would shard across GPUs with no communication, each GPU running this kernel on "
              "its share; run with --gpus 1",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    if args.calibrate_copy_mib:
        n = args.calibrate_copy_mib * (1 << 20) // 4
        x = torch.ones(n, device="cuda")
        y = torch.empty_like(x)
        for _ in range(5):
            y.copy_(x)
        torch.cuda.synchronize()
        log(f"[bench] copied {args.calibrate_copy_mib} MiB x5")
        return 0

    import flash_attention_amd as fa
    from flash_attention_amd import traffic as trf

    fa.init()
    peaks, peaks_error = {}, None
    if not args.no_peaks:
        try:   # a measurement aid: a failure here must not cost the benchmark line
            peaks = measure_peaks(torch, fa)
        except (RuntimeError, fa.FaError) as e:
            peaks_error = f"{type(e).__name__}: {e}"
            log(f"[bench] peak probes skipped: {peaks_error}")
            torch.cuda.empty_cache()
    traffic_table = os.path.join(ROOT, "profiles", "traffic.json")
    pmc_table = os.path.join(ROOT, "profiles", "pmc.json")
    configs = {}
    pending_cpu = []   # (name, workload, host inputs, {variant: GPU output})
    result_head = None
    history = []       # (name, label, wl, wall ms, kernel ms, entry) for --csv

    chosen = {c for c in args.configs.split(",") if c}
    unknown = chosen - {c[0] for c in CONFIGS}
    if unknown:
        print(f"bench.py: unknown config(s) {sorted(unknown)}", file=sys.stderr)
        return 2

    def counters(ent, kernels, ms_kernel):
        """Measured HBM bytes and PMC figures of the call's first kernel, where profiled on these sources."""
        key = (kernels.split()[0], grid_threads(kernels))
        tb, _ = trf.lookup(traffic_table, *key)
        if tb is not None:
            ent["hbm_mb"] = round(tb / 1e6, 1)
        tent = trf.lookup_entry(traffic_table, *key)
        if tent is not None and ms_kernel > 0:
            ent["fetch_gbs"] = round(tent["fetch_bytes_per_launch"] / (ms_kernel * 1e-3) / 1e9, 1)
        pent = trf.lookup_entry(pmc_table, *key)
        if pent is not None:
            ent["mfma_busy"] = pent["mfma_busy_pct"]
            ent["lds_conflicts"] = pent["lds_bank_conflicts"]

    for (name, bh, sq, sk, d, causal, sig, vu, kind) in CONFIGS:
        if name != HEADLINE and (args.quick or (chosen and name not in chosen)):
            continue
        wl = Workload(torch, name, bh, sq, sk, d, causal, sig, vu, kind)
        entry = {"shape": wl.describe(), "flop": wl.flops, "bytes": wl.bytes}
        outs = {}
        variants = (1, 2, 3)
        if name == HEADLINE:   # the headline variant first, with the requested step counts
            variants = (args.variant,) + tuple(x for x in (1, 2, 3) if x != args.variant)
        for var in variants:
            call = f32_call(torch, fa, wl, var)
            kernels = fa.describe_launch(var, 1, bh, sq, sk, d, causal)
            if name == HEADLINE and var == args.variant:
                ms_step, ms_kernel = time_calls(torch, call, args.steps, args.warmup)
                result_head = (wl, kernels, ms_step, ms_kernel)
                log(f"[bench] {name} v{var}: {ms_step * 1e3:.1f} us/step wall, {ms_kernel * 1e3:.1f} us kernel")
                if not args.quick:
                    # Repeat protocol: R = 5 repeats of 20 launches, median us/call.
                    reps = sorted(time_calls(torch, call, 20, 3)[1] for _ in range(5))
                    entry[f"v{var}_median_5x20_us"] = round(reps[2] * 1e3, 1)
            else:
                steps = auto_steps(torch, call, max(5, args.steps))
                ms_step, ms_kernel = time_calls(torch, call, steps, 2)
            torch.cuda.synchronize()
            outs[var] = wl.o.cpu().numpy().copy()
            ent = {"us": round(ms_kernel * 1e3, 1)}
            tf = wl.flops / (ms_kernel * 1e-3) / 1e12
            if kind == "prefill":
                ent.update(tflops=round(tf, 2), pct_peak=round(100 * tf / PEAK_TFLOPS, 1))
            else:
                gbs = wl.bytes / (ms_kernel * 1e-3) / 1e9
                ent.update(gbs=round(gbs, 1), pct_hbm=round(100 * gbs / PEAK_GBS, 1))
            counters(ent, kernels, ms_kernel)
            entry[f"v{var}"] = ent
            history.append((name, f"v{var}", wl, ms_step, ms_kernel, ent))
            log(f"[bench] {name} v{var}: {ent} [{kernels}]")
        if not args.quick and name in ("config2", "config4a"):
            var = args.variant if name == HEADLINE else 2
            ms = time_host_slice(fa, wl, var, 5 if name == "config2" else 2)
            hs = {"ms": round(ms, 3)}
            if kind == "prefill":
                hs["tflops"] = round(wl.flops / (ms * 1e-3) / 1e12, 2)
            else:
                hs["gbs"] = round(wl.bytes / (ms * 1e-3) / 1e9, 1)
            entry[f"host_slice_v{var}"] = hs
            log(f"[bench] {name} host-slice v{var}: {ms:.2f} ms/call incl. PCIe copies")
        if not args.quick:
            for tname, dt, tdt in (("bf16", fa.DTYPE_BF16, torch.bfloat16), ("f16", fa.DTYPE_F16, torch.float16)):
                if name not in ("config2", "config3", "config4a", "config5"):
                    continue
                # 16-bit inputs (fa_device_lp): the same inputs rounded; FLOP
                # against the 16-bit MFMA peak, bytes at 2 B per input element.
                if name == "config3" and tname == "f16":
                    continue
                lq, lk, lv = wl.q.to(tdt), wl.k.to(tdt), wl.v.to(tdt)
                handle = torch.cuda.current_stream().cuda_stream

                def call_lp(lq=lq, lk=lk, lv=lv, dt=dt):
                    fa.attention_device_lp(dt, lq.data_ptr(), lk.data_ptr(), lv.data_ptr(), 1, wl.bh, wl.sq,
                                           wl.sk, wl.d, wl.causal, wl.o.data_ptr(), handle)

                steps = auto_steps(torch, call_lp, max(10, args.steps))
                ms_step, ms = time_calls(torch, call_lp, steps, 2)
                kernels = fa.describe_launch(3, 1, wl.bh, wl.sq, wl.sk, wl.d, wl.causal, dtype=dt)
                ent = {"us": round(ms * 1e3, 1)}
                if kind == "prefill":
                    tf = wl.flops / (ms * 1e-3) / 1e12
                    ent.update(tflops=round(tf, 1), pct_peak16=round(100 * tf / PEAK_TFLOPS_16, 1))
                else:
                    lp_bytes = wl.bh * wl.d * (2 * wl.sq + 4 * wl.sk + 4 * wl.sq)   # 16-bit Q, K, V; f32 O
                    gbs = lp_bytes / (ms * 1e-3) / 1e9
                    ent.update(gbs=round(gbs, 1), pct_hbm=round(100 * gbs / PEAK_GBS, 1))
                counters(ent, kernels, ms)
                entry[tname] = ent
                history.append((name, tname, wl, ms_step, ms, ent))
                log(f"[bench] {name} {tname}: {ent} [{kernels}]")
                del lq, lk, lv
        configs[name] = entry
        if not args.no_cpu_baseline:
            inputs = (wl.q.cpu().numpy(), wl.k.cpu().numpy(), wl.v.cpu().numpy())
            pending_cpu.append((name, wl, inputs, outs))
        if name != HEADLINE:
            wl.q = wl.k = wl.v = wl.o = None
        torch.cuda.empty_cache()

    wl, kernels, ms_step, ms_kernel = result_head
    kernel = kernels.split()[0]
    value = wl.flops / (ms_step * 1e-3) / 1e12
    achieved = wl.flops / (ms_kernel * 1e-3) / 1e12
    traffic, traffic_note = trf.lookup(traffic_table, kernel, grid_threads(kernels))
    result = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "config2: multihead prefill, 32 heads x 2048 x 2048, d_head 128, causal, "
                               "f32 N(0,1) Q/K/V (seeds 1/2/3), [heads, seq, d] contiguous",
                   "heads": 32, "seq_q": 2048, "seq_k": 2048, "d_head": 128, "causal": True,
                   "variant": f"v{args.variant}", "kernel": kernel},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_TFLOPS, 4), "traffic": traffic},
        "extra": {"configs": configs, "traffic_note": traffic_note,
                  "kernel_source_sha256": trf.kernel_source_hash()},
    }
    if peaks_error:
        result["extra"]["measured_peaks"] = {"error": peaks_error}
    if peaks:
        # the headline kernel against the FP32 MFMA rate this GPU itself sustains
        result["extra"]["measured_peaks"] = dict(
            peaks, headline_frac_of_measured=round(achieved / peaks["fp32_mfma_16x16x4"]["value"], 4))

    if pending_cpu:
        threads = host_cores()
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle

        tier = oracle.TIER_NAMES[oracle.best_tier()]
        for name, cwl, inputs, outs in pending_cpu:
            budget = args.cpu_seconds if name == HEADLINE else args.cpu_seconds_other
            log(f"[bench] cpu baseline {name} ({budget:.1f} s budget, {threads} threads) ...")
            want, sec, n = cpu_v2(inputs, cwl, budget, threads)
            ent = {"ms": round(sec * 1e3, 3), "calls": n, "threads": threads, "gflops": round(cwl.flops / sec / 1e9, 2)}
            if cwl.kind == "decode":
                ent["gbs"] = round(cwl.bytes / sec / 1e9, 2)
            configs[name]["cpu_v2"] = ent
            par = {f"v{var}": parity(o, want) for var, o in sorted(outs.items())}
            # [max-abs, rel-L2] per variant; "ok": every variant within the bar
            configs[name]["parity"] = dict({k: [p["max_abs"], p["rel_l2"]] for k, p in par.items()},
                                           ok=all(p["within_bar"] for p in par.values()))
            log(f"[bench] {name} cpu v2: {ent}; parity {par}")
            if name == HEADLINE:
                result["cpu_baseline"] = {
                    "value": round(cwl.flops / sec / 1e12, 4),
                    "unit": "TFLOP/s",
                    "cores": threads,
                    "kind": "port",
                    "sample": (f"{cwl.describe()}: full workload ({cwl.bh} heads), {n} calls after 1 warm-up, "
                               f"{sec * 1e3:.1f} ms/call, oracle v2 {tier} tier, Br=64 Bc=128, {threads} threads "
                               f"on {cpu_model()} ({threads} logical CPUs available)"),
                }
                p = par[f"v{args.variant}"]
                result["parity"] = dict(p, vs="oracle v2 on the host, same inputs as the timed calls",
                                        bar={"max_abs": MAX_ABS_TOL, "rel_l2": REL_L2_TOL})
            del want
        result["extra"]["cpu"] = {"threads": threads, "tier": tier, "model": cpu_model()}
    if args.csv:
        append_history(args.csv, history)
    for line in summary_lines(configs):
        log(line)
    if peaks:
        log("[summary] peaks: " + " | ".join(f"{k} {v['value']:g} {v['unit']} ({v['frac_of_datasheet'] * 100:.1f} %)"
                                            for k, v in peaks.items()))
    print(json.dumps(result, separators=(",", ":")), flush=True)
    return 0


def summary_lines(configs: dict) -> list[str]:
    """One short line per config: per variant us/call, TFLOP/s (GB/s for
    decode), % of peak (16-bit rows: of the 16-bit peak), MFMA busy % of a
    prefill kernel where profiled; then the worst max-abs / rel-L2 of the f32
    variants against CPU v2 and whether all are within the bar."""
    out = ["[summary] variant us TF|GB/s %peak [mMFMA-busy%] | ... ; worst f32 parity max-abs/rel-L2 vs CPU v2"]
    for name, e in configs.items():
        parts = []
        for var in ("v1", "v2", "v3", "bf16", "f16"):
            v = e.get(var)
            if not v:
                continue
            if "tflops" in v:
                rate = f"{v['tflops']:.1f}TF"
                mb = f" m{v['mfma_busy']:.0f}" if "mfma_busy" in v else ""
            else:
                rate, mb = f"{v['gbs']:.0f}GB/s", ""
            pct = v.get("pct_peak", v.get("pct_peak16", v.get("pct_hbm")))
            parts.append(f"{var} {v['us']:g}us {rate} {pct:g}%{mb}")
        par = e.get("parity")
        ptxt = ""
        if par:
            worst = [max(par[k][i] for k in ("v1", "v2", "v3") if k in par) for i in (0, 1)]
            ptxt = f" ; {worst[0]:.1e}/{worst[1]:.1e} " + ("ok" if par["ok"] else "FAIL")
        out.append(f"{name}: " + " | ".join(parts) + ptxt)
    return out


def append_history(path: str, history) -> None:
    """Benchmark-history rows (flash_attention_amd.bench_quick's extended
    schema): one per config and variant, keyed by the workload name."""
    from flash_attention_amd import bench_quick as bq

    import torch

    props = torch.cuda.get_device_properties(0)
    device = (getattr(props, "gcnArchName", "") or props.name).split(":")[0]
    cus = int(props.multi_processor_count)
    ts, commit = int(time.time()), bq.resolve_commit()
    import platform

    rows = []
    for name, label, wl, ms_wall, ms_kernel, ent in history:
        rows.append(bq.csv_row(ts, commit, platform.system().lower(), platform.machine(), cus, label, wl.causal,
                               wl.sq, wl.d, ms_wall, device, ms_kernel, workload=name, seq_len_k=wl.sk,
                               heads=wl.bh, tflops=ent.get("tflops"),
                               pct_peak=ent.get("pct_peak", ent.get("pct_peak16")), gbps=ent.get("gbs"),
                               pct_hbm=ent.get("pct_hbm"), mfma_busy=ent.get("mfma_busy"),
                               lds_bank_conflicts=ent.get("lds_conflicts"), fetch_gbps=ent.get("fetch_gbs")))
    new = not os.path.exists(path) or os.path.getsize(path) == 0
    with open(path, "a", encoding="utf-8") as f:
        if new:
            f.write(bq.HEADER_EXT + "\n")
        f.write("\n".join(rows) + "\n")
    log(f"[bench] appended {len(rows)} history rows to {path}")


if __name__ == "__main__":
    sys.exit(main())
