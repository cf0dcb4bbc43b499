"""Foreign callers of libfa_hip.so: a C program and a C++ program.

The reference is a Rust crate; its users would bind the C ABI through FFI.
Without rustc here, the nearest stand-ins are a plain C caller compiled with
gcc against include/fa_hip.h (tests/callers/fa_c_caller.c) and a C++ caller
of the header-only mirror of the crate's API
(flash-attention-cpu_amd/csrc/flash_attention.hpp,
tests/callers/fa_cpp_caller.cpp), each linked with -lfa_hip and run as its
own process.

Both call every public entry point -- the aliases fa_attention /
fa_attention_multihead (src/lib.rs:86-87), fa_v1..v3, fa_multihead_v1..v3
and naive_attention -- on the golden inputs (tests/golden/golden.npz) and a
multi-head case, with the default block sizes, with block_size_q =
block_size_kv = 0 (clamped by the crate, tests/correctness.rs:511-537) and
with block sizes that are not multiples of 4.

* CPU (here): both programs build and link; without a device every compute
  call returns FA_ERR_NO_DEVICE and leaves out untouched, zero-sized calls
  return FA_OK untouched, and the shape check reports "q shape mismatch".
* GPU: every output against the oracle's CPU v2 (north_star bar, max-abs
  2e-5, relative L2 1e-5) and the golden float64 result; naive_attention
  against the oracle's f32 naive; the aliases equal v2 bit for bit.
"""
from __future__ import annotations

import os
import struct
import subprocess

import numpy as np
import pytest

import flash_attention_amd as fa
import oracle
from fa_testutil import NAIVE_TOL, assert_parity, max_abs_diff

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "flash-attention-cpu_amd")
INCLUDE = os.path.join(ROOT, "include")
CALLERS = os.path.join(ROOT, "tests", "callers")

E_ALIAS, E_V1, E_V2, E_V3, E_MH_ALIAS, E_MH_V1, E_MH_V2, E_MH_V3, E_NAIVE = range(9)
BLOCKS = [(64, 128), (0, 0), (7, 13)]


def _has_gpu() -> bool:
    return os.path.exists("/dev/kfd")


def build_callers(tmp) -> dict[str, str]:
    c_exe = os.path.join(tmp, "fa_c_caller")
    cpp_exe = os.path.join(tmp, "fa_cpp_caller")
    link = ["-L", PKG, "-lfa_hip", "-Wl,-rpath," + PKG]
    subprocess.run(["gcc", "-std=c11", "-O1", "-Wall", "-Wextra", "-Werror", "-I", INCLUDE,
                    os.path.join(CALLERS, "fa_c_caller.c"), *link, "-o", c_exe], check=True)
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Wextra", "-Werror", "-I", INCLUDE,
                    "-I", os.path.join(PKG, "csrc"), os.path.join(CALLERS, "fa_cpp_caller.cpp"), *link,
                    "-o", cpp_exe], check=True)
    return {"c": c_exe, "cpp": cpp_exe}


def golden_cases():
    from golden.make_golden import load as load_golden
    return load_golden()


def make_cases():
    """[(entry, batch, heads, sq, sk, d, bq, bkv, causal, q, k, v)]"""
    cases = []
    for name, (bh, sq, sk, d, causal, q, k, v, _exp) in sorted(golden_cases().items()):
        if bh == 1:
            for e in (E_ALIAS, E_V1, E_V2, E_V3):
                for bq, bkv in BLOCKS:
                    cases.append((e, 1, 1, sq, sk, d, bq, bkv, causal, q, k, v))
            if sq * sk <= 256 * 256:
                cases.append((E_NAIVE, 1, 1, sq, sk, d, 64, 128, causal, q, k, v))
        batch, heads = (2, 3) if bh == 6 else (1, bh)
        for e in (E_MH_ALIAS, E_MH_V1, E_MH_V2, E_MH_V3):
            for bq, bkv in BLOCKS:
                cases.append((e, batch, heads, sq, sk, d, bq, bkv, causal, q, k, v))
    # zero-sized dimensions: FA_OK, out untouched (src/common.rs:56)
    z = np.zeros(0, np.float32)
    cases.append((E_ALIAS, 1, 1, 0, 5, 8, 64, 128, False, z, np.ones(40, np.float32), np.ones(40, np.float32)))
    cases.append((E_MH_ALIAS, 0, 3, 4, 4, 8, 64, 128, False, z, z, z))
    return cases


def write_cases(path, cases):
    with open(path, "wb") as f:
        f.write(struct.pack("<II", 0x31434146, len(cases)))
        for (e, b, h, sq, sk, d, bq, bkv, causal, q, k, v) in cases:
            f.write(struct.pack("<9q", e, b, h, sq, sk, d, bq, bkv, int(causal)))
            for a in (q, k, v):
                f.write(np.ascontiguousarray(a, np.float32).tobytes())


def read_outputs(path, cases):
    data = open(path, "rb").read()
    off, res = 0, []
    for (e, b, h, sq, sk, d, *_rest) in cases:
        (st,) = struct.unpack_from("<i", data, off)
        off += 4
        n = b * h * sq * d
        res.append((st, np.frombuffer(data, np.float32, n, off).copy()))
        off += 4 * n
    assert off == len(data)
    return res


def run_caller(exe, tmp, cases, tag):
    cin, cout = os.path.join(tmp, f"{tag}_cases.bin"), os.path.join(tmp, f"{tag}_out.bin")
    write_cases(cin, cases)
    print(f"[callers] running {tag}: {len(cases)} cases", flush=True)
    r = subprocess.run([exe, cin, cout], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, (tag, r.returncode, r.stdout, r.stderr)
    assert r.stdout.strip().endswith(f"{tag}-caller ok"), r.stdout
    return read_outputs(cout, cases)


@pytest.mark.skipif(_has_gpu(), reason="checks the no-device path")
def test_callers_build_and_fail_loudly_without_device(tmp_path):
    exes = build_callers(str(tmp_path))
    cases = make_cases()
    for tag, exe in exes.items():
        for (case, (st, out)) in zip(cases, run_caller(exe, str(tmp_path), cases, tag)):
            e, b, h, sq, sk, d = case[:6]
            if b * h * sq * sk * d == 0:
                assert st == fa.FA_OK
            else:
                assert st == fa.FA_ERR_NO_DEVICE, (tag, case[:9], st)
            assert np.all(out == 12.5), (tag, case[:9])


@pytest.mark.gpu
def test_c_and_cpp_callers_match_oracle(tmp_path):
    exes = build_callers(str(tmp_path))
    cases = make_cases()
    v2_bits = {}
    for tag, exe in exes.items():
        results = run_caller(exe, str(tmp_path), cases, tag)
        for (case, (st, out)) in zip(cases, results):
            e, b, h, sq, sk, d, bq, bkv, causal, q, k, v = case
            what = f"{tag} entry={e} b={b} h={h} sq={sq} sk={sk} d={d} blocks=({bq},{bkv}) causal={causal}"
            assert st == fa.FA_OK, (what, st, fa.status_string(st))
            if b * h * sq * sk * d == 0:
                assert np.all(out == 12.5), what
                continue
            bh = b * h
            if e == E_NAIVE:
                want = oracle.naive_f32(q, k, v, sq, sk, d, causal)
                assert max_abs_diff(out, want) < 1e-5, what
                continue
            want = oracle.run(2, q, k, v, bh, sq, sk, d, causal, 64, 128)
            assert_parity(out, want, what)
            exact = oracle.naive_f64(q, k, v, sq, sk, d, causal) if bh == 1 else None
            if exact is not None:
                assert max_abs_diff(out, exact) < NAIVE_TOL, what
            key = (tag, b, h, sq, sk, d, bq, bkv, causal, e in (E_MH_ALIAS, E_MH_V1, E_MH_V2, E_MH_V3))
            if e in (E_V2, E_MH_V2):
                v2_bits[key] = out
        # the aliases are v2 (src/lib.rs:86-87): the same bits
        for (case, (st, out)) in zip(cases, results):
            e, b, h, sq, sk, d, bq, bkv, causal = case[:9]
            if e in (E_ALIAS, E_MH_ALIAS) and b * h * sq * sk * d:
                key = (tag, b, h, sq, sk, d, bq, bkv, causal, e == E_MH_ALIAS)
                assert np.array_equal(out, v2_bits[key]), (tag, case[:9])
