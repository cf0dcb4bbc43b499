"""AddressSanitizer + UndefinedBehaviorSanitizer builds of the CPU code.

GPU code cannot be sanitised on this pool, so the checks cover what runs on
the host:

* the host library's CPU-side paths -- flash-attention-cpu_amd/csrc/fa_host.cpp
  compiled with -fsanitize=address,undefined into
  tests/callers/asan_host_driver.cpp, which sweeps the launch planner
  (fa_describe_launch over shapes, paths, split counts, dtypes), the shape
  checks of every host-slice entry point, zero-sized dimensions, argument
  errors and the no-device path;
* the oracle -- oracle/*.c compiled the same way into
  tests/callers/asan_oracle_driver.c, which runs v1/v2/v3 on every tier over
  ragged shapes and block sizes (0 included) and checks them against the f64
  naive result, plus the naive forms and the SIMD primitives at odd lengths.

Any sanitizer report aborts the program (-fno-sanitize-recover=all), which
fails the test.
"""
from __future__ import annotations

import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "flash-attention-cpu_amd", "csrc")
CALLERS = os.path.join(ROOT, "tests", "callers")
ORACLE = os.path.join(ROOT, "oracle")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")


def _run(exe, tag, timeout=600):
    r = subprocess.run([exe], capture_output=True, text=True, env=ENV, timeout=timeout)
    assert r.returncode == 0 and r.stdout.strip().endswith(f"{tag} ok"), (r.returncode, r.stdout[-2000:],
                                                                          r.stderr[-4000:])
    return r.stdout


def test_host_library_cpu_paths_under_asan_ubsan(tmp_path):
    exe = str(tmp_path / "asan_host")
    subprocess.run([os.path.join(ROCM, "llvm", "bin", "clang++"), "-std=c++17", *SAN, "-D__HIP_PLATFORM_AMD__",
                    "-I", os.path.join(ROCM, "include"), "-I", os.path.join(ROOT, "include"), "-I", CSRC,
                    os.path.join(CALLERS, "asan_host_driver.cpp"), os.path.join(CSRC, "fa_host.cpp"),
                    "-L", os.path.join(ROCM, "lib"), "-lamdhip64", "-Wl,-rpath," + os.path.join(ROCM, "lib"),
                    "-lpthread", "-ldl", "-o", exe], check=True)
    out = _run(exe, "asan-host")
    assert "failures=0" in out


def test_oracle_under_asan_ubsan(tmp_path):
    exe = str(tmp_path / "asan_oracle")
    srcs = [os.path.join(ORACLE, f) for f in ("fa_oracle.c", "fa_avx2.c", "fa_avx512.c")]
    subprocess.run(["gcc", "-std=c11", "-D_GNU_SOURCE", "-ffp-contract=off", *SAN, "-I", ORACLE,
                    os.path.join(CALLERS, "asan_oracle_driver.c"), *srcs, "-lm", "-lpthread", "-o", exe],
                   check=True)
    out = _run(exe, "asan-oracle")
    assert "failures=0" in out
