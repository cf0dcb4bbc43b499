"""ctypes view of the CPU oracle (``oracle/liboracle.so``).

TEST INFRASTRUCTURE ONLY.  Imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg, always as the checker or the timed CPU
baseline, never as the thing measured or shipped.  The product library
(``libfa_hip.so``) has no path into this module.

The C library restates the reference crate's CPU path (amaye15/flash-attention-cpu):
``run_v1`` src/v1.rs:162-396, ``run_v2`` src/v2.rs:160-385 (the parity oracle),
``run_v3`` src/v3.rs:177-512, ``naive_attention`` src/naive.rs:14-75 and the
Kernel-trait tiers src/scalar.rs, src/avx2.rs, src/avx512.rs.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

TIER_AUTO, TIER_SCALAR, TIER_AVX2, TIER_AVX512 = -1, 0, 1, 2
TIER_NAMES = {TIER_SCALAR: "scalar", TIER_AVX2: "avx2+fma", TIER_AVX512: "avx512f"}
MUTANT_NONE, MUTANT_NO_CORRECTION, MUTANT_MASK_DIAGONAL, MUTANT_SCALE_1_OVER_D, MUTANT_V_SHIFT = range(5)

_lib = None

_F = ctypes.POINTER(ctypes.c_float)
_D = ctypes.POINTER(ctypes.c_double)
_SZ = ctypes.c_size_t


def build() -> str:
    """Compile liboracle.so with the committed Makefile (gcc only)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_best_tier.restype = ctypes.c_int
        L.oracle_tier_available.argtypes = [ctypes.c_int]
        L.oracle_run.restype = ctypes.c_int
        L.oracle_run.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, _F, _F, _F,
                                 _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, ctypes.c_int, _F]
        L.oracle_naive_f32.argtypes = [_F, _F, _F, _SZ, _SZ, _SZ, ctypes.c_int, _F]
        L.oracle_naive_f64.argtypes = [_F, _F, _F, _SZ, _SZ, _SZ, ctypes.c_int, _D]
        L.oracle_naive_f64_rows.argtypes = [_F, _F, _F, _SZ, _SZ, _SZ, ctypes.c_int, _SZ, _SZ, _D]
        L.oracle_exp_simd.argtypes = [ctypes.c_int, _F, _F, _SZ]
        L.oracle_k_dot.restype = ctypes.c_float
        L.oracle_k_dot.argtypes = [ctypes.c_int, _F, _F, _SZ]
        L.oracle_k_dot4x4.argtypes = [ctypes.c_int, _F, _F, _SZ, _F]
        L.oracle_k_pv4.argtypes = [ctypes.c_int, _F, _F, _F, _SZ, _SZ]
        L.oracle_k_max_reduce.restype = ctypes.c_float
        L.oracle_k_max_reduce.argtypes = [ctypes.c_int, _F, _SZ]
        L.oracle_k_sub_exp_sum.restype = ctypes.c_float
        L.oracle_k_sub_exp_sum.argtypes = [ctypes.c_int, _F, _SZ, ctypes.c_float]
        L.oracle_set_mutant.argtypes = [ctypes.c_int]
        _lib = L
    return _lib


def _fp(a: np.ndarray):
    return a.ctypes.data_as(_F)


def _c32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def best_tier() -> int:
    return lib().oracle_best_tier()


def tier_available(tier: int) -> bool:
    return bool(lib().oracle_tier_available(tier))


def run(variant: int, q, k, v, bh: int, seq_q: int, seq_k: int, d: int, causal: bool,
        block_q: int = 64, block_kv: int = 128, tier: int = TIER_AUTO, nthreads: int = 0,
        out: np.ndarray | None = None) -> np.ndarray:
    """Tiled attention over ``bh`` heads laid out [bh, seq, d] (run_v{1,2,3})."""
    q, k, v = _c32(q), _c32(k), _c32(v)
    if out is None:
        out = np.zeros(bh * seq_q * d, dtype=np.float32)
    rc = lib().oracle_run(int(variant), int(tier), int(nthreads), _fp(q), _fp(k), _fp(v), bh, seq_q,
                          seq_k, d, block_q, block_kv, int(bool(causal)), _fp(out))
    if rc != 0:
        raise ValueError(f"oracle_run rejected variant={variant} tier={tier}")
    return out


def naive_f32(q, k, v, seq_q, seq_k, d, causal) -> np.ndarray:
    q, k, v = _c32(q), _c32(k), _c32(v)
    out = np.zeros(seq_q * d, dtype=np.float32)
    lib().oracle_naive_f32(_fp(q), _fp(k), _fp(v), seq_q, seq_k, d, int(bool(causal)), _fp(out))
    return out


def naive_f64(q, k, v, seq_q, seq_k, d, causal, row0: int = 0, nrows: int | None = None) -> np.ndarray:
    q, k, v = _c32(q), _c32(k), _c32(v)
    if nrows is None:
        nrows = seq_q - row0
    out = np.zeros(nrows * d, dtype=np.float64)
    lib().oracle_naive_f64_rows(_fp(q), _fp(k), _fp(v), seq_q, seq_k, d, int(bool(causal)), row0,
                                nrows, out.ctypes.data_as(_D))
    return out


def exp_simd(tier: int, x) -> np.ndarray:
    x = _c32(x)
    y = np.zeros_like(x)
    lib().oracle_exp_simd(tier, _fp(x), _fp(y), x.size)
    return y


def set_mutant(which: int) -> None:
    lib().oracle_set_mutant(int(which))
