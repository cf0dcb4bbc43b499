"""Helpers shared by the test modules (inputs, error metrics, tolerances)."""
from __future__ import annotations

import numpy as np

# north_star parity bar for the GPU path vs the CPU v2 oracle.
MAX_ABS_TOL = 2e-5
REL_L2_TOL = 1e-5
# The reference's own bar vs naive attention (tests/correctness.rs:109).
NAIVE_TOL = 1e-3


def random_vec(n: int, seed_shift: int) -> np.ndarray:
    """U(-1, 1) inputs seeded like tests/correctness.rs:63-66 (0xC0FFEE ^ shift).

    The crate draws from rand's StdRng; this draws from numpy's PCG64 with the
    same seed expression, so values differ but the distribution matches.
    """
    rng = np.random.default_rng(0xC0FFEE ^ seed_shift)
    return rng.uniform(-1.0, 1.0, n).astype(np.float32)


def normal_vec(n: int, seed: int, sigma: float = 1.0) -> np.ndarray:
    """N(0, sigma^2) float32 inputs (benchmark configs: seeds Q=1, K=2, V=3)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n, dtype=np.float32)
    if sigma != 1.0:
        x *= np.float32(sigma)
    return x


def uniform_vec(n: int, seed: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return rng.uniform(lo, hi, n).astype(np.float32)


def max_abs_diff(a, b) -> float:
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    if a.size == 0:
        return 0.0
    return float(np.max(np.abs(a - b)))


def rel_l2(a, b) -> float:
    """||a - b|| / ||b||."""
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    den = float(np.linalg.norm(b))
    return float(np.linalg.norm(a - b)) / (den if den > 0 else 1.0)


def assert_parity(got, want, what: str = "", max_abs: float = MAX_ABS_TOL, rel: float = REL_L2_TOL):
    ma = max_abs_diff(got, want)
    rl = rel_l2(got, want)
    print(f"[parity] {what}: max-abs {ma:.3g} rel-L2 {rl:.3g}", flush=True)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    assert ma < max_abs and rl < rel, f"{what}: max-abs {ma:.3g} (tol {max_abs}), rel-L2 {rl:.3g} (tol {rel})"
    return ma, rl


def attention_f64(q, k, v, seq_q, seq_k, d, causal):
    """Textbook softmax attention in float64 numpy (independent of the oracle)."""
    q = np.asarray(q, dtype=np.float64).reshape(seq_q, d)
    k = np.asarray(k, dtype=np.float64).reshape(seq_k, d)
    v = np.asarray(v, dtype=np.float64).reshape(seq_k, d)
    s = (q @ k.T) / np.sqrt(float(np.float32(d)))
    if causal:
        i = np.arange(seq_q)[:, None]
        j = np.arange(seq_k)[None, :]
        s = np.where(j > i, -np.inf, s)
    m = np.max(s, axis=1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    p = np.exp(s - m)
    den = p.sum(axis=1, keepdims=True)
    p = np.divide(p, den, out=np.zeros_like(p), where=den > 0)
    return (p @ v).ravel()


def long_row_f16_case():
    """A row of n keys whose probabilities (all but one) equal t ~ 179.5 x 2^-24,
    inside f16's subnormal range: key 0 scores 48 (q = 4 e0, k0 = 12 e0, scale
    1/8) and sets the reference, the others score 4 b with b = -10.890625, and
    n = 1/t so that their total weight equals key 0's.  V row 0 is -1, the
    others +1, so O = (-1 + n t) / (1 + n t) ~ 0 and any common rounding of t
    moves O by about half its relative error.  Rounded as a subnormal, t is
    off by 2.7e-3 (O by 1.4e-3, three times the u/(1-u) bound); rounded as
    2^7 t, a normal f16, by at most u = 2^-11."""
    d, sq, n = 64, 16, 93462
    q = np.zeros((sq, d), np.float16)
    q[:, 0] = 4.0
    k = np.zeros((n + 1, d), np.float16)
    k[0, 0], k[1:, 0] = 12.0, -10.890625
    v = np.ones((n + 1, d), np.float16)
    v[0] = -1.0
    return q.ravel(), k.ravel(), v.ravel(), sq, n + 1, d
