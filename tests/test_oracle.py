"""Pin the CPU oracle (oracle/fa_oracle.c) before trusting it as the checker.

The oracle restates the reference crate's CPU path (amaye15/flash-attention-cpu):
run_v1 src/v1.rs:162-396, run_v2 src/v2.rs:160-385, run_v3 src/v3.rs:177-512,
naive_attention src/naive.rs:14-75, and the scalar / AVX2 / AVX-512 Kernel
tiers.  The crate ships no golden vectors, so the checks here are:

* independent float64 attention (numpy, not the oracle's code) on the shape
  matrix of tests/correctness.rs, and the committed golden vectors
  (tests/golden/golden.npz, also float64 numpy);
* known answers: causal row 0 == V[0] (tests/correctness.rs:240-263),
  seq_k == 1 => every row == V[0], Q == 0 => uniform weights over visible
  keys (prefix means when causal);
* invariances: permuting K/V rows together (non-causal), adding one vector to
  every K row (shifts each score row by a constant), block sizes (incl. the
  0 clamp, tests/correctness.rs:510-537);
* variant relations: v2 and v3 bit-identical (same per-row arithmetic,
  src/v3.rs docs), v1 within 1e-5 of v2 (tests/correctness.rs:299-375);
* primitives: the SIMD exp within 1e-5 relative of libm on [-80, 80) step
  0.1 (src/avx512.rs:596-623), each SIMD primitive against the scalar one;
* planted mistakes (oracle_set_mutant): each one fails at least one pin.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
from fa_testutil import attention_f64, max_abs_diff, random_vec
from golden.make_golden import load as load_golden

TIERS = [t for t in (oracle.TIER_SCALAR, oracle.TIER_AVX2, oracle.TIER_AVX512) if oracle.tier_available(t)]
VARIANTS = (1, 2, 3)

# tests/correctness.rs shape matrix: (seq_q, seq_k, d, br, bc, causal)
SHAPES = [
    (64, 64, 64, 32, 32, False), (128, 128, 64, 64, 64, False),
    (17, 23, 32, 8, 8, False), (1, 1, 16, 8, 8, False), (1, 50, 33, 16, 16, False),
    (50, 1, 33, 16, 16, False), (97, 131, 17, 32, 40, False), (200, 200, 128, 64, 128, False),
    (64, 64, 64, 32, 32, True), (97, 97, 33, 16, 24, True), (1, 1, 16, 8, 8, True), (5, 5, 8, 64, 64, True),
    (10, 40, 32, 4, 8, True), (10, 10, 8, 1024, 1024, False), (10, 10, 8, 1024, 1024, True),
    (23, 29, 24, 3, 12, True), (23, 29, 24, 7, 12, False), (29, 23, 24, 12, 5, True), (29, 23, 24, 12, 6, False),
]


def qkv(sq, sk, d, shift=0):
    return random_vec(sq * d, 1 + shift), random_vec(sk * d, 2 + shift), random_vec(sk * d, 3 + shift)


@pytest.fixture(autouse=True)
def _no_mutant():
    oracle.set_mutant(oracle.MUTANT_NONE)
    yield
    oracle.set_mutant(oracle.MUTANT_NONE)


@pytest.mark.parametrize("shape", SHAPES)
def test_every_variant_and_tier_matches_float64(shape):
    sq, sk, d, br, bc, causal = shape
    q, k, v = qkv(sq, sk, d)
    want = attention_f64(q, k, v, sq, sk, d, causal)
    naive64 = oracle.naive_f64(q, k, v, sq, sk, d, causal)
    assert max_abs_diff(naive64, want) < 1e-12          # two float64 routes agree
    assert max_abs_diff(oracle.naive_f32(q, k, v, sq, sk, d, causal), want) < 1e-5
    for variant in VARIANTS:
        for tier in TIERS:
            got = oracle.run(variant, q, k, v, 1, sq, sk, d, causal, br, bc, tier=tier)
            # the reference's bar is 1e-3 (tests/correctness.rs:109); f32 lands ~1e-7
            assert max_abs_diff(got, want) < 1e-5, (variant, tier, shape)


def test_golden_vectors():
    for name, (bh, sq, sk, d, causal, q, k, v, exp) in load_golden().items():
        for variant in VARIANTS:
            got = oracle.run(variant, q, k, v, bh, sq, sk, d, causal)
            tol = 2e-5 if name.startswith("peaky") else 2e-6
            assert max_abs_diff(got, exp) < tol, (name, variant, max_abs_diff(got, exp))


@pytest.mark.parametrize("variant", VARIANTS)
def test_causal_first_query_equals_first_value_row(variant):
    seq, d = 256, 64
    q, k, v = random_vec(seq * d, 30), random_vec(seq * d, 31), random_vec(seq * d, 32)
    for br, bc in [(64, 128), (32, 32), (1024, 1024), (1, 1)]:
        got = oracle.run(variant, q, k, v, 1, seq, seq, d, True, br, bc)
        assert max_abs_diff(got[:d], v[:d]) < 1e-5


@pytest.mark.parametrize("variant", VARIANTS)
def test_single_key_gives_first_value_row(variant):
    sq, d = 33, 40
    q, k, v = random_vec(sq * d, 5), random_vec(d, 6), random_vec(d, 7)
    got = oracle.run(variant, q, k, v, 1, sq, 1, d, False, 8, 8).reshape(sq, d)
    assert max_abs_diff(got, np.broadcast_to(v, (sq, d))) < 1e-6


@pytest.mark.parametrize("causal", (False, True))
def test_zero_queries_average_visible_values(causal):
    sq, sk, d = 70, 70, 16
    q = np.zeros(sq * d, np.float32)
    k, v = random_vec(sk * d, 2), random_vec(sk * d, 3)
    vv = v.reshape(sk, d).astype(np.float64)
    if causal:
        want = np.cumsum(vv, axis=0) / np.arange(1, sk + 1)[:, None]
    else:
        want = np.broadcast_to(vv.mean(axis=0), (sq, d))
    for variant in VARIANTS:
        got = oracle.run(variant, q, k, v, 1, sq, sk, d, causal, 16, 24).reshape(sq, d)
        assert max_abs_diff(got, want) < 1e-6


def test_permuting_keys_and_values_together_is_invariant():
    sq, sk, d = 40, 77, 24
    q, k, v = qkv(sq, sk, d)
    perm = np.random.default_rng(7).permutation(sk)
    kp = k.reshape(sk, d)[perm].ravel()
    vp = v.reshape(sk, d)[perm].ravel()
    for variant in VARIANTS:
        a = oracle.run(variant, q, k, v, 1, sq, sk, d, False, 16, 16)
        b = oracle.run(variant, q, kp, vp, 1, sq, sk, d, False, 16, 16)
        assert max_abs_diff(a, b) < 1e-6


def test_shifting_every_key_by_one_vector_is_invariant():
    # q.(k_j + u) = q.k_j + q.u: every score of a row moves by one constant.
    sq, sk, d = 30, 50, 16
    q, k, v = qkv(sq, sk, d)
    u = random_vec(d, 99)
    k2 = (k.reshape(sk, d) + u).ravel().astype(np.float32)
    want = attention_f64(q, k2, v, sq, sk, d, True)
    for variant in VARIANTS:
        a = oracle.run(variant, q, k, v, 1, sq, sk, d, True, 8, 8)
        b = oracle.run(variant, q, k2, v, 1, sq, sk, d, True, 8, 8)
        assert max_abs_diff(a, b) < 1e-5
        assert max_abs_diff(b, want) < 1e-5


@pytest.mark.parametrize("causal", (False, True))
def test_block_sizes_do_not_change_results(causal):
    sq, sk, d = 23, 29, 16
    q, k, v = qkv(sq, sk, d)
    ref = oracle.run(2, q, k, v, 1, sq, sk, d, causal, 64, 128)
    for br, bc in [(0, 0), (1, 1), (3, 5), (7, 12), (1024, 1024)]:
        for variant in VARIANTS:
            got = oracle.run(variant, q, k, v, 1, sq, sk, d, causal, br, bc)
            assert max_abs_diff(got, ref) < 1e-5, (br, bc, variant)


def test_v2_v3_bit_identical_and_v1_close():
    for sq, sk, d, br, bc, causal in [(64, 64, 64, 32, 32, False), (97, 131, 17, 32, 40, True),
                                      (5, 5, 8, 64, 64, True), (200, 200, 128, 64, 128, True)]:
        q, k, v = qkv(sq, sk, d)
        for tier in TIERS:
            o1 = oracle.run(1, q, k, v, 1, sq, sk, d, causal, br, bc, tier=tier)
            o2 = oracle.run(2, q, k, v, 1, sq, sk, d, causal, br, bc, tier=tier)
            o3 = oracle.run(3, q, k, v, 1, sq, sk, d, causal, br, bc, tier=tier)
            assert np.array_equal(o2, o3)
            assert max_abs_diff(o1, o2) < 1e-5


def test_multihead_equals_per_head():
    bh, sq, sk, d = 6, 37, 50, 16
    q, k, v = random_vec(bh * sq * d, 21), random_vec(bh * sk * d, 22), random_vec(bh * sk * d, 23)
    for variant in VARIANTS:
        got = oracle.run(variant, q, k, v, bh, sq, sk, d, True, 8, 12, nthreads=3)
        for h in range(bh):
            one = oracle.run(variant, q[h * sq * d:(h + 1) * sq * d], k[h * sk * d:(h + 1) * sk * d],
                             v[h * sk * d:(h + 1) * sk * d], 1, sq, sk, d, True, 8, 12, nthreads=1)
            assert np.array_equal(got[h * sq * d:(h + 1) * sq * d], one)


def test_zero_sized_dimensions_leave_out_untouched():
    d = 8
    out = np.full(4 * d, 12.5, np.float32)
    oracle.run(2, random_vec(4 * d, 1), np.zeros(0, np.float32), np.zeros(0, np.float32), 1, 4, 0, d, False,
               out=out)
    assert np.all(out == 12.5)
    out = np.full(4, 12.5, np.float32)
    oracle.run(2, np.zeros(0, np.float32), np.zeros(0, np.float32), np.zeros(0, np.float32), 1, 4, 4, 0, False,
               out=out)
    assert np.all(out == 12.5)


def test_thread_count_does_not_change_bits():
    bh, sq, sk, d = 4, 150, 170, 64
    q, k, v = random_vec(bh * sq * d, 1), random_vec(bh * sk * d, 2), random_vec(bh * sk * d, 3)
    a = oracle.run(2, q, k, v, bh, sq, sk, d, True, nthreads=1)
    b = oracle.run(2, q, k, v, bh, sq, sk, d, True, nthreads=8)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("tier", [t for t in TIERS if t != oracle.TIER_SCALAR])
def test_simd_exp_matches_libm(tier):
    x = (np.arange(-800, 800) * 0.1).astype(np.float32)
    y = oracle.exp_simd(tier, x)
    want = np.exp(x.astype(np.float64))
    assert np.max(np.abs(y - want) / want) < 1e-5


@pytest.mark.parametrize("tier", [t for t in TIERS if t != oracle.TIER_SCALAR])
def test_simd_primitives_match_scalar(tier):
    L = oracle.lib()
    fp = lambda a: a.ctypes.data_as(oracle._F)   # noqa: E731
    rng = np.random.default_rng(3)
    for n in (0, 1, 3, 7, 8, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127):
        a = rng.uniform(-1, 1, n).astype(np.float32)
        b = rng.uniform(-1, 1, n).astype(np.float32)
        s0 = L.oracle_k_dot(oracle.TIER_SCALAR, fp(a), fp(b), n)
        s1 = L.oracle_k_dot(tier, fp(a), fp(b), n)
        assert abs(s0 - s1) < 1e-4 * (np.sum(np.abs(a * b)) + 1)
        if n:
            assert L.oracle_k_max_reduce(tier, fp(a), n) == np.max(a)
            x0, x1 = a.copy(), a.copy()
            r0 = L.oracle_k_sub_exp_sum(oracle.TIER_SCALAR, fp(x0), n, 0.5)
            r1 = L.oracle_k_sub_exp_sum(tier, fp(x1), n, 0.5)
            assert abs(r0 - r1) < 1e-5 * abs(r0)
            assert np.max(np.abs(x0 - x1)) < 1e-6
    for d in (8, 16, 17, 51, 64, 128):
        qs = rng.uniform(-1, 1, 4 * d).astype(np.float32)
        ks = rng.uniform(-1, 1, 4 * d).astype(np.float32)
        o0, o1 = np.zeros(16, np.float32), np.zeros(16, np.float32)
        L.oracle_k_dot4x4(oracle.TIER_SCALAR, fp(qs), fp(ks), d, fp(o0))
        L.oracle_k_dot4x4(tier, fp(qs), fp(ks), d, fp(o1))
        want = qs.reshape(4, d).astype(np.float64) @ ks.reshape(4, d).T.astype(np.float64)
        assert max_abs_diff(o1, want) < 1e-4 and max_abs_diff(o0, want) < 1e-4
    for bc, d in ((9, 51), (16, 64), (5, 8), (1, 128)):
        acc0 = rng.uniform(-1, 1, 4 * d).astype(np.float32)
        acc1 = acc0.copy()
        vb = rng.uniform(-1, 1, bc * d).astype(np.float32)
        p = rng.uniform(0, 1, 4 * bc).astype(np.float32)
        want = acc0.reshape(4, d) + p.reshape(4, bc).astype(np.float64) @ vb.reshape(bc, d)
        L.oracle_k_pv4(oracle.TIER_SCALAR, fp(acc0), fp(vb), fp(p), bc, d)
        L.oracle_k_pv4(tier, fp(acc1), fp(vb), fp(p), bc, d)
        assert max_abs_diff(acc0, want) < 1e-5 and max_abs_diff(acc1, want) < 1e-5


def _pins_fail(variant: int) -> bool:
    """True if at least one of the pins above catches the active mutant."""
    seq, d = 64, 16
    q, k, v = random_vec(seq * d, 30), random_vec(seq * d, 31), random_vec(seq * d, 32)
    got = oracle.run(variant, q, k, v, 1, seq, seq, d, True, 16, 16)
    if not np.all(np.isfinite(got)) or max_abs_diff(got[:d], v[:d]) > 1e-5:
        return True
    for sq, sk, dd, br, bc, causal in [(97, 131, 17, 32, 40, True), (64, 64, 64, 32, 32, False)]:
        q, k, v = qkv(sq, sk, dd)
        got = oracle.run(variant, q, k, v, 1, sq, sk, dd, causal, br, bc)
        if not np.all(np.isfinite(got)) or max_abs_diff(got, attention_f64(q, k, v, sq, sk, dd, causal)) > 1e-5:
            return True
    return False


@pytest.mark.parametrize("mutant", [oracle.MUTANT_NO_CORRECTION, oracle.MUTANT_MASK_DIAGONAL,
                                    oracle.MUTANT_SCALE_1_OVER_D, oracle.MUTANT_V_SHIFT])
@pytest.mark.parametrize("variant", VARIANTS)
def test_planted_mistakes_are_caught(mutant, variant):
    assert not _pins_fail(variant)
    oracle.set_mutant(mutant)
    try:
        assert _pins_fail(variant), f"mutant {mutant} slipped through for v{variant}"
    finally:
        oracle.set_mutant(oracle.MUTANT_NONE)
    assert not _pins_fail(variant)


def test_float64_reference_itself_on_closed_forms():
    # attention_f64 is the yardstick: check it where the answer is known.
    d = 4
    q = np.zeros(3 * d, np.float32)
    k = random_vec(3 * d, 1)
    v = np.arange(3 * d, dtype=np.float32)
    got = attention_f64(q, k, v, 3, 3, d, True).reshape(3, d)
    vv = v.reshape(3, d)
    assert np.allclose(got, np.cumsum(vv, 0) / np.arange(1, 4)[:, None])
    # two keys with score gap g: weights 1/(1+e^-g)
    q1 = np.array([2.0, 0, 0, 0], np.float32)
    k1 = np.array([[1.0, 0, 0, 0], [0, 0, 0, 0]], np.float32).ravel()
    v1 = np.array([[1.0, 0, 0, 0], [0, 1.0, 0, 0]], np.float32).ravel()
    w = 1.0 / (1.0 + math.exp(-2.0 / math.sqrt(4.0)))
    assert np.allclose(attention_f64(q1, k1, v1, 1, 2, 4, False), [w, 1 - w, 0, 0])
